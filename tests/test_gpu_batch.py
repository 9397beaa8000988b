"""Batched decoding (independent sequences, paged fp16 K/V, one GEMM per
linear layer over the batch rows) against the oracle run one sequence at a
time: every sequence's greedy ids identical and its logits within 1e-3 of
max|ref| at every step, for any subset and order of sequences per step."""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, ChonkError, load_llama_wgsl_model
from chonklm_amd.runtime import LlamaWgslBatch
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _setup(synth, name, n_seq, max_tokens):
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path)
    loaded = load_llama_wgsl_model(md)
    refs = [OracleModel(path, w.spec.vocab, w.spec.layers, md.max_context, kv_f16=True, eos_ids=w.eos_ids)
            for _ in range(n_seq)]
    return w, loaded, LlamaWgslBatch(loaded.engine, n_seq, max_tokens), refs


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama", "tiny-gemma3"])
def test_batch_matches_per_sequence_oracle(name, synth):
    w, loaded, batch, refs = _setup(synth, name, 3, 90)
    rng = np.random.default_rng(41)
    prompts = [rng.integers(0, w.spec.vocab, n).tolist() for n in (11, 30, 5)]
    cur = []
    for s, p in enumerate(prompts):
        got = batch.prefill(s, p)
        for t in p[:-1]:
            refs[s].run_token(t, False)
        want = refs[s].run_token(p[-1], True)
        assert rel_err(batch.read_logits(0), refs[s].logits()) <= 1e-3
        assert got == want, f"seq {s} prefill: {got} != {want}"
        cur.append(got)
    orders = [[0, 1, 2], [2, 0], [1], [0, 1, 2], [2, 1, 0], [0, 2]]
    for step, seqs in enumerate(orders):
        got = batch.step(seqs, [cur[s] for s in seqs])
        for row, s in enumerate(seqs):
            want = refs[s].run_token(cur[s], True)
            assert rel_err(batch.read_logits(row), refs[s].logits()) <= 1e-3, f"step {step} seq {s}"
            assert got[row] == want, f"step {step} seq {s}: {got[row]} != {want}"
            cur[s] = got[row]
    for s in range(3):
        assert batch.position(s) == refs[s].position
    batch.close()


def test_batch_errors_and_restart(synth):
    w, loaded, batch, refs = _setup(synth, "tiny-qwen3", 2, 20)
    with pytest.raises(ChonkError):
        batch.step([0, 0], [1, 2])
    with pytest.raises(ChonkError):
        batch.prefill(2, [1, 2])
    with pytest.raises(ChonkError) as ei:
        batch.prefill(0, list(range(21)))
    assert ei.value.status_name == "ECONTEXT"
    t = batch.prefill(0, list(range(1, 20)))
    t = batch.step([0], [t])[0]
    with pytest.raises(ChonkError) as ei:
        batch.step([0], [t])
    assert ei.value.status_name == "ECONTEXT"
    # a sequence started over forgets its earlier tokens
    a = batch.prefill(0, [5, 6, 7])
    for tok in [5, 6]:
        refs[0].run_token(tok, False)
    assert a == refs[0].run_token(7, True)
    batch.close()
