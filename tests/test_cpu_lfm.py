"""The oracle's LFM2 decoder (src/lib/lfm-wgsl-runtime.ts) against closed forms.

tests/numpy_ref.py's NumpyLfm2 restates the hybrid decoder in float64 numpy,
the short convolution from the list of every position's B*x rather than from a
shifted three-slot state, attention over the whole cache. Bars: logits within
1e-4 relative at every step, identical greedy ids to the golden fixture
(tests/golden/greedy_golden.json, written by make_greedy_golden.py from the
float64 decoder), and the selection rules of TOPK256_WGSL / ARGMAX_WGSL
(:1880-1947) pinned by per-class first-maximum closed forms and hand-derived
tie cases.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from chonklm_amd import WORKLOADS
from oracle import oracle as orc
from oracle.oracle import OracleModel
from tests.conftest import rel_err
from tests.numpy_ref import NumpyLfm2

TINY_LFM = ["tiny-lfm2", "tiny-lfm2-q8"]
GOLDEN = json.loads((Path(__file__).parent / "golden" / "greedy_golden.json").read_text())
NEG_BIG = np.float32(-3.402823e38)


def _oracle(synth, name, kv_f16=True, **kw):
    w = WORKLOADS[name]
    path = synth(name)
    return w, path, OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=kv_f16,
                                eos_ids=w.eos_ids, threads=4, **kw)


def _pairs(p: np.ndarray):
    v = p.view(np.float32)[0::2]
    i = p.view(np.uint32)[1::2]
    return v, i


@pytest.mark.parametrize("name", TINY_LFM)
def test_lfm_logits_match_float64_decoder(name, synth):
    w, path, ref = _oracle(synth, name)
    assert ref.lfm and not ref.gpt
    dec = NumpyLfm2(path, w.spec.vocab, w.max_context, kv_f16=True)
    prompt = np.random.default_rng(5).integers(0, w.spec.vocab, 14).tolist()
    tok = prompt[0]
    for i in range(len(prompt) + 8):
        if i < len(prompt):
            tok = prompt[i]
        a = ref.run_token(tok, True)
        want = dec.step(tok)
        assert rel_err(ref.logits(), want) <= 1e-4, f"{name} step {i}"
        assert a == int(np.argmax(ref.logits()))
        if i >= len(prompt) - 1:
            tok = a


def test_lfm_convolution_state_matters(synth):
    """The convolution reaches two positions back: the same token after different
    histories gives different logits, and reset restores the first-position result."""
    w, path, ref = _oracle(synth, "tiny-lfm2")
    ref.run_token(5, True)
    first = ref.logits().copy()
    ref.run_token(7, True)
    ref.run_token(5, True)
    assert rel_err(ref.logits(), first) > 1e-3
    ref.reset()
    ref.run_token(5, True)
    assert np.array_equal(ref.logits(), first)


@pytest.mark.parametrize("name", TINY_LFM)
def test_lfm_greedy_ids_match_golden(name, synth):
    g = GOLDEN[name]
    w, path, ref = _oracle(synth, name)
    if hashlib.sha256(Path(path).read_bytes()).hexdigest() != g["sha256"]:
        pytest.fail("synthetic GGUF writer output changed: rerun tests/golden/make_greedy_golden.py")
    ids = ref.generate(g["prompt"], len(g["ids"]))
    n = next((i for i, m in enumerate(g["margins"]) if m < 1e-3), len(g["ids"]))
    assert n >= 8
    assert ids[:n] == g["ids"][:n]


def test_lfm_select_classes_closed_form():
    """TOPK256 slot t: the largest logit among ids t, t + 256, ... and its first id
    (numpy's argmax over the strided view); the greedy token is the overall maximum."""
    rng = np.random.default_rng(3)
    for vocab in (65536, 1000, 700, 300):
        lg = rng.standard_normal(vocab).astype(np.float32)
        lg[rng.integers(0, vocab, 40)] = 2.5  # repeated maxima inside classes
        tok, pairs = orc.lfm_select(lg)
        v, ids = _pairs(pairs)
        for t in range(256):
            col = lg[t::256]
            if col.size == 0:
                assert v[t] == NEG_BIG and ids[t] == 0
                continue
            j = int(np.argmax(col))
            assert v[t] == col[j] and ids[t] == t + 256 * j, (vocab, t)
        assert lg[tok] == lg.max()


def test_lfm_select_ties_follow_the_tree():
    """Equal slot maxima resolve by ARGMAX_WGSL's stride-128..1 tree, which keeps the
    left slot unless the right one is strictly greater (worked by hand):
    slots 64 and 128 tie above the rest -> stride 128 moves slot 128 into slot 0,
    stride 64 keeps slot 0 against slot 64 -> the id from slot 128, not slot 64."""
    lg = np.full(1024, -1.0, dtype=np.float32)
    lg[64 + 256] = 3.0  # slot 64
    lg[128 + 512] = 3.0  # slot 128
    tok, _ = orc.lfm_select(lg)
    assert tok == 128 + 512
    # slots 0 and 128 tie: stride 128 keeps slot 0
    lg = np.full(1024, -1.0, dtype=np.float32)
    lg[0 + 768] = 3.0
    lg[128] = 3.0
    tok, _ = orc.lfm_select(lg)
    assert tok == 768


def test_lfm_select_nan_and_floor():
    """NaN never wins a slot; a slot whose values never exceed -3.402823e38 keeps its start
    value (-3.402823e38, id 0)."""
    lg = np.full(512, -np.inf, dtype=np.float32)
    lg[3] = np.nan
    lg[3 + 256] = 0.5
    lg[7] = NEG_BIG
    tok, pairs = orc.lfm_select(lg)
    v, ids = _pairs(pairs)
    assert v[3] == np.float32(0.5) and ids[3] == 259
    assert v[7] == NEG_BIG and ids[7] == 0
    assert v[8] == NEG_BIG and ids[8] == 0
    assert tok == 259


def test_lfm_sampling_uses_class_candidates(synth):
    """The candidate path runs for sampling or any penalty other than 1 (needsCandidateReadback,
    sampling.ts:18-21) over the 256 slots: with temperature 0 and a penalty it picks the best
    penalized slot, which a penalty list over all logits would not always do."""
    w, path, ref = _oracle(synth, "tiny-lfm2")
    prompt = np.random.default_rng(8).integers(0, w.spec.vocab, 6).tolist()
    for t in prompt[:-1]:
        ref.run_token(t, False)
    greedy = ref.run_token(prompt[-1], True)
    lg = ref.logits().copy()
    _, pairs = orc.lfm_select(lg)
    seen = prompt + [greedy]
    ref.reset()
    for t in prompt[:-1]:
        ref.run_token(t, False)
    got = ref.run_token(prompt[-1], True, repetition_penalty=1.5, seen=seen)
    v, ids = _pairs(pairs)
    pen = np.where(np.isin(ids, seen), np.where(v > 0, v.astype(np.float64) / 1.5, v * 1.5), v.astype(np.float64))
    assert got == int(ids[int(np.argmax(pen))])
    assert got == orc.sample_candidates(pairs, 0.0, 1.0, 0, 1.5, seen, 0.0)


def test_lfm_generate_loop(synth):
    """generateLfmWgsl (:219-306): one more step runs after the last generated id (its pick
    is the cached next id), an empty prompt with no cached id starts from id 0, and the
    definition's default penalty is not applied."""
    w, path, ref = _oracle(synth, "tiny-lfm2", default_repetition_penalty=1.7)
    prompt = np.random.default_rng(9).integers(0, w.spec.vocab, 8).tolist()
    ids = ref.generate(prompt, 5)
    assert len(ids) == 5 and ref.position == len(prompt) + 5
    assert ref.cached_next_id is not None
    ref2 = _oracle(synth, "tiny-lfm2")[2]
    assert ref2.generate(prompt, 5, repetition_penalty=1.0) == ids
    ref3 = _oracle(synth, "tiny-lfm2")[2]
    first = ref3.generate([], 3)
    assert first[0] == 0 and ref3.position == 3


def test_lfm_context_exhaustion_message(synth):
    w, path, ref = _oracle(synth, "tiny-lfm2")
    for t in range(w.max_context):
        ref.run_token(t % w.spec.vocab, False)
    with pytest.raises(RuntimeError, match=f"LFM WGSL context exhausted at {w.max_context} tokens"):
        ref.run_token(1, True)
