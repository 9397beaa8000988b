"""Engines on different threads decoding on one GPU at the same time.

The reference runs one engine per page and guards each engine with its own
`active` flag (llama-wgsl-runtime.ts:1221-1224); several engines may exist at
once. This build's spin-merging decode attention needs its whole grid resident,
so only the first engine on a GPU that qualifies uses it and later engines use
the arrival-counter attention; the no-allocation prompt pass shares one scratch
array per GPU and takes turns on a per-GPU lock. Both are checked under real
concurrency: two Qwen3-0.6B-shaped engines at a 2K context decode on two
threads at once and each matches the oracle, and two engines run the
no-allocation prompt pass on two threads at once with the results of running
them one after the other.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, load_llama_wgsl_model
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

NAME = "qwen3-0.6b-q4_k_m"


def _run_threads(fns):
    errs = []

    def wrap(f):
        try:
            f()
        except BaseException as x:  # noqa: BLE001 (re-raised below)
            errs.append(x)

    ts = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in ts), "a decoding thread did not finish"
    if errs:
        raise errs[0]


def test_two_engines_decode_concurrently(synth):
    w = WORKLOADS[NAME]
    path = synth(NAME)
    ctx, pos0, steps = 2112, 2048, 12
    engines = []
    for _ in range(2):
        md = w.model_def(path)
        md.max_context = ctx
        engines.append(load_llama_wgsl_model(md).engine)
    # at most one engine on the GPU holds the spin-merging attention (the first one,
    # unless an engine of an earlier test is still alive), and never the second
    spin = [e.info["spin_attention"] for e in engines]
    assert spin[1] == 0 and sum(spin) <= 1
    out = [dict(ids=[], logits=[]) for _ in engines]
    starts = [101, 202]

    def decode(i):
        def run():
            eng = engines[i]
            eng.fake_context(pos0, seed=starts[i])
            tok = starts[i]
            for _ in range(steps):
                tok = eng.run_token(tok, True)
                out[i]["ids"].append(tok)
                out[i]["logits"].append(eng.read_logits())
        return run

    for _ in range(2):  # twice, so both engines decode through each other's steps
        for o in out:
            o["ids"].clear()
            o["logits"].clear()
        _run_threads([decode(0), decode(1)])
    for i, eng in enumerate(engines):
        ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=16)
        ref.fake_context(pos0, seed=starts[i])
        tok = starts[i]
        for s in range(steps):
            tok = ref.run_token(tok, True)
            e = rel_err(out[i]["logits"][s], ref.logits())
            assert e <= 1e-3, f"engine {i} step {s}: logits rel err {e:.3e}"
            assert out[i]["ids"][s] == tok, f"engine {i} step {s}: id {out[i]['ids'][s]} != {tok}"
        ref.close()
    # a third engine created after the first is gone takes the spin-merging attention again
    engines[0].dispose()
    md = w.model_def(path)
    md.max_context = ctx
    third = load_llama_wgsl_model(md).engine
    assert third.info["spin_attention"] == spin[0]
    third.dispose()
    engines[1].dispose()


def test_noalloc_prompt_passes_take_turns(synth):
    w = WORKLOADS[NAME]
    path = synth(NAME)
    engines = []
    for _ in range(2):
        md = w.model_def(path)
        md.max_context = 512
        engines.append(load_llama_wgsl_model(md).engine)
    n = min(engines[0].info["noalloc_prefill_rows"], 300)
    assert n >= 64
    rng = np.random.default_rng(3)
    prompts = [rng.integers(0, w.spec.vocab, n + 1).tolist() for _ in engines]

    def logits_after(i):
        return engines[i].run_token(prompts[i][-1], True), engines[i].read_logits()

    # one after the other
    want = []
    for i, eng in enumerate(engines):
        eng.reset()
        eng.prefill_noalloc(prompts[i][:-1])
        want.append(logits_after(i))
    # at the same time, several times
    for _ in range(3):
        for eng in engines:
            eng.reset()
        _run_threads([lambda i=i: engines[i].prefill_noalloc(prompts[i][:-1]) for i in range(2)])
        for i in range(2):
            tok, lg = logits_after(i)
            assert tok == want[i][0]
            assert rel_err(lg, want[i][1]) <= 1e-6, f"engine {i}: logits differ from the sequential passes"
    for eng in engines:
        eng.dispose()
