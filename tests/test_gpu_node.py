"""The Node host on the GPU: generateLlamaWgsl / runToken through the N-API addon.

Token ids must equal the oracle's for the device-driven loop, the stepped
loop with onToken (including prefix reuse of the previous conversation), a
sampled run, and shouldStop; the loaded object's cachedTokenIds /
cachedNextId follow the reference's rules (llama-wgsl-runtime.ts:242-324).
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import WORKLOADS
from oracle.oracle import OracleModel
from tests.test_cpu_node import ADDON, model, run_driver

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not ADDON.exists(), reason="N-API addon not built")]


def test_node_generate_matches_oracle(synth):
    w = WORKLOADS["tiny-qwen3"]
    path = synth("tiny-qwen3")
    rng = np.random.default_rng(31)
    p1 = rng.integers(0, w.spec.vocab, 14).tolist()
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True, eos_ids=w.eos_ids)
    want1 = ref.generate(p1, 10)
    cache1 = (list(ref.cached_token_ids), ref.cached_next_id)
    p2 = p1 + want1 + rng.integers(0, w.spec.vocab, 3).tolist()
    want2 = ref.generate(p2, 8)
    cache2 = (list(ref.cached_token_ids), ref.cached_next_id)
    # shouldStop after three tokens: the first three ids of an unbounded run
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    want3 = ref.generate(p1, 3)
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    want4 = ref.generate(p1, 12, temperature=0.8, top_k=20, seed=5)

    md = model(path, vocab=w.spec.vocab, layers=w.spec.layers, maxContext=w.max_context, eosIds=w.eos_ids,
               kvDtype="float16")
    out = run_driver({"kind": "generate", "model": md, "prompt": p1[:6], "generate": [
        {"prompt": p1, "opts": {"maxNewTokens": 10}},
        {"prompt": p2, "opts": {"maxNewTokens": 8}, "stepped": True, "busyProbe": True},
        {"prompt": p1, "opts": {"maxNewTokens": 50}, "stepped": True, "stopAfter": 3, "reset": True},
        {"prompt": p1, "opts": {"maxNewTokens": 12, "temperature": 0.8, "topK": 20, "seed": 5}, "reset": True},
    ]}, timeout=300)
    r = out["runs"]
    assert out["steps"] == ["runtime", "ready"]
    assert r[0]["ids"] == want1 and (r[0]["cached"], r[0]["next"]) == cache1
    assert r[1]["ids"] == want2 == r[1]["seen"] and (r[1]["cached"], r[1]["next"]) == cache2
    assert r[2]["ids"] == want3 == r[2]["seen"]
    assert r[3]["ids"] == want4
    assert r[0]["position"] == len(p1) + len(want1) - 1
    st = out["step"]
    assert st["position"] == 6 and st["logitsLength"] == w.spec.vocab
    ref2 = OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True)
    for i, t in enumerate(p1[:6]):
        tok = ref2.run_token(t, i == 5)
    assert st["token"] == tok
    assert np.allclose(st["logitsHead"], ref2.logits()[:8], rtol=1e-3, atol=1e-4)
    # a synchronous call made while the stepped loop holds the engine is refused, and the
    # loop itself continues unharmed (its ids matched above)
    assert r[1]["busy"] == "EBUSY"
    assert out["busy"] in ("EBUSY", None)  # two queued async calls may also run back to back
    assert "disposed" in out["afterDispose"]


def test_node_gpt2_generate_matches_oracle(synth):
    """loadGptWgslModel / generateGptWgsl (gpt-wgsl-runtime.ts:130-249) through the addon on a
    gpt2 file: ids, cachedNextId (the step after the last id also runs) as the oracle."""
    w = WORKLOADS["tiny-gpt2"]
    path = synth("tiny-gpt2")
    rng = np.random.default_rng(37)
    p1 = rng.integers(0, w.spec.vocab, 12).tolist()
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True, eos_ids=w.eos_ids)
    want1 = ref.generate(p1, 9)
    cache1 = (list(ref.cached_token_ids), ref.cached_next_id)
    # a definition default penalty is not applied by generateGptWgsl (gpt-wgsl-runtime.ts:198-203)
    md = model(path, runtime="gpt-webgpu", vocab=w.spec.vocab, layers=w.spec.layers, maxContext=w.max_context,
               eosIds=w.eos_ids, kvDtype="float16", defaultRepetitionPenalty=1.5)
    out = run_driver({"kind": "generate", "model": md, "prompt": p1[:4], "generate": [
        {"prompt": p1, "opts": {"maxNewTokens": 9}},
    ]}, timeout=300)
    r = out["runs"]
    assert r[0]["ids"] == want1 and (r[0]["cached"], r[0]["next"]) == cache1
    assert r[0]["position"] == ref.position


def test_node_lfm2_generate_matches_oracle(synth):
    """loadLfmWgslModel / generateLfmWgsl (lfm-wgsl-runtime.ts:169-306) through the addon on an
    lfm2 file: ids and cachedNextId (the step after the last id also runs) as the oracle,
    greedy and sampled; the definition's default penalty is not applied."""
    w = WORKLOADS["tiny-lfm2"]
    path = synth("tiny-lfm2")
    rng = np.random.default_rng(41)
    p1 = rng.integers(0, w.spec.vocab, 12).tolist()
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True, eos_ids=w.eos_ids)
    want1 = ref.generate(p1, 9)
    cache1 = (list(ref.cached_token_ids), ref.cached_next_id)
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    want2 = ref.generate(p1, 10, temperature=0.8, top_k=20, seed=5)
    md = model(path, runtime="lfm2-webgpu", vocab=w.spec.vocab, layers=w.spec.layers, maxContext=w.max_context,
               eosIds=w.eos_ids, kvDtype="float16", defaultRepetitionPenalty=1.5)
    out = run_driver({"kind": "generate", "model": md, "prompt": p1[:4], "generate": [
        {"prompt": p1, "opts": {"maxNewTokens": 9}},
        {"prompt": p1, "opts": {"maxNewTokens": 10, "temperature": 0.8, "topK": 20, "seed": 5}, "reset": True},
    ]}, timeout=300)
    r = out["runs"]
    assert r[0]["ids"] == want1 and (r[0]["cached"], r[0]["next"]) == cache1
    assert r[1]["ids"] == want2
