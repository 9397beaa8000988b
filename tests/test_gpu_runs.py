"""128-step runs at the benchmark configurations, with logits along the run.

tests/golden/run_golden.json (tests/golden/make_run_golden.py) holds, for each
configuration and for both K/V caches (this build's fp16 and the reference's
fp32, llama-wgsl-runtime.ts:830-831), the oracle's 128 ids from the workload's
seeded prompt and every 16th step's 16 largest logits. SmolLM2-135M Q4_K_M /
Q8_0 and Qwen3-0.6B Q4_K_M decode greedily with repetitionPenalty 1.3 (the
reference's stage-1 penalty path, :1646-1662, :3684-3690), which keeps the ids
changing over the whole run (45-109 distinct ids) instead of settling into the
short cycles of plain greedy decoding; Gemma-3-270M samples with top-k 40 /
T 0.8.

The GPU runs the reference loop (generateLlamaWgsl, :242-314: the prompt's
last token and every generated id through runToken with the prompt + generated
ids as the penalty and seen lists) and must give the same 128 ids, with the
logits at the snapshot steps within 1e-3 of the oracle's (max |d| over the 16
ids / max |logit|).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, load_llama_wgsl_model

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "run_golden.json").read_text())
CONFIGS = ["smollm2-135m-q4_k_m", "smollm2-135m-q8_0", "qwen3-0.6b-q4_k_m", "gemma3-270m-q4_k_m"]


def _sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    return h.hexdigest()


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("name", CONFIGS)
def test_config_run_matches_golden(synth, name, kv):
    w = WORKLOADS[name]
    path = synth(name)
    g = GOLDEN[name]
    if _sha256(path) != g["sha256"]:
        pytest.fail(f"{name}: synthetic GGUF writer output changed; rerun tests/golden/make_run_golden.py")
    prompt = w.prompt(g["prompt_seed"])
    assert hashlib.sha256(",".join(map(str, prompt)).encode()).hexdigest()[:16] == g["prompt_digest"]
    want = g[kv]
    samp = g["sampling"]
    md = w.model_def(path, kv_dtype=kv)
    md.max_context = len(prompt) + len(want["ids"]) + 8
    eng = load_llama_wgsl_model(md).engine
    eng.prefill(prompt[:-1])
    ids: list[int] = []
    tok = prompt[-1]
    worst = 0.0
    for step in range(len(want["ids"])):
        hist = prompt + ids
        tok = eng.run_token(tok, True, penalized_token_ids=hist, seen_ids=hist, **samp)
        snap = want["logits"].get(str(step))
        if snap is not None:
            lg = eng.read_logits()
            e = float(np.max(np.abs(lg[snap["ids"]] - np.asarray(snap["values"])))) / snap["absmax"]
            worst = max(worst, e)
            assert e <= 1e-3, f"{name} ({kv} K/V) step {step}: logits rel err {e:.3e}"
        ids.append(tok)
        if ids[-1] != want["ids"][step]:
            m = want["margins"][step]
            pytest.fail(f"{name} ({kv} K/V): id {ids[-1]} != {want['ids'][step]} at step {step} "
                        f"(oracle top-2 margin there {m:.3e})")
    assert len(set(ids)) >= 40, f"{name}: only {len(set(ids))} distinct ids over the run"
    eng.dispose()
    print(f"{name} {kv}: 128 ids equal, {len(set(ids))} distinct, worst snapshot logits rel err {worst:.2e}")
