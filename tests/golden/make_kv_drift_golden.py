"""Writes kv_drift_golden.json: the fp16 K/V cache against the reference's fp32 K/V.

The reference keeps K and V in fp32 (llama-wgsl-runtime.ts:830-831); this
build's default cache is fp16. For the Qwen3-0.6B Q4_K_M configuration
(2048-token prompt, greedy), the Gemma-3-270M Q4_K_M configuration
(1024-token prompt, top-k 40 / T 0.8, seed 9) and the SmolLM2-135M Q4_K_M
configuration (32-token prompt, greedy) the oracle runs the reference
loop twice in lockstep over the same token stream, once with an fp32 cache
(the reference's semantics, whose choices drive the stream) and once with
fp16 rounding on store. Every step records the fp32 run's token, its top-1 /
top-2 logit margin, the drift max|l16 - l32| / max|l32| of the logits, and
whether the fp16 run picks the same token.

Run: python tests/golden/make_kv_drift_golden.py [name ...]   (~25 min on 8 cores)
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from chonklm_amd import WORKLOADS, write_synthetic_gguf  # noqa: E402
from oracle.oracle import OracleModel  # noqa: E402

CONFIGS = ["qwen3-0.6b-q4_k_m", "gemma3-270m-q4_k_m", "smollm2-135m-q4_k_m"]
STEPS = 128
OUT = Path(__file__).with_name("kv_drift_golden.json")


def sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    return h.hexdigest()


def main(names) -> None:
    out = json.loads(OUT.read_text()) if OUT.exists() else {}
    threads = max(1, (os.cpu_count() or 8) // 2)
    with tempfile.TemporaryDirectory() as tmp:
        for name in names:
            w = WORKLOADS[name]
            path = str(Path(tmp) / f"{name}.gguf")
            write_synthetic_gguf(w, path, threads=threads)
            prompt = w.prompt(1234)
            ctx = w.prompt_tokens + STEPS + 8
            r32 = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=False, threads=threads)
            r16 = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=threads)
            samp = dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, seed=9)
            t0 = time.time()
            for t in prompt[:-1]:
                r32.run_token(t, False)
                r16.run_token(t, False)
            ids, margins, drift, agree = [], [], [], []
            tok = prompt[-1]
            hist = list(prompt)
            for step in range(STEPS):
                a = r32.run_token(tok, True, penalized=hist, seen=hist, **samp)
                b = r16.run_token(tok, True, penalized=hist, seen=hist, **samp)
                l32, l16 = r32.logits().astype(np.float64), r16.logits().astype(np.float64)
                top2 = np.sort(l32)[-2:]
                ids.append(a)
                margins.append(float(top2[1] - top2[0]))
                drift.append(float(np.max(np.abs(l16 - l32)) / np.max(np.abs(l32))))
                agree.append(bool(a == b))
                tok = a
                hist.append(a)
            out[name] = {"sha256": sha256_file(path), "prompt_seed": 1234, "sampling": samp, "ids_fp32_kv": ids,
                         "margins_fp32_kv": margins, "drift_fp16_vs_fp32": drift, "same_token_fp16": agree}
            print(f"{name}: {time.time() - t0:.0f} s, max drift {max(drift):.3e}, min margin {min(margins):.3e}, "
                  f"fp16 picks differ at {sum(not x for x in agree)} steps", flush=True)
            r32.close()
            r16.close()
            os.remove(path)
            OUT.write_text(json.dumps(out, separators=(",", ":")) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or CONFIGS)
