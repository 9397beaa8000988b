"""Writes run_golden.json: 128-step runs of the benchmark-sized decoders with logits.

For each configuration the oracle (the CPU restatement of the reference's
runToken + generateLlamaWgsl, llama-wgsl-runtime.ts:242-314, :1025-1150)
generates 128 tokens from the workload's seeded prompt, token by token as the
reference does, once with an fp16 K/V cache (this build's default) and once
with the reference's fp32 cache (:830-831):

* SmolLM2-135M Q4_K_M and Q8_0 (32-token prompts) and Qwen3-0.6B Q4_K_M
  (2048-token prompt) greedy with repetitionPenalty 1.3: the reference's
  penalty path (stage-1 penalty on the listed ids, :1646-1662, :3684-3690)
  keeps the random-weight models out of the short fixed-point cycles that
  plain greedy decoding falls into, so the 128 ids keep changing;
* Gemma-3-270M Q4_K_M (1024-token prompt) with its top-k 40 / T 0.8 seeded
  sampling and no penalty.

Each run keeps the ids, the float32 top-1/top-2 margin of the (unpenalized)
logits after every step, and every 16th step's 16 largest logits (ids and
values, steps 0, 16, ..., 112 and 127), so that the GPU's logits can be held
to the oracle's along the whole run. The GGUF file's SHA-256 and a digest of
the prompt key the fixture.

Run: python tests/golden/make_run_golden.py [names...]   (~40 min on 8 cores)
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

CONFIGS = ["smollm2-135m-q4_k_m", "smollm2-135m-q8_0", "qwen3-0.6b-q4_k_m", "gemma3-270m-q4_k_m"]
STEPS = 128
PROMPT_SEED = 1234
SAMPLE_SEED = 9
PENALTY = 1.3
TOP = 16
OUT = Path(__file__).with_name("run_golden.json")


def snapshot_steps(n: int = STEPS) -> list[int]:
    return sorted(set(list(range(0, n, 16)) + [n - 1]))


def sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    return h.hexdigest()


def prompt_digest(ids) -> str:
    return hashlib.sha256(",".join(map(str, ids)).encode()).hexdigest()[:16]


def sampling(w) -> dict:
    if w.temperature > 0:
        return {"temperature": w.temperature, "top_k": w.top_k, "top_p": w.top_p, "repetition_penalty": 1.0,
                "seed": SAMPLE_SEED}
    return {"temperature": 0.0, "top_k": 0, "top_p": 1.0, "repetition_penalty": PENALTY, "seed": SAMPLE_SEED}


def main(names, threads: int) -> None:
    out = json.loads(OUT.read_text()) if OUT.exists() else {}
    want = set(snapshot_steps())
    with tempfile.TemporaryDirectory() as tmp:
        for name in names:
            w = WORKLOADS[name]
            path = str(Path(tmp) / f"{name}.gguf")
            write_synthetic_gguf(w, path, threads=threads)
            prompt = w.prompt(PROMPT_SEED)
            samp = sampling(w)
            entry = {"sha256": sha256_file(path), "prompt_seed": PROMPT_SEED, "prompt_tokens": len(prompt),
                     "prompt_digest": prompt_digest(prompt), "sampling": samp}
            for kv in ("f16", "f32"):
                ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.prompt_tokens + STEPS + 8,
                                  kv_f16=kv == "f16", threads=threads, eos_ids=w.eos_ids)
                margins: list[float] = []
                snaps: dict[str, dict] = {}

                def keep(i: int, lg: np.ndarray) -> None:
                    if i in want:
                        top = np.argsort(-lg, kind="stable")[:TOP]
                        snaps[str(i)] = {"ids": [int(t) for t in top], "values": [float(lg[t]) for t in top],
                                         "absmax": float(np.max(np.abs(lg)))}

                t0 = time.time()
                ids = ref.generate(prompt, STEPS, temperature=samp["temperature"], top_k=samp["top_k"],
                                   top_p=samp["top_p"], repetition_penalty=samp["repetition_penalty"],
                                   seed=samp["seed"], margins=margins, on_logits=keep)
                ref.close()
                entry[kv] = {"ids": ids, "margins": margins, "logits": snaps}
                print(f"{name} {kv}: {len(ids)} ids ({len(set(ids))} distinct) in {time.time() - t0:.0f} s, "
                      f"min margin {min(margins):.3e}", flush=True)
            same = sum(a == b for a, b in zip(entry["f16"]["ids"], entry["f32"]["ids"]))
            print(f"{name}: fp16 and fp32 runs agree on {same} of {STEPS} ids", flush=True)
            out[name] = entry
            os.remove(path)
            OUT.write_text(json.dumps(out, indent=None, separators=(",", ":")) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or CONFIGS, int(os.environ.get("GOLDEN_THREADS", os.cpu_count() or 8)))
