"""Writes config_golden.json: token ids of the benchmark-sized decoders.

For each configuration (SmolLM2-135M Q4_K_M and Q8_0 with 32-token prompts,
Qwen3-0.6B Q4_K_M with a 2048-token prompt, Gemma-3-270M Q4_K_M with a
1024-token prompt and top-k 40 / T 0.8 sampling) the oracle, the CPU
restatement of the reference's runToken + generateLlamaWgsl
(llama-wgsl-runtime.ts:242-314, :1025-1150), generates 128 tokens from the
workload's seeded prompt with an fp16 K/V cache, token by token as the
reference does. Each entry keeps the GGUF file's SHA-256 (a change of the
synthetic writer shows up as a stale fixture), a digest of the prompt ids,
the ids, and the float32 top-1/top-2 logit margin after every step.

Run: python tests/golden/make_config_golden.py [names...]   (~15 min on 8 cores)
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from chonklm_amd import WORKLOADS, write_synthetic_gguf  # noqa: E402
from oracle.oracle import OracleModel  # noqa: E402

CONFIGS = ["smollm2-135m-q4_k_m", "smollm2-135m-q8_0", "qwen3-0.6b-q4_k_m", "gemma3-270m-q4_k_m"]
STEPS = 128
PROMPT_SEED = 1234
SAMPLE_SEED = 9
OUT = Path(__file__).with_name("config_golden.json")


def sha256_file(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    return h.hexdigest()


def prompt_digest(ids) -> str:
    return hashlib.sha256(",".join(map(str, ids)).encode()).hexdigest()[:16]


def main(names) -> None:
    out = json.loads(OUT.read_text()) if OUT.exists() else {}
    threads = os.cpu_count() or 8
    with tempfile.TemporaryDirectory() as tmp:
        for name in names:
            w = WORKLOADS[name]
            path = str(Path(tmp) / f"{name}.gguf")
            write_synthetic_gguf(w, path, threads=threads)
            prompt = w.prompt(PROMPT_SEED)
            ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.prompt_tokens + STEPS + 8, kv_f16=True,
                              threads=threads, eos_ids=w.eos_ids)
            margins: list[float] = []
            t0 = time.time()
            ids = ref.generate(prompt, STEPS, temperature=w.temperature, top_k=w.top_k, top_p=w.top_p,
                               seed=SAMPLE_SEED, margins=margins)
            out[name] = {"sha256": sha256_file(path), "prompt_seed": PROMPT_SEED, "prompt_tokens": len(prompt),
                         "prompt_digest": prompt_digest(prompt), "temperature": w.temperature, "top_k": w.top_k,
                         "top_p": w.top_p, "seed": SAMPLE_SEED, "ids": ids, "margins": margins}
            ref.close()
            os.remove(path)
            print(f"{name}: {len(ids)} ids in {time.time() - t0:.0f} s, min margin {min(margins):.3e}", flush=True)
            OUT.write_text(json.dumps(out, indent=None, separators=(",", ":")) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or CONFIGS)
