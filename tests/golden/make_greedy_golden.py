"""Writes greedy_golden.json: greedy token ids of the tiny synthetic decoders.

The ids come from tests/numpy_ref.py, a float64 forward pass written from the
model's closed forms (no fp32 reduction-order mimicry) over the synthetic
GGUF files that chonklm_amd.write_synthetic_gguf produces. Each file's
SHA-256 is stored with its ids, so a change of the writer shows up as a
stale fixture rather than as a parity failure. Every step also records the
float64 top-2 logit margin; the test compares a step only while every margin
so far exceeds the fp32 noise floor.

Run: python tests/golden/make_greedy_golden.py [model ...]   (default: every model;
entries of models not named are kept)
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from chonklm_amd import WORKLOADS, write_synthetic_gguf  # noqa: E402
from tests.numpy_ref import NumpyDecoder, NumpyLfm2  # noqa: E402

MODELS = ["tiny-qwen3", "tiny-llama", "tiny-llama-q8", "tiny-gemma3", "tiny-openelm", "tiny-lfm2", "tiny-lfm2-q8"]
STEPS = 24


def sha256(path: str) -> str:
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def main(models: list[str]) -> None:
    dst = Path(__file__).with_name("greedy_golden.json")
    out = json.loads(dst.read_text()) if dst.exists() else {}
    with tempfile.TemporaryDirectory() as tmp:
        for name in models:
            w = WORKLOADS[name]
            path = str(Path(tmp) / f"{name}.gguf")
            write_synthetic_gguf(w, path, threads=4)
            prompt = np.random.default_rng(1234).integers(0, w.spec.vocab, 12).tolist()
            cls = NumpyLfm2 if w.spec.arch == "lfm2" else NumpyDecoder
            dec = cls(path, w.spec.vocab, w.max_context, kv_f16=True)
            for t in prompt[:-1]:
                dec.step(t)
            lg = dec.step(prompt[-1])
            ids, margins = [], []
            for _ in range(STEPS):
                top2 = np.sort(lg)[-2:]
                tok = int(np.argmax(lg))
                ids.append(tok)
                margins.append(float(top2[1] - top2[0]))
                lg = dec.step(tok)
            out[name] = {"sha256": sha256(path), "prompt": prompt, "ids": ids, "margins": margins}
            print(name, ids[:8], min(margins))
    dst.write_text(json.dumps({k: out[k] for k in MODELS if k in out}, indent=1) + "\n")


if __name__ == "__main__":
    main(sys.argv[1:] or MODELS)
