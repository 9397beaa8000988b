"""The oracle's Granite-4.0-H decoder (src/lib/granite-wgsl-runtime.ts) against closed forms.

tests/numpy_ref.py's NumpyGranite restates the hybrid decoder in float64 numpy
and evaluates each Mamba2 block in its dual form from the history of every
position's (dt, B, x): y_t = sum_tau (C_t . B_tau) prod_u exp(dt_u A) dt_tau
x_tau + D x_t, the convolution over the history of xBC, where the oracle runs
the reference's shifted window and 128-state recurrence. Bars: logits within
2e-5 relative at every step (the oracle sits at ~2e-7); a decoder with D
dropped misses that bar by four orders of magnitude, so the check sees the
Mamba2 terms. The generate loop is pinned by invariants of generateGraniteWgsl
(:223-292), and the loader's checks (:359-395) by files built to fail them.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, _lib
from chonklm_amd._lib import lib
from oracle.oracle import OracleModel
from tests.conftest import rel_err
from tests.numpy_ref import NumpyGranite

TINY_GRANITE = ["tiny-granite", "tiny-granite-q8"]


def _oracle(synth, name, kv_f16=True):
    w = WORKLOADS[name]
    path = synth(name)
    return w, path, OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=kv_f16, eos_ids=w.eos_ids,
                                threads=4)


def _walk(ref, dec, prompt, extra):
    errs = []
    tok = prompt[0]
    for i in range(len(prompt) + extra):
        if i < len(prompt):
            tok = prompt[i]
        a = ref.run_token(tok, True)
        want = dec.step(tok)
        errs.append(rel_err(ref.logits(), want))
        assert a == int(np.argmax(ref.logits()))
        if i >= len(prompt) - 1:
            tok = a
    return errs


@pytest.mark.parametrize("kv_f16", [True, False])
@pytest.mark.parametrize("name", TINY_GRANITE)
def test_granite_logits_match_float64_decoder(name, kv_f16, synth):
    w, path, ref = _oracle(synth, name, kv_f16)
    assert ref.granite and not ref.lfm and ref.context == 4096
    dec = NumpyGranite(path, kv_f16=kv_f16)
    prompt = np.random.default_rng(5).integers(0, w.spec.vocab, 14).tolist()
    errs = _walk(ref, dec, prompt, 10)
    assert max(errs) <= 2e-5, [f"{e:.2e}" for e in errs]


def test_the_float64_check_sees_the_mamba_terms(synth):
    """Without D * x (or with the taps reversed) the float64 decoder leaves the bar far behind,
    so agreement within it is not the embedding and the attention layer alone."""
    w, path, _ = _oracle(synth, "tiny-granite")
    prompt = np.random.default_rng(5).integers(0, w.spec.vocab, 8).tolist()
    for mutate in ("D", "taps"):
        _, _, ref = _oracle(synth, "tiny-granite")
        dec = NumpyGranite(path, kv_f16=True)
        for lay in dec.layers:
            if lay["mamba"]:
                if mutate == "D":
                    lay["D"] = lay["D"] * 0
                else:
                    lay["cw"] = lay["cw"][:, ::-1].copy()
        errs = _walk(ref, dec, prompt, 0)
        assert max(errs) > 1e-2, mutate


def test_granite_generate_loop_invariants(synth):
    """generateGraniteWgsl runs the token after the last generated one (position = prompt +
    generated), caches prompt + generated and the next pick, starts an empty prompt with no
    cached id from id 0, and continues from the cached id with an empty suffix; greedy ids
    follow the oracle's own argmax of its logits."""
    w, path, ref = _oracle(synth, "tiny-granite")
    prompt = np.random.default_rng(2).integers(0, w.spec.vocab, 9).tolist()
    g = ref.generate(prompt, 6)
    assert len(g) == 6 and ref.position == len(prompt) + 6
    assert ref.cached_token_ids == prompt + g
    nxt = ref.cached_next_id
    assert nxt == int(np.argmax(ref.logits()))
    # same prompt again: the suffix is empty and the cached id is the first pick
    g2 = ref.generate(prompt + g, 3)
    assert g2[0] == nxt
    # a fresh run of the whole history reaches the same next id
    _, _, fresh = _oracle(synth, "tiny-granite")
    fresh.generate(prompt + g, 1)
    assert fresh.cached_token_ids[-1] == nxt
    # empty prompt, nothing cached: the reference's nextId default 0 is the first id
    _, _, empty = _oracle(synth, "tiny-granite")
    assert empty.generate([], 3)[0] == 0


def _gguf(kv: list[tuple[str, int, bytes]]) -> bytes:
    def s(x: str) -> bytes:
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    body = b"".join(s(k) + struct.pack("<I", t) + v for k, t, v in kv)
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, len(kv)) + body
    return head + bytes(4096 - len(head))


def _create(path):
    d = _lib.ModelDefC()
    d.id = b"granite-t"
    d.vocab, d.layers, d.max_context = 1000, 2, 64
    d.default_repetition_penalty = 1.0
    h = C.c_void_p()
    rc = lib().chonk_engine_create(C.byref(d), str(path).encode(), C.byref(h))
    return rc, lib().chonk_last_error().decode()


def test_granite_loader_refuses_files_the_reference_refuses(tmp_path):
    """validateGraniteGguf (:359-371): file types other than Q8_0 (7) / Q4_K_M (15), and the
    tensors every Granite file holds, with the reference's wording."""
    arch = ("general.architecture", 8, struct.pack("<Q", 13) + b"granitehybrid")
    p = tmp_path / "ft.gguf"
    p.write_bytes(_gguf([arch, ("general.file_type", 4, struct.pack("<I", 2))]))
    rc, msg = _create(p)
    assert rc == _lib.CHONK_EINVAL and "Granite WGSL granite-t: expected GGUF Q8_0 or Q4_K_M file_type, got 2" in msg
    p.write_bytes(_gguf([arch, ("general.file_type", 4, struct.pack("<I", 15))]))
    rc, msg = _create(p)
    assert rc == _lib.CHONK_EINVAL and "Granite WGSL granite-t: GGUF missing tensor token_embd.weight" in msg
