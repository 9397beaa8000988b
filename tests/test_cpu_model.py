"""The oracle's decoder against an independent float64 forward pass and closed forms.

tests/numpy_ref.py restates the decoder in float64 numpy (vectorised, no
WGSL reduction order); the oracle follows the WGSL fp32 arithmetic. Bars:
logits within 1e-4 relative (1e-3 for gemma3) at every step of a short prompt + decode,
identical greedy ids (golden fixture tests/golden/greedy_golden.json), K/V
cache rows within one binary16 ulp, and closed forms that a wrong head
mapping, norm or projection would break.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from chonklm_amd import WORKLOADS
from oracle.oracle import OracleModel
from tests import ggufpy
from tests.conftest import rel_err
from tests.numpy_ref import NumpyDecoder, NumpyGpt2

TINY = ["tiny-qwen3", "tiny-llama", "tiny-llama-q8", "tiny-gemma3", "tiny-openelm"]
GOLDEN = json.loads((Path(__file__).parent / "golden" / "greedy_golden.json").read_text())


def _oracle(synth, name, kv_f16=True):
    w = WORKLOADS[name]
    path = synth(name)
    return w, path, OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=kv_f16,
                                eos_ids=w.eos_ids, threads=4)


@pytest.mark.parametrize("name", TINY + ["tiny-qwen3-hd128"])
def test_logits_match_float64_decoder(name, synth):
    w, path, ref = _oracle(synth, name)
    dec = NumpyDecoder(path, w.spec.vocab, w.max_context, kv_f16=True)
    prompt = np.random.default_rng(5).integers(0, w.spec.vocab, 10).tolist()
    tok = prompt[0]
    for i in range(len(prompt) + 6):
        if i < len(prompt):
            tok = prompt[i]
        a = ref.run_token(tok, True)
        want = dec.step(tok)
        # gemma3: sqrt(H)-scaled residual, sandwich norms and binary16 rounding edges of the
        # fp32-vs-fp64 K/V amplify differences; the contract is 1e-3
        bar = 1e-3 if name == "tiny-gemma3" else 1e-4
        assert rel_err(ref.logits(), want) <= bar, f"{name} step {i}"
        if i >= len(prompt) - 1:
            tok = a


@pytest.mark.parametrize("name", TINY)
def test_greedy_ids_match_golden(name, synth):
    g = GOLDEN[name]
    w, path, ref = _oracle(synth, name)
    digest = hashlib.sha256(Path(path).read_bytes()).hexdigest()
    if digest != g["sha256"]:
        pytest.fail("synthetic GGUF writer output changed: rerun tests/golden/make_greedy_golden.py")
    ids = ref.generate(g["prompt"], len(g["ids"]) + 1)
    # compare while the float64 top-2 margin is far above fp32 noise
    n = next((i for i, m in enumerate(g["margins"]) if m < 1e-3), len(g["ids"]))
    assert n >= 8
    assert ids[:n] == g["ids"][:n]


def _layer_heads(w, layer):
    sp = w.spec
    return ((sp.layer_heads or [sp.heads] * sp.layers)[layer], (sp.layer_kv_heads or [sp.kv_heads] * sp.layers)[layer])


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-gemma3", "tiny-openelm"])
def test_kv_rows_match_float64_decoder(name, synth):
    w, path, ref = _oracle(synth, name)
    dec = NumpyDecoder(path, w.spec.vocab, w.max_context, kv_f16=True)
    for t in np.random.default_rng(6).integers(0, w.spec.vocab, 7).tolist():
        ref.run_token(t, False)
        dec.step(t)
    for layer in range(w.spec.layers):
        nkv = _layer_heads(w, layer)[1]
        n = nkv * dec.hd
        for pos in (0, 3, 6):
            for is_v in (False, True):
                got = ref.read_kv(layer, is_v, pos, n)
                want = (dec.V if is_v else dec.K)[layer, :nkv, pos].reshape(-1)
                # both round to binary16; allow one ulp where fp32 and fp64 straddle a rounding edge
                assert np.max(np.abs(got - want)) <= np.max(np.abs(want)) * 2e-3 + 1e-6


@pytest.mark.parametrize("name", TINY)
def test_first_position_attention_returns_value_row(name, synth):
    # softmax over one position is exactly 1: every q head of a group returns its kv head's V row
    w, path, ref = _oracle(synth, name)
    ref.run_token(17, True)
    g = ggufpy.read_gguf(path)
    arch = g.kv["general.architecture"]
    nh, nkv = _layer_heads(w, w.spec.layers - 1)  # the last layer's (openelm varies them per layer)
    hdim = int(g.kv.get(arch + ".attention.key_length", int(g.kv[arch + ".embedding_length"]) // w.spec.heads))
    attn = ref.read(5, nh * hdim).reshape(nh, hdim)
    v = ref.read_kv(w.spec.layers - 1, True, 0, nkv * hdim).reshape(nkv, hdim)
    for h in range(nh):
        assert np.array_equal(attn[h], v[h // (nh // nkv)])


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama"])
def test_final_norm_and_lm_head_closed_form(name, synth):
    w, path, ref = _oracle(synth, name)
    for t in (3, 99, 250):
        ref.run_token(t, True)
    g = ggufpy.read_gguf(path)
    arch = g.kv["general.architecture"]
    H = int(g.kv[arch + ".embedding_length"])
    eps = float(np.float32(g.kv[arch + ".attention.layer_norm_rms_epsilon"]))
    res = ref.read(1, H).astype(np.float64)
    normed = ref.read(2, H).astype(np.float64)
    wn = ggufpy.matrix(g, "output_norm.weight").astype(np.float64)
    want = res / np.sqrt(np.mean(res * res) + eps) * wn
    assert rel_err(normed, want) <= 1e-6
    lm = ggufpy.matrix(g, "output.weight" if "output.weight" in g.tensors else "token_embd.weight")
    logits = lm[: w.spec.vocab].astype(np.float64) @ normed
    assert rel_err(ref.logits(), logits) <= 1e-5


def test_context_exhaustion_message(synth):
    w = WORKLOADS["tiny-llama-q8"]
    path = synth("tiny-llama-q8")
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, 4, eos_ids=w.eos_ids)
    for t in range(4):
        ref.run_token(t + 1, False)
    with pytest.raises(RuntimeError, match="context exhausted at 4 tokens"):
        ref.run_token(1, True)


def test_gpt2_logits_match_float64_decoder(synth):
    """The oracle's GPT-2 path (gpt-wgsl-runtime.ts:749-840: LayerNorm with bias, fused q|k|v,
    biases, GELU-tanh, +-10000 residual clamp, learned positions) against the float64 decoder."""
    w, path, ref = _oracle(synth, "tiny-gpt2")
    assert ref.gpt and ref.vocab == w.spec.vocab
    dec = NumpyGpt2(path, w.max_context, kv_f16=True)
    prompt = np.random.default_rng(6).integers(0, w.spec.vocab, 10).tolist()
    tok = prompt[0]
    for i in range(len(prompt) + 8):
        if i < len(prompt):
            tok = prompt[i]
        a = ref.run_token(tok, True)
        want = dec.step(tok)
        assert rel_err(ref.logits(), want) <= 1e-4, f"step {i}"
        if i >= len(prompt) - 1:
            tok = a


def test_gpt2_generate_loop(synth):
    """generateGptWgsl (:182-249): one runToken past the last generated token, and an empty
    prompt needs a cached next token."""
    w, path, ref = _oracle(synth, "tiny-gpt2")
    prompt = np.random.default_rng(7).integers(0, w.spec.vocab, 9).tolist()
    ids = ref.generate(prompt, 6)
    assert len(ids) <= 6
    if w.eos_ids[0] not in ids:
        assert ref.position == len(prompt) + len(ids)
        assert ref.cached_next_id is not None
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    with pytest.raises(RuntimeError, match="no cached next token"):
        ref.generate([], 3)
