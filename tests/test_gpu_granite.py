"""The Granite-4.0-H runtime (src/lib/granite-wgsl-runtime.ts) on the device against the oracle.

A Mamba2 layer runs as three launches: in_proj with the input RMSNorm in its
prologue; one kernel for the causal 4-tap convolution (+ bias, silu) of the
xBC channels and the 128-state selective scan of every (head, channel), the
convolution window double-buffered by position parity; and out_proj whose
prologue is MAMBA_GATE_NORM (y * silu(z) through an RMSNorm) and whose
epilogue is the residual add scaled by 0.246. Attention layers take the decode
attention kernel with no rotary embedding and scores x 1/64. The lm_head reads
the embedding class-major and scales logits by 1/3 before TOPK256_WGSL's slots.
Workloads: tiny-granite (Q4_K / Q6_K, Mamba2-attention-Mamba2-Mamba2, 16 SSM
heads, GQA 2), tiny-granite-q8 (Q8_0, 12 SSM heads, GQA 3, vocab 700 so the
last classes hold two ids), and the Granite-4.0-H-350M shape (28 Mamba2 and 4
attention layers, vocab 100352: 392 ids per class). Bars: identical token ids;
logits max|d| / max|ref| <= 1e-3.
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import (WORKLOADS, ChonkError, dispose_granite_wgsl, generate_granite_wgsl, load_granite_wgsl_model,
                         load_llama_wgsl_model, reset_granite_wgsl_conversation)
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TINY_GRANITE = ["tiny-granite", "tiny-granite-q8"]


def _pair(synth, name, kv="f16", **over):
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path, kv_dtype=kv)
    for k, v in over.items():
        setattr(md, k, v)
    loaded = load_granite_wgsl_model(md)
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, md.max_context, kv_f16=(kv == "f16"), eos_ids=w.eos_ids)
    return w, loaded, ref


def _prompt(w, seed=0, n=None):
    return np.random.default_rng(seed).integers(0, w.spec.vocab, n or w.prompt_tokens).tolist()


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("name", TINY_GRANITE)
def test_granite_step_logits_and_tokens(name, kv, synth):
    w, loaded, ref = _pair(synth, name, kv=kv)
    eng = loaded.engine
    assert eng.info["architecture"] == 6
    assert eng.info["context"] == 4096
    prompt = _prompt(w)
    tok = prompt[0]
    for i in range(len(prompt) + 12):
        need = i >= len(prompt) - 1 or i % 5 == 0
        if i < len(prompt):
            tok = prompt[i]
        a = eng.run_token(tok, need)
        b = ref.run_token(tok, need)
        if need:
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"{name} step {i}: logits rel err {e:.3e}"
            assert a == b, f"{name} step {i}: token {a} != {b}"
            if i >= len(prompt) - 1:
                tok = a
    assert eng.position == ref.position == len(prompt) + 12


def test_granite_candidates_are_class_maxima_of_scaled_logits(synth):
    """The lm_head epilogue's 256 candidates equal TOPK256_WGSL's slots of the device's own
    (x 1/3) logits: slot t holds the first maximum of ids t, t + 256, ..."""
    w, loaded, ref = _pair(synth, "tiny-granite-q8")
    eng = loaded.engine
    for t in _prompt(w, seed=3, n=5):
        eng.run_token(t, True)
        ref.run_token(t, True)
        lg = eng.read_logits()
        assert rel_err(lg, ref.logits()) <= 1e-3
        pairs = eng.read_buffer(2)
        v = pairs.view(np.float32)[0::2]
        ids = pairs.view(np.uint32)[1::2]
        for c in range(256):
            col = lg[c::256]
            j = int(np.argmax(col))
            assert v[c] == col[j] and ids[c] == c + 256 * j, c


@pytest.mark.parametrize("temperature,top_k,top_p,rp", [(0.0, 0, 1.0, 1.0), (0.8, 40, 1.0, 1.0), (0.0, 0, 1.0, 1.3),
                                                        (0.9, 0, 0.7, 1.2)])
@pytest.mark.parametrize("name", TINY_GRANITE)
def test_granite_generate_matches_oracle(name, synth, temperature, top_k, top_p, rp):
    """generateGraniteWgsl (:223-292) on the device: ids, position (one step past the last id),
    the cached ids and next id match the oracle, greedy, sampled and through the candidate
    path that any penalty other than 1 takes."""
    w, loaded, ref = _pair(synth, name)
    prompt = _prompt(w, seed=1)
    kw = dict(temperature=temperature, top_k=top_k, top_p=top_p, repetition_penalty=rp, seed=9)
    out = generate_granite_wgsl(loaded, prompt, w.decode_tokens, **kw)
    want = ref.generate(prompt, w.decode_tokens, **kw)
    assert out["ids"] == want
    assert loaded.engine.position == ref.position
    assert loaded.cached_token_ids == ref.cached_token_ids
    assert loaded.cached_next_id == ref.cached_next_id


def test_granite_prefix_reuse_keeps_the_ssm_state(synth):
    """Conversation reuse keeps the convolution windows and SSM states; an empty prompt with
    no cached id starts from id 0 and one with a cached id continues."""
    w, loaded, ref = _pair(synth, "tiny-granite")
    p = _prompt(w, seed=4, n=10)
    for turn in range(3):
        g = generate_granite_wgsl(loaded, p, 6, temperature=0.7, seed=5)["ids"]
        r = ref.generate(p, 6, temperature=0.7, seed=5)
        assert g == r, f"turn {turn}"
        assert loaded.engine.position == ref.position
        assert rel_err(loaded.engine.read_logits(), ref.logits()) <= 1e-3
        p = p + g + _prompt(w, seed=10 + turn, n=3)
    reset_granite_wgsl_conversation(loaded)
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    assert generate_granite_wgsl(loaded, [], 5)["ids"] == ref.generate([], 5)


def test_granite_reset_clears_ssm_and_conv_state(synth):
    w, loaded, _ = _pair(synth, "tiny-granite")
    eng = loaded.engine
    prompt = _prompt(w, seed=6, n=9)
    for t in prompt:
        eng.run_token(t, True)
    first = eng.read_logits().copy()
    for t in _prompt(w, seed=7, n=5):
        eng.run_token(t, False)
    eng.reset()
    for t in prompt:
        eng.run_token(t, True)
    assert np.array_equal(eng.read_logits(), first)


def test_granite_loader_tags_and_errors(synth):
    """loadGraniteWgslModel refuses a definition not tagged granite-webgpu (:173-175) and a GGUF
    whose architecture is not granitehybrid (:359-363); the Llama loader refuses a granitehybrid
    file; batched decoding, the prompt pass without allocation and reading K/V of a Mamba2 layer
    are refused; the context is the engine's 4096 positions and its exhaustion keeps the
    reference's wording (:773-775)."""
    w = WORKLOADS["tiny-granite"]
    md = w.model_def(synth("tiny-granite"))
    md.runtime = "llama-webgpu"
    with pytest.raises(ValueError, match="does not support architecture granitehybrid"):
        load_llama_wgsl_model(md)
    with pytest.raises(ValueError, match="loadGraniteWgslModel: unsupported model"):
        load_granite_wgsl_model(md)
    q = WORKLOADS["tiny-qwen3"].model_def(synth("tiny-qwen3"))
    q.runtime = "granite-webgpu"
    with pytest.raises(ValueError, match="expected GGUF architecture granitehybrid, got qwen3"):
        load_granite_wgsl_model(q)
    md.runtime = "granite-webgpu"
    md.max_context = 8192
    loaded = load_granite_wgsl_model(md)
    eng = loaded.engine
    from chonklm_amd.runtime import LlamaWgslBatch
    with pytest.raises(ChonkError, match="granitehybrid"):
        LlamaWgslBatch(eng, 2, 64)
    with pytest.raises(ChonkError, match="no row-batch prompt pass"):
        eng.prefill_noalloc([1, 2, 3])
    with pytest.raises(ChonkError, match="Mamba2 layer"):
        eng.read_kv(0, False, 0)
    eng.prefill([1] * 4096)
    assert eng.position == 4096
    with pytest.raises(ChonkError, match="Granite WGSL context exhausted at 4096 tokens"):
        eng.run_token(1, True)
    dispose_granite_wgsl(loaded)


@pytest.mark.parametrize("name", ["granite-4.0-h-350m-q4_k_m", "granite-4.0-h-350m-q8_0"])
def test_granite_350m_shape_steps_match_oracle(name, synth):
    """The Granite-4.0-H-350M shape (hidden 768, 28 Mamba2 layers of 48 SSM heads x 32 x 128
    states and 4 attention layers of 12 query / 4 kv heads of 64, feed-forward 2048, vocab
    100352 over 256 classes of 392 ids): a 32-token prompt then 8 greedy steps, logits within
    1e-3 and identical ids."""
    w, loaded, ref = _pair(synth, name)
    eng = loaded.engine
    assert eng.info["architecture"] == 6
    prompt = _prompt(w, seed=21, n=32)
    eng.prefill(prompt[:-1])
    for t in prompt[:-1]:
        ref.run_token(t, False)
    tok = prompt[-1]
    for i in range(8):
        a = eng.run_token(tok, True)
        b = ref.run_token(tok, True)
        e = rel_err(eng.read_logits(), ref.logits())
        assert e <= 1e-3, f"step {i}: logits rel err {e:.3e}"
        assert a == b, f"step {i}: token {a} != {b}"
        tok = a
