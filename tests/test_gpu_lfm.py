"""The LFM2 runtime (src/lib/lfm-wgsl-runtime.ts) on the device against the oracle.

The engine runs a convolution layer as two launches: in_proj with the operator
RMSNorm in its prologue, and out_proj whose prologue is CONV_BLOCK_WGSL over
this token's B | C | x and the layer's two-value state and whose epilogue adds
the residual; the gate|up launch then shifts the state. Attention layers take
the qk-norm / split-RoPE attention kernel. The lm_head reads the embedding
stored class-major, so that each workgroup's argmax candidate is
TOPK256_WGSL's slot. Workloads: tiny-lfm2 (Q4_K / Q6_K, convolution and
attention layers alternating, GQA 2, head_dim 64, vocab 1024), tiny-lfm2-q8
(Q8_0 everywhere, two convolution layers then attention, head_dim 32, GQA 3,
vocab 700 so the last classes hold two ids), and the LFM2.5-350M shape in
Q4_K_M and Q8_0. Bars: identical token ids; logits max|d| / max|ref| <= 1e-3.
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import (WORKLOADS, ChonkError, dispose_lfm_wgsl, generate_lfm_wgsl, load_llama_wgsl_model,
                         load_lfm_wgsl_model, reset_lfm_wgsl_conversation)
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TINY_LFM = ["tiny-lfm2", "tiny-lfm2-q8"]


def _pair(synth, name, kv="f16", **over):
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path, kv_dtype=kv)
    for k, v in over.items():
        setattr(md, k, v)
    loaded = load_lfm_wgsl_model(md)
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, md.max_context, kv_f16=(kv == "f16"), eos_ids=w.eos_ids)
    return w, loaded, ref


def _prompt(w, seed=0, n=None):
    return np.random.default_rng(seed).integers(0, w.spec.vocab, n or w.prompt_tokens).tolist()


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("name", TINY_LFM)
def test_lfm_step_logits_and_tokens(name, kv, synth):
    w, loaded, ref = _pair(synth, name, kv=kv)
    eng = loaded.engine
    assert eng.info["architecture"] == 5
    prompt = _prompt(w)
    tok = prompt[0]
    for i in range(len(prompt) + 12):
        need = i >= len(prompt) - 1
        if i < len(prompt):
            tok = prompt[i]
        a = eng.run_token(tok, need)
        b = ref.run_token(tok, need)
        if need:
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"{name} step {i}: logits rel err {e:.3e}"
            assert a == b, f"{name} step {i}: token {a} != {b}"
            tok = a
    assert eng.position == ref.position == len(prompt) + 12


def test_lfm_candidates_are_class_maxima(synth):
    """The lm_head epilogue's 256 candidates equal TOPK256_WGSL's slots of the device's
    own logits (slot t: the first maximum of ids t, t + 256, ...)."""
    w, loaded, ref = _pair(synth, "tiny-lfm2-q8")
    eng = loaded.engine
    for t in _prompt(w, seed=3, n=5):
        eng.run_token(t, True)
        lg = eng.read_logits()
        pairs = eng.read_buffer(2)
        v = pairs.view(np.float32)[0::2]
        ids = pairs.view(np.uint32)[1::2]
        for c in range(256):
            col = lg[c::256]
            j = int(np.argmax(col))
            assert v[c] == col[j] and ids[c] == c + 256 * j, c


@pytest.mark.parametrize("temperature,top_k,top_p,rp", [(0.0, 0, 1.0, 1.0), (0.8, 40, 1.0, 1.0), (0.0, 0, 1.0, 1.3),
                                                        (0.0, 0, 1.0, 0.8), (0.9, 0, 0.7, 1.2)])
@pytest.mark.parametrize("name", TINY_LFM)
def test_lfm_generate_matches_oracle(name, synth, temperature, top_k, top_p, rp):
    """generateLfmWgsl (:219-306) on the device: ids, position (one step past the last id),
    the cached ids and next id match the oracle, greedy, sampled and through the candidate
    path that any penalty other than 1 takes."""
    w, loaded, ref = _pair(synth, name)
    prompt = _prompt(w, seed=1)
    kw = dict(temperature=temperature, top_k=top_k, top_p=top_p, repetition_penalty=rp, seed=9)
    out = generate_lfm_wgsl(loaded, prompt, w.decode_tokens, **kw)
    want = ref.generate(prompt, w.decode_tokens, **kw)
    assert out["ids"] == want
    assert loaded.engine.position == ref.position
    assert loaded.cached_token_ids == ref.cached_token_ids
    assert loaded.cached_next_id == ref.cached_next_id


def test_lfm_stepped_equals_device_loop(synth):
    w, loaded, _ = _pair(synth, "tiny-lfm2")
    prompt = _prompt(w, seed=2)
    a = generate_lfm_wgsl(loaded, prompt, 20, temperature=0.8, top_k=40, seed=3)["ids"]
    nxt = loaded.cached_next_id
    reset_lfm_wgsl_conversation(loaded)
    seen = []
    b = generate_lfm_wgsl(loaded, prompt, 20, temperature=0.8, top_k=40, seed=3,
                          on_token=lambda info: seen.append(info["id"]))["ids"]
    assert a == b == seen
    assert loaded.cached_next_id == nxt


def test_lfm_prefix_reuse_and_empty_prompt(synth):
    """Conversation reuse keeps the convolution states; an empty prompt with no cached id
    starts from id 0 (the reference's nextId default) and one with a cached id continues."""
    w, loaded, ref = _pair(synth, "tiny-lfm2")
    p = _prompt(w, seed=4, n=10)
    for turn in range(3):
        g = generate_lfm_wgsl(loaded, p, 6)["ids"]
        r = ref.generate(p, 6)
        assert g == r, f"turn {turn}"
        assert loaded.engine.position == ref.position
        p = p + g + _prompt(w, seed=10 + turn, n=3)
    same = list(ref.cached_token_ids)
    assert generate_lfm_wgsl(loaded, same, 4)["ids"] == ref.generate(same, 4)
    reset_lfm_wgsl_conversation(loaded)
    ref.reset()
    ref.cached_token_ids, ref.cached_next_id = [], None
    assert generate_lfm_wgsl(loaded, [], 5)["ids"] == ref.generate([], 5)


def test_lfm_reset_clears_convolution_state(synth):
    w, loaded, ref = _pair(synth, "tiny-lfm2")
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


def test_lfm_loader_tags_and_errors(synth):
    """loadLfmWgslModel refuses a definition not tagged lfm2-webgpu (:173-175) and a GGUF whose
    architecture is not lfm2 (:320-322); the Llama loader refuses an lfm2 file; batched decoding,
    the row-batch prompt pass without allocation and reading K/V of a convolution layer are refused;
    context exhaustion keeps the reference's wording (:732-734)."""
    w = WORKLOADS["tiny-lfm2"]
    md = w.model_def(synth("tiny-lfm2"))
    md.runtime = "llama-webgpu"
    with pytest.raises(ValueError, match="does not support architecture lfm2"):
        load_llama_wgsl_model(md)
    with pytest.raises(ValueError, match="loadLfmWgslModel: unsupported model"):
        load_lfm_wgsl_model(md)
    q = WORKLOADS["tiny-qwen3"].model_def(synth("tiny-qwen3"))
    q.runtime = "lfm2-webgpu"
    with pytest.raises(ValueError, match="unsupported LFM GGUF architecture: qwen3"):
        load_lfm_wgsl_model(q)
    md.runtime = "lfm2-webgpu"
    loaded = load_lfm_wgsl_model(md)
    eng = loaded.engine
    from chonklm_amd.runtime import LlamaWgslBatch
    with pytest.raises(ChonkError, match="not lfm2"):
        LlamaWgslBatch(eng, 2, 64)
    with pytest.raises(ChonkError, match="no row-batch prompt pass"):
        eng.prefill_noalloc([1, 2, 3])
    with pytest.raises(ChonkError, match="convolution layer"):
        eng.read_kv(0, False, 0)
    eng.prefill(list(range(w.max_context)))
    with pytest.raises(ChonkError, match=f"LFM WGSL context exhausted at {w.max_context} tokens"):
        eng.run_token(1, True)
    dispose_lfm_wgsl(loaded)


@pytest.mark.parametrize("name", ["lfm2.5-350m-q4_k_m", "lfm2.5-350m-q8_0"])
def test_lfm2_350m_shape_steps_match_oracle(name, synth):
    """The LFM2.5-350M shape (hidden 1024, 10 convolution and 6 attention layers, 16 query / 8
    kv heads of 64, feed-forward 4608, vocab 65536 over 256 classes of 256 ids): prompt then 8
    greedy steps, logits within 1e-3 and identical ids."""
    w, loaded, ref = _pair(synth, name)
    eng = loaded.engine
    assert eng.info["architecture"] == 5
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
