"""GPU engine parity against the oracle on small synthetic decoders.

Each tiny workload exercises a different type mix and architecture branch:
tiny-qwen3 (Q4_K/Q6_K, qk-norm, split RoPE), tiny-qwen3-hd128 (head_dim 128,
150-token prompts: decode attention over several 64-position chunks), tiny-llama (Q5_0/Q8_0/Q4_K
fallbacks, interleaved RoPE, head_dim 32, GQA 3), tiny-llama-q8 (Q8_0
everywhere), tiny-gemma3 (gemma3 sandwich norms, GELU-tanh, sliding window,
Q8_0 tied lm_head, top-k/temperature sampling), tiny-openelm (fused q|k|v in
Q5_K, per-layer head / kv-head / feed-forward counts, GQA groups 2-4). Bars: identical token ids;
logits max|d| / max|ref| <= 1e-3 at every step.
"""
from __future__ import annotations

import numpy as np
import pytest

from chonklm_amd import (WORKLOADS, ChonkError, generate_gpt_wgsl, generate_llama_wgsl, load_gpt_wgsl_model,
                         load_llama_wgsl_model)
from chonklm_amd.runtime import LlamaWgslEngine, reset_llama_wgsl_conversation
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

TINY = ["tiny-qwen3", "tiny-qwen3-hd128", "tiny-llama", "tiny-llama-q8", "tiny-gemma3", "tiny-openelm"]


def _layer_kv_heads(w, layer):
    """K/V heads of one layer (openelm varies them per layer)."""
    return (w.spec.layer_kv_heads or [w.spec.kv_heads] * w.spec.layers)[layer]


def _pair(synth, name, kv="f16", **over):
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path, kv_dtype=kv)
    for k, v in over.items():
        setattr(md, k, v)
    loaded = (load_gpt_wgsl_model if md.runtime == "gpt-webgpu" else load_llama_wgsl_model)(md)
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, md.max_context, kv_f16=(kv == "f16"), eos_ids=w.eos_ids)
    return w, loaded, ref


def _prompt(w, seed=0, n=None):
    rng = np.random.default_rng(seed)
    return rng.integers(0, w.spec.vocab, n or w.prompt_tokens).tolist()


@pytest.mark.parametrize("name", TINY)
def test_step_logits_and_tokens(name, synth):
    w, loaded, ref = _pair(synth, name)
    eng = loaded.engine
    prompt = _prompt(w)
    toks_g, toks_r = [], []
    tok = prompt[0]
    for i in range(len(prompt) + 12):
        need = i >= len(prompt) - 1
        if i < len(prompt):
            tok = prompt[i]
        a = eng.run_token(tok, need)
        b = ref.run_token(tok, need)
        if need:
            lg, lr = eng.read_logits(), ref.logits()
            e = rel_err(lg, lr)
            assert e <= 1e-3, f"{name} step {i}: logits rel err {e:.3e}"
            assert a == b, f"{name} step {i}: token {a} != {b}"
            toks_g.append(a)
            toks_r.append(b)
            tok = a
    assert eng.position == ref.position == len(prompt) + 12


@pytest.mark.parametrize("name", TINY)
def test_generate_matches_oracle(name, synth):
    w, loaded, ref = _pair(synth, name)
    prompt = _prompt(w, seed=1)
    out = generate_llama_wgsl(loaded, prompt, w.decode_tokens, temperature=w.temperature, top_k=w.top_k, seed=9)
    want = ref.generate(prompt, w.decode_tokens, temperature=w.temperature, top_k=w.top_k, seed=9)
    assert out["ids"] == want
    assert loaded.engine.position == ref.position
    assert loaded.cached_token_ids == ref.cached_token_ids
    assert loaded.cached_next_id == ref.cached_next_id


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-gemma3"])
def test_stepped_equals_device_loop(name, synth):
    """The device-driven loop (19 steps: two replays of the eight-step graph, then three
    single steps) gives the ids of the loop stepped from the host (one graph per step)."""
    w, loaded, _ = _pair(synth, name)
    prompt = _prompt(w, seed=2)
    a = generate_llama_wgsl(loaded, prompt, 20, temperature=w.temperature, top_k=w.top_k, seed=3)["ids"]
    reset_llama_wgsl_conversation(loaded)
    seen = []
    b = generate_llama_wgsl(loaded, prompt, 20, temperature=w.temperature, top_k=w.top_k, seed=3,
                            on_token=lambda info: seen.append(info["id"]))["ids"]
    assert a == b == seen


def test_prefix_reuse_matches_oracle(synth):
    w, loaded, ref = _pair(synth, "tiny-qwen3")
    p1 = _prompt(w, seed=4, n=10)
    for turn in range(3):
        g = generate_llama_wgsl(loaded, p1, 6)["ids"]
        r = ref.generate(p1, 6)
        assert g == r, f"turn {turn}"
        assert loaded.engine.position == ref.position
        p1 = p1 + g + _prompt(w, seed=10 + turn, n=3)
    # identical prompt again: cachedNextId path
    same = list(ref.cached_token_ids)
    assert generate_llama_wgsl(loaded, same, 4)["ids"] == ref.generate(same, 4)


def test_repetition_penalty_and_sampling_paths(synth):
    w, loaded, ref = _pair(synth, "tiny-llama")
    eng = loaded.engine
    prompt = _prompt(w, seed=5, n=12)
    for i, t in enumerate(prompt[:-1]):
        eng.run_token(t, False)
        ref.run_token(t, False)
    ids = prompt
    for opts in [dict(repetition_penalty=1.3), dict(temperature=0.7, top_k=5, repetition_penalty=1.2),
                 dict(temperature=1.1, top_p=0.6), dict(top_k=3)]:
        a = eng.run_token(ids[-1], True, penalized_token_ids=ids, seen_ids=ids, seed=21, **opts)
        b = ref.run_token(ids[-1], True, penalized=ids, seen=ids, seed=21, **opts)
        assert a == b, f"{opts}: {a} != {b}"
        assert rel_err(eng.read_logits(), ref.logits()) <= 1e-3
        ids = ids + [a]


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama"])
def test_fp32_kv_cache(name, synth):
    w, loaded, ref = _pair(synth, name, kv="f32")
    prompt = _prompt(w, seed=6)
    out = generate_llama_wgsl(loaded, prompt, 16)
    assert out["ids"] == ref.generate(prompt, 16)
    assert rel_err(loaded.engine.read_logits(), ref.logits()) <= 1e-3


def test_kv_cache_rows_match(synth):
    w, loaded, ref = _pair(synth, "tiny-qwen3")
    eng = loaded.engine
    for t in _prompt(w, seed=7, n=9):
        eng.run_token(t, False)
        ref.run_token(t, False)
    n = w.spec.kv_heads * w.spec.head_dim
    for layer in range(w.spec.layers):
        for pos in (0, 4, 8):
            for is_v in (False, True):
                g = eng.read_kv(layer, is_v, pos)
                r = ref.read_kv(layer, is_v, pos, n)
                # fp16 cache: at most one binary16 ulp apart
                assert np.max(np.abs(g - r)) <= np.max(np.abs(r)) * 2e-3 + 1e-6


def test_long_context_window(synth):
    """Sliding-window layers and long positions via the synthetic K/V fill."""
    w, loaded, ref = _pair(synth, "tiny-gemma3")
    eng = loaded.engine
    pos = 80
    eng.fake_context(pos, seed=3)
    ref.fake_context(pos, seed=3)
    tok = 123
    for _ in range(3):
        a = eng.run_token(tok, True)
        b = ref.run_token(tok, True)
        assert rel_err(eng.read_logits(), ref.logits()) <= 1e-3
        assert a == b
        tok = a


def test_context_exhaustion_and_reset(synth):
    w, loaded, _ = _pair(synth, "tiny-llama-q8", max_context=20)
    eng = loaded.engine
    for i in range(20):
        eng.run_token(i + 3, i == 19)
    with pytest.raises(ChonkError) as ei:
        eng.run_token(5, True)
    assert ei.value.status_name == "ECONTEXT"
    assert "context exhausted at 20 tokens" in str(ei.value)
    eng.reset()
    assert eng.position == 0
    eng.run_token(5, True)
    assert eng.position == 1


def test_bad_token_rejected(synth):
    w, loaded, _ = _pair(synth, "tiny-llama-q8")
    with pytest.raises(ChonkError) as ei:
        loaded.engine.run_token(w.spec.vocab + 5, True)
    assert "outside embedding table" in str(ei.value)
    # the engine stays usable
    loaded.engine.run_token(1, True)


def test_shard_directory_load(synth, tmp_path):
    from chonklm_amd import shard_gguf

    w = WORKLOADS["tiny-qwen3"]
    path = synth("tiny-qwen3")
    shard_dir = shard_gguf(path, str(tmp_path / "shards"), shard_size=65536)
    prompt = _prompt(w, seed=8, n=6)
    out = []
    # one engine at a time: the two then run the same decode attention (only
    # one engine per GPU holds the spin-merging one, whose sums run in another
    # order than the arrival-counter attention's)
    for src in (shard_dir, path):
        eng = LlamaWgslEngine(w.model_def(src))
        ids = [eng.run_token(t, i == len(prompt) - 1) for i, t in enumerate(prompt)]
        out.append((ids[-1], eng.read_logits(), eng.info["spin_attention"]))
        eng.dispose()
    assert out[0][2] == out[1][2]
    assert out[0][0] == out[1][0]
    np.testing.assert_array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("name", TINY)
def test_batched_prefill_matches_token_steps(name, synth):
    """chonk_engine_prefill leaves the K/V rows, position and next-token logits
    of the reference's token-by-token prompt loop (oracle)."""
    w, loaded, ref = _pair(synth, name)
    eng = loaded.engine
    prompt = _prompt(w, seed=12, n=min(40, w.prompt_tokens + 9))
    eng.prefill(prompt[:-1])
    for t in prompt[:-1]:
        ref.run_token(t, False)
    assert eng.position == ref.position == len(prompt) - 1
    for layer in range(w.spec.layers):
        n = _layer_kv_heads(w, layer) * eng.info["head_dim"]
        for pos in (0, len(prompt) // 2, len(prompt) - 2):
            for is_v in (False, True):
                g = eng.read_kv(layer, is_v, pos)[:n]
                r = ref.read_kv(layer, is_v, pos, n)
                assert np.max(np.abs(g - r)) <= np.max(np.abs(r)) * 2e-3 + 1e-6, f"layer {layer} pos {pos} v={is_v}"
    a = eng.run_token(prompt[-1], True)
    b = ref.run_token(prompt[-1], True)
    assert rel_err(eng.read_logits(), ref.logits()) <= 1e-3
    assert a == b


def test_batched_prefill_in_chunks_and_after_context(synth):
    """A prompt longer than one 2048-row pass, appended after earlier tokens."""
    w, loaded, ref = _pair(synth, "tiny-llama-q8", max_context=2200)
    eng = loaded.engine
    head = _prompt(w, seed=13, n=5)
    for t in head:
        eng.run_token(t, False)
        ref.run_token(t, False)
    body = _prompt(w, seed=14, n=2100)
    eng.prefill(body)
    for t in body:
        ref.run_token(t, False)
    a = eng.run_token(7, True)
    b = ref.run_token(7, True)
    assert rel_err(eng.read_logits(), ref.logits()) <= 1e-3
    assert a == b


def test_gpt2_step_logits_and_tokens(synth):
    """The GPT-2 runtime (gpt-wgsl-runtime.ts:749-840) on the device: LayerNorm prologues,
    fused q|k|v with bias, attention without rotary, bias + clamped residual epilogues,
    GELU-tanh MLP, its argmax tree; token ids identical and logits within 1e-3."""
    w, loaded, ref = _pair(synth, "tiny-gpt2")
    eng = loaded.engine
    assert eng.info["vocab"] == ref.vocab
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
            assert e <= 1e-3, f"step {i}: logits rel err {e:.3e}"
            assert a == b, f"step {i}: token {a} != {b}"
            tok = a
    assert eng.position == ref.position == len(prompt) + 12


@pytest.mark.parametrize("temperature,top_k,rp", [(0.0, 0, 1.0), (0.8, 40, 1.0), (0.0, 0, 1.3), (0.0, 0, 0.8),
                                                  (0.8, 40, 0.8)])
def test_gpt2_generate_matches_oracle(synth, temperature, top_k, rp):
    """generateGptWgsl (:182-249): ids, position (one step past the last id) and the cached
    next id match the oracle, greedy, sampled and with a repetition penalty; a penalty below
    1 applies in ARGMAX_STAGE1 too (the GPT runtime penalizes whenever it is not 1, :789-798)."""
    w, loaded, ref = _pair(synth, "tiny-gpt2")
    prompt = _prompt(w, seed=3)
    out = generate_gpt_wgsl(loaded, prompt, w.decode_tokens, temperature=temperature, top_k=top_k,
                            repetition_penalty=rp, seed=5)
    want = ref.generate(prompt, w.decode_tokens, temperature=temperature, top_k=top_k, repetition_penalty=rp, seed=5)
    assert out["ids"] == want
    assert loaded.engine.position == ref.position
    assert loaded.cached_next_id == ref.cached_next_id


def test_gpt2_ignores_definition_default_penalty(synth):
    """generateGptWgsl takes opts.repetitionPenalty ?? 1 (gpt-wgsl-runtime.ts:198-203): a
    definition's defaultRepetitionPenalty is not applied, unlike generateLlamaWgsl's."""
    w, loaded, ref = _pair(synth, "tiny-gpt2", default_repetition_penalty=1.6)
    prompt = _prompt(w, seed=6)
    assert generate_gpt_wgsl(loaded, prompt, 12)["ids"] == ref.generate(prompt, 12, repetition_penalty=1.0)


def test_gpt2_loader_tags(synth):
    """loadGptWgslModel refuses a definition not tagged gpt-webgpu; the Llama loader refuses a
    gpt2 file (gpt-wgsl-runtime.ts:135-137, llama-wgsl-runtime.ts architecture check)."""
    w = WORKLOADS["tiny-gpt2"]
    md = w.model_def(synth("tiny-gpt2"))
    loaded = load_gpt_wgsl_model(md)
    assert loaded.runtime == "gpt-webgpu" and loaded.engine.info["architecture"] == 3
    dispose_gpt = __import__("chonklm_amd").dispose_gpt_wgsl
    dispose_gpt(loaded)
    md.runtime = "llama-webgpu"
    with pytest.raises(ValueError, match="does not support architecture gpt2"):
        load_llama_wgsl_model(md)
    q = WORKLOADS["tiny-qwen3"].model_def(synth("tiny-qwen3"))
    with pytest.raises(ValueError, match="loadGptWgslModel: unsupported model"):
        load_gpt_wgsl_model(q)


def test_gpt2_errors_and_empty_prompt(synth):
    """GPT errors keep the reference's wording (gpt-wgsl-runtime.ts:218, :752); an empty
    suffix after a finished run continues from the cached next id, as the oracle does."""
    w, loaded, ref = _pair(synth, "tiny-gpt2")
    with pytest.raises(ChonkError, match="GPT WGSL has no cached next token for an empty prompt"):
        generate_gpt_wgsl(loaded, [], 4)
    prompt = _prompt(w, seed=11, n=10)
    a = generate_gpt_wgsl(loaded, prompt, 5)["ids"]
    b = ref.generate(prompt, 5)
    assert a == b
    # the same prompt + ids again: empty suffix, continue from cachedNextId
    a2 = generate_gpt_wgsl(loaded, prompt + a, 4)["ids"]
    b2 = ref.generate(prompt + b, 4)
    assert a2 == b2 and loaded.cached_next_id == ref.cached_next_id
    eng = loaded.engine
    eng.reset()
    for t in range(w.max_context):
        eng.run_token(t % w.spec.vocab, False)
    with pytest.raises(ChonkError, match=f"GPT WGSL context exhausted at {w.max_context} tokens"):
        eng.run_token(1, True)


def test_gpt2_wide_ffn_matches_oracle(tmp_path):
    """A gpt2 file with a feed-forward width above 4096 (GPT-2 large has 5120): ffn_down
    runs on the LDS-staged row kernel; logits and ids match the oracle at every step."""
    import dataclasses

    from chonklm_amd import write_synthetic_gguf

    base = WORKLOADS["tiny-gpt2"]
    w = dataclasses.replace(base, name="tiny-gpt2-wide", spec=dataclasses.replace(base.spec, ffn=5120, layers=2))
    path = str(tmp_path / "wide.gguf")
    write_synthetic_gguf(w, path)
    loaded = load_gpt_wgsl_model(w.model_def(path))
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True, eos_ids=w.eos_ids)
    eng = loaded.engine
    tok = 5
    for i in range(10):
        a = eng.run_token(tok, True)
        b = ref.run_token(tok, True)
        e = rel_err(eng.read_logits(), ref.logits())
        assert e <= 1e-3, f"step {i}: logits rel err {e:.3e}"
        assert a == b, f"step {i}: token {a} != {b}"
        tok = a


def test_openelm_270m_shape_steps_match_oracle(synth):
    """The OpenELM-270M shape: per-layer GQA of 12/16/20 query heads over 3/4/5 kv heads, a
    Q5_K fused q|k|v, feed-forward widths 768..5120 (ffn_down rows above 4096 take the generic
    matvec; the prompt runs through the batched pass): prompt then 8 greedy steps, logits
    within 1e-3 and identical ids."""
    w, loaded, ref = _pair(synth, "openelm-270m-q4_k_m")
    eng = loaded.engine
    assert eng.info["architecture"] == 4
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
