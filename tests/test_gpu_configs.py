"""GPU parity at the benchmark configurations' real shapes.

* 128-step generation from each configuration's seeded prompt (SmolLM2-135M
  Q4_K_M and Q8_0 with 32 tokens, Qwen3-0.6B Q4_K_M with 2048, Gemma-3-270M
  Q4_K_M with 1024 and top-k 40 / T 0.8 seeded sampling): the GPU's ids equal
  the oracle's, stored in tests/golden/config_golden.json by
  tests/golden/make_config_golden.py (the oracle runs the reference's
  token-by-token loop, llama-wgsl-runtime.ts:242-314, in the build
  container; the fixture is keyed by the GGUF file's SHA-256).
* Sixteen decode steps at the configurations' contexts against the oracle run
  live, with this build's fp16 K/V cache and with the reference's fp32 cache
  (llama-wgsl-runtime.ts:830-831) on both sides: logits within 1e-3 (max |d| / max |ref|) and identical ids. The K/V cache
  holds the same synthetic positions on both sides (SmolLM2: the real prompt),
  so these steps run the kernels at their configuration geometry: decode
  attention with interleaved rotary over a 3-group GQA (SmolLM2), 33 chunks
  of 64 positions and their merge (Qwen3 at position 2048), head_dim 256 with
  a 4-head group and 512-position windows (Gemma-3), the row matvecs at
  K = 576 / 640 / 1024 / 1536 / 2048 / 3072, and the lm_head's group argmax
  over 192, 594 and 1024 groups.
* Batched decoding at 64 sequences x 512-token prompts, 128 greedy steps:
  every row follows the batch-1 engine on the same prompt (ids up to the
  first near-tie of the batch-1 logits, logits at the end); four of the 64
  rows against the oracle at three positions; two rows at a short prompt
  against the oracle.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from chonklm_amd import WORKLOADS, generate_llama_wgsl, load_llama_wgsl_model
from chonklm_amd.runtime import LlamaWgslBatch
from oracle.oracle import OracleModel
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "config_golden.json").read_text())
CONFIGS = ["smollm2-135m-q4_k_m", "smollm2-135m-q8_0", "qwen3-0.6b-q4_k_m", "gemma3-270m-q4_k_m"]
STEPS = 128


def _sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 22), b""):
            h.update(block)
    return h.hexdigest()


def _fixture(name: str, path: str) -> dict:
    g = GOLDEN[name]
    if _sha256(path) != g["sha256"]:
        pytest.fail(f"{name}: synthetic GGUF writer output changed; rerun tests/golden/make_config_golden.py")
    w = WORKLOADS[name]
    prompt = w.prompt(g["prompt_seed"])
    digest = hashlib.sha256(",".join(map(str, prompt)).encode()).hexdigest()[:16]
    assert digest == g["prompt_digest"], "prompt generator changed"
    return g


@pytest.mark.parametrize("name", CONFIGS)
def test_config_generate_matches_golden(synth, name):
    w = WORKLOADS[name]
    path = synth(name)
    g = _fixture(name, path)
    md = w.model_def(path)
    md.max_context = w.prompt_tokens + STEPS + 8
    loaded = load_llama_wgsl_model(md)
    out = generate_llama_wgsl(loaded, w.prompt(g["prompt_seed"]), STEPS, temperature=g["temperature"],
                              top_k=g["top_k"], top_p=g["top_p"], seed=g["seed"])
    ids, want = out["ids"], g["ids"]
    if ids != want:
        j = next((i for i, (a, b) in enumerate(zip(ids, want)) if a != b), min(len(ids), len(want)))
        m = g["margins"][j] if j < len(g["margins"]) else float("nan")
        pytest.fail(f"{name}: ids differ first at step {j} ({ids[j:j + 3]} vs {want[j:j + 3]}; "
                    f"oracle top-2 margin there {m:.3e}); lengths {len(ids)} / {len(want)}")
    assert loaded.cached_token_ids == w.prompt(g["prompt_seed"]) + want
    loaded.engine.dispose()


@pytest.mark.parametrize("kv", ["f16", "f32"])
@pytest.mark.parametrize("name", CONFIGS)
def test_config_steps_match_oracle(synth, name, kv):
    w = WORKLOADS[name]
    path = synth(name)
    ctx = w.prompt_tokens + 24
    md = w.model_def(path, kv_dtype=kv)
    md.max_context = ctx
    loaded = load_llama_wgsl_model(md)
    eng = loaded.engine
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=kv == "f16", threads=16)
    prompt = w.prompt(1234)
    samp = dict(temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, seed=9)
    if w.prompt_tokens <= 64:
        # the real prompt on both sides (batched prompt pass on the GPU)
        eng.prefill(prompt[:-1])
        for t in prompt[:-1]:
            ref.run_token(t, False)
        tok = prompt[-1]
    else:
        eng.fake_context(w.prompt_tokens, seed=3)
        ref.fake_context(w.prompt_tokens, seed=3)
        tok = prompt[-1]
    hist = list(prompt)
    for i in range(16):
        a = eng.run_token(tok, True, penalized_token_ids=hist, seen_ids=hist, **samp)
        b = ref.run_token(tok, True, penalized=hist, seen=hist, **samp)
        e = rel_err(eng.read_logits(), ref.logits())
        assert e <= 1e-3, f"{name} ({kv} K/V) step {i} at position {eng.position - 1}: logits rel err {e:.3e}"
        assert a == b, f"{name} ({kv} K/V) step {i}: token {a} != {b}"
        tok = a
        hist.append(a)
    assert eng.position == ref.position
    eng.dispose()
    ref.close()


def _margin(lg: np.ndarray) -> float:
    top2 = np.partition(lg, -2)[-2:]
    return float(abs(top2[1] - top2[0]))


def test_batched_64x512_follows_batch1(synth):
    """Config 5: 64 sequences x 512-token prompts, 128 greedy steps over all rows at once.
    Each row must produce the batch-1 engine's ids for the same prompt (both are checked
    against the oracle elsewhere; they differ in arithmetic only: MFMA GEMM rows vs
    integer-digit matvecs), compared up to the first step where the batch-1 top-2 margin is
    within 1e-4 of the largest logit (a near-tie either may resolve), and logits within 1e-3
    at the last compared step."""
    name = "qwen3-0.6b-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    seqs, plen = 64, 512
    md = w.model_def(path)
    md.max_context = plen + STEPS + 8
    loaded = load_llama_wgsl_model(md)
    eng = loaded.engine
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, w.spec.vocab, plen).tolist() for _ in range(seqs)]
    b = LlamaWgslBatch(eng, seqs, plen + STEPS + 2)
    cur = [b.prefill(s, prompts[s]) for s in range(seqs)]
    ids = [[c] for c in cur]
    rows = list(range(seqs))
    last_logits = {}
    for step in range(STEPS - 1):
        cur = b.step(rows, cur)
        for s in rows:
            ids[s].append(cur[s])
    for s in (0, 31, 63):
        last_logits[s] = b.read_logits(s)
    b.close()

    full = 0
    for s in range(seqs):
        eng.reset()
        eng.prefill(prompts[s][:-1])
        tok = eng.run_token(prompts[s][-1], True)
        ref_ids = [tok]
        lg = eng.read_logits()
        margins = [_margin(lg)]
        scale = float(np.max(np.abs(lg)))
        for _ in range(STEPS - 1):
            tok = eng.run_token(tok, True)
            ref_ids.append(tok)
            lg = eng.read_logits()
            margins.append(_margin(lg))
        tie = next((i for i, m in enumerate(margins) if m <= 1e-4 * scale), STEPS)
        assert ids[s][:tie] == ref_ids[:tie], f"row {s}: ids differ before the first near-tie (step {tie})"
        if tie == STEPS:
            full += 1
            if s in last_logits:
                e = rel_err(last_logits[s], lg)
                assert e <= 1e-3, f"row {s}: last-step logits rel err {e:.3e}"
    assert full >= seqs // 2, f"only {full} of {seqs} rows compared over all {STEPS} steps"
    eng.dispose()


def test_batched_64x512_rows_match_oracle(synth):
    """Config 5 at its full size against the oracle: 64 sequences x 512-token prompts,
    the batched prompt pass and three greedy steps over all 64 rows at once; rows 0,
    21, 42 and 63 (each with its own page set) are run token by token by four oracle
    models over the same prompts, and at the prompt's end and the next two positions
    the row's logits are within 1e-3 of the oracle's and its ids are the oracle's."""
    name = "qwen3-0.6b-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    seqs, plen, steps = 64, 512, 3
    md = w.model_def(path)
    md.max_context = plen + 16
    loaded = load_llama_wgsl_model(md)
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, w.spec.vocab, plen).tolist() for _ in range(seqs)]
    b = LlamaWgslBatch(loaded.engine, seqs, plen + 16)
    check = (0, 21, 42, 63)
    cur, got_logits = [], {}
    for s in range(seqs):
        cur.append(b.prefill(s, prompts[s]))
        if s in check:
            got_logits[s] = [b.read_logits(0)]  # (a prefill's logits are its batch's row 0)
    got_ids = {s: [cur[s]] for s in check}
    rows = list(range(seqs))
    for _ in range(steps - 1):
        cur = b.step(rows, cur)
        for s in check:
            got_logits[s].append(b.read_logits(s))
            got_ids[s].append(cur[s])
    b.close()
    loaded.engine.dispose()
    for s in check:
        ref = OracleModel(path, w.spec.vocab, w.spec.layers, plen + 16, kv_f16=True, threads=16)
        for t in prompts[s][:-1]:
            ref.run_token(t, False)
        tok = prompts[s][-1]
        for i in range(steps):
            want = ref.run_token(tok, True)
            e = rel_err(got_logits[s][i], ref.logits())
            assert e <= 1e-3, f"row {s} position {plen - 1 + i}: logits rel err {e:.3e}"
            assert got_ids[s][i] == want, f"row {s} position {plen - 1 + i}: id {got_ids[s][i]} != {want}"
            tok = want
        ref.close()


def test_batched_rows_match_oracle_at_config_shape(synth):
    """Two batch rows of the Qwen3-0.6B shape with short prompts, stepped together, against
    two oracle runs: logits within 1e-3 and identical ids at every step."""
    name = "qwen3-0.6b-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path)
    md.max_context = 64
    loaded = load_llama_wgsl_model(md)
    b = LlamaWgslBatch(loaded.engine, 2, 40)
    prompts = [w.prompt(11, 12), w.prompt(12, 9)]
    refs = [OracleModel(path, w.spec.vocab, w.spec.layers, 64, kv_f16=True, threads=16) for _ in prompts]
    cur = []
    for s, p in enumerate(prompts):
        got = b.prefill(s, p)
        for t in p[:-1]:
            refs[s].run_token(t, False)
        want = refs[s].run_token(p[-1], True)
        assert got == want
        assert rel_err(b.read_logits(0), refs[s].logits()) <= 1e-3
        cur.append(got)
    for step in range(6):
        nxt = b.step([0, 1], cur)
        for s in (0, 1):
            want = refs[s].run_token(cur[s], True)
            e = rel_err(b.read_logits(s), refs[s].logits())
            assert e <= 1e-3, f"row {s} step {step}: logits rel err {e:.3e}"
            assert nxt[s] == want, f"row {s} step {step}"
        cur = nxt
    b.close()
    loaded.engine.dispose()


def test_decode_attention_across_chunk_counts(synth):
    """The Qwen3-0.6B shape with the benchmark's 2304-position cache (36 chunks of 64) stepped
    at positions that give every kind of merge: one chunk, a full last chunk, a newest chunk
    holding only the new position, and 30-36 active chunks, where the output dims divide
    unevenly over the chunks and some chunks merge no dims. The newest chunk advances the kv
    head's epoch only after it has seen every chunk's row; a launch that waited on a stale
    epoch would report error 4 here. Logits within 1e-3 of the oracle, identical ids."""
    name = "qwen3-0.6b-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    ctx = 2304
    md = w.model_def(path)
    md.max_context = ctx
    loaded = load_llama_wgsl_model(md)
    eng = loaded.engine
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=16)
    tok = 17
    for pos in (1, 63, 64, 127, 700, 1900, 1919, 1920, 2047, 2048, 2111, 2112, 2240, 2302):
        eng.fake_context(pos, seed=pos)
        ref.fake_context(pos, seed=pos)
        for i in range(2):
            a = eng.run_token(tok, True)
            b = ref.run_token(tok, True)
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"position {pos + i}: logits rel err {e:.3e}"
            assert a == b, f"position {pos + i}: token {a} != {b}"
            tok = a
    eng.dispose()
    ref.close()


def test_batched_walk_with_interleaved_rope_matches_oracle(synth):
    """The SmolLM2-135M shape (3 kv heads of 64, a 3-head group, interleaved RoPE, no q/k norm)
    in a 200-sequence batch: 200 rows x 3 kv heads cover the device, so one workgroup walks
    each (row, kv head)'s pages and also does its rotary and K/V write from the projections'
    partial sums, and writes the o-projection's operand planes. Two rows against two oracle
    runs: logits within 1e-3 and identical ids at every step."""
    name = "smollm2-135m-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    md = w.model_def(path)
    md.max_context = 64
    loaded = load_llama_wgsl_model(md)
    n = 200
    b = LlamaWgslBatch(loaded.engine, n, 40)
    rng = np.random.default_rng(17)
    prompts = [rng.integers(0, w.spec.vocab, 6 + (s % 7)).tolist() for s in range(n)]
    check = [0, n - 1]
    refs = {s: OracleModel(path, w.spec.vocab, w.spec.layers, 64, kv_f16=True, threads=16) for s in check}
    cur = []
    for s, p in enumerate(prompts):
        got = b.prefill(s, p)
        if s in refs:
            for t in p[:-1]:
                refs[s].run_token(t, False)
            assert got == refs[s].run_token(p[-1], True)
        cur.append(got)
    rows = list(range(n))
    for step in range(4):
        nxt = b.step(rows, cur)
        for s in check:
            want = refs[s].run_token(cur[s], True)
            e = rel_err(b.read_logits(s), refs[s].logits())
            assert e <= 1e-3, f"row {s} step {step}: logits rel err {e:.3e}"
            assert nxt[s] == want, f"row {s} step {step}"
        cur = nxt
    b.close()
    loaded.engine.dispose()


def test_decode_attention_walks_sub_chunks_at_long_context(synth):
    """The Qwen3-0.6B shape with a 9000-position cache: 141 chunks of 64 positions are more
    than one workgroup per chunk can merge, so each workgroup walks two 64-position sub-chunks
    with an online softmax (running maximum and sum, accumulators rescaled). Positions where a
    workgroup's second sub-chunk is empty, partial and full, and where the newest workgroup
    holds only the new position; logits within 1e-3 of the oracle and identical ids."""
    name = "qwen3-0.6b-q4_k_m"
    w = WORKLOADS[name]
    path = synth(name)
    ctx = 9000
    md = w.model_def(path)
    md.max_context = ctx
    loaded = load_llama_wgsl_model(md)
    eng = loaded.engine
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=16)
    tok = 23
    for pos in (100, 8000, 8063, 8064, 8191, 8960, 8998):
        eng.fake_context(pos, seed=pos)
        ref.fake_context(pos, seed=pos)
        for i in range(2 if pos + 2 <= ctx else 1):
            a = eng.run_token(tok, True)
            b = ref.run_token(tok, True)
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"position {pos + i}: logits rel err {e:.3e}"
            assert a == b, f"position {pos + i}: token {a} != {b}"
            tok = a
    eng.dispose()
    ref.close()


@pytest.mark.parametrize("name", ["tiny-gemma3-hd256", "tiny-gemma3-hd64"])
def test_decode_attention_windows_past_8192_positions(synth, name):
    """Sliding windows of 512 positions (5 of 6 layers) on a 9000-position cache, where each
    attention workgroup walks two 64-position sub-chunks: head_dim 256 with a 4-head group
    (Gemma-3's geometry) and head_dim 64. Positions whose window starts in the middle of a
    workgroup's first sub-chunk (8211: start 7700), of its second (8300: start 7789), on a
    workgroup boundary (8959: start 8448), near the cache's end, and a short position;
    logits within 1e-3 of the oracle and identical ids."""
    w = WORKLOADS[name]
    path = synth(name)
    ctx = 9000
    md = w.model_def(path)
    md.max_context = ctx
    loaded = load_llama_wgsl_model(md)
    eng = loaded.engine
    assert eng.info["spin_attention"] == 1 or eng.info["kv_dtype"] != 0
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=16)
    tok = 29
    for pos in (100, 8211, 8300, 8959, 8997):
        eng.fake_context(pos, seed=pos)
        ref.fake_context(pos, seed=pos)
        for i in range(2):
            a = eng.run_token(tok, True)
            b = ref.run_token(tok, True)
            e = rel_err(eng.read_logits(), ref.logits())
            assert e <= 1e-3, f"{name} position {pos + i}: logits rel err {e:.3e}"
            assert a == b, f"{name} position {pos + i}: token {a} != {b}"
            tok = a
    eng.dispose()
    ref.close()
