"""Pins of oracle functions that the float64 decoders do not reach.

* Row decode (``orc_decode_rows``, the block-at-a-time decode inside the
  oracle's matvec) equals the element-wise decode ``orc_dequant`` bit for bit
  (which the known-answer blocks pin) on random and special-scale blocks of
  every type.
* The generate loop's prefix reuse and cachedNextId
  (llama-wgsl-runtime.ts:268-313; gpt-wgsl-runtime.ts:205-249): with the
  penalty at 1 and greedy selection, the loop semantics fix what a second
  call must return, independent of how the oracle implements them:
    - the last generated id never enters the cache (the loop breaks before
      running it), so generate(p1) -> g then generate(p1 + g + x) equals a
      fresh generate(p1 + g[:-1] + x);
    - an empty suffix resumes from cachedNextId, which is g[-1]: the second
      call returns [g[-1]] + what a single longer call generates after g;
    - a prompt that does not extend the conversation resets it.
* The GPT-2 argmax tree (gpt-wgsl-runtime.ts:1882-2004): strict ">" trees
  with the left slot kept on ties give, among equal maxima, the slot whose
  8-bit index is smallest after bit reversal (two slots meet at the stride of
  their lowest differing bit, where the one with a 0 there is on the left);
  NaN in slot 0 is never replaced; padding slots carry index 0.
* The sampler (sampling.ts:23-76) as a distribution: over a uniform grid of
  draws U, the share of draws that picks each candidate equals the
  temperature softmax over the top-k group winners, cut at the top-p prefix,
  to within the grid spacing.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from chonklm_amd import WORKLOADS
from oracle import oracle as orc
from oracle.oracle import OracleModel
from tests.blocks import TYPES, random_blocks


@pytest.mark.parametrize("tname", list(TYPES))
def test_row_decode_equals_element_decode(tname):
    t = TYPES[tname]
    be, _ = orc.BLOCK[t]
    rng = np.random.default_rng(t)
    row_len = 512 if be == 256 else 96
    for special in (False, True):
        raw = random_blocks(t, 7 * row_len, rng, special=special)
        a = orc.dequant(t, raw, 7 * row_len)
        b = orc.decode_rows(t, raw, 7, row_len)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), tname


def _oracle(synth, name, **kw):
    w = WORKLOADS[name]
    return w, OracleModel(synth(name), w.spec.vocab, w.spec.layers, w.max_context, kv_f16=True,
                          eos_ids=kw.get("eos", ()))


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama"])
def test_prefix_reuse_skips_the_last_generated_id(synth, name):
    w, a = _oracle(synth, name)
    _, b = _oracle(synth, name)
    rng = np.random.default_rng(3)
    p1 = rng.integers(0, w.spec.vocab, 9).tolist()
    x = rng.integers(0, w.spec.vocab, 4).tolist()
    g = a.generate(p1, 5)
    assert len(g) == 5 and a.position == len(p1) + len(g) - 1
    h = a.generate(p1 + g + x, 6)
    h_fresh = b.generate(p1 + g[:-1] + x, 6)
    assert h == h_fresh
    assert a.position == b.position == len(p1) + len(g) - 1 + len(x) + len(h) - 1
    assert np.array_equal(a.logits(), b.logits())


@pytest.mark.parametrize("name", ["tiny-qwen3", "tiny-llama"])
def test_empty_suffix_resumes_from_cached_next_id(synth, name):
    w, a = _oracle(synth, name)
    _, b = _oracle(synth, name)
    p1 = np.random.default_rng(4).integers(0, w.spec.vocab, 8).tolist()
    n, m = 5, 6
    g = a.generate(p1, n)
    assert a.cached_next_id == g[-1] and a.cached_token_ids == p1 + g
    h = a.generate(p1 + g, m)
    long = b.generate(p1, n + m - 1)
    assert long[:n] == g
    assert h == [g[-1]] + long[n:]
    assert a.position == b.position


def test_diverging_prompt_resets_the_conversation(synth):
    w, a = _oracle(synth, "tiny-qwen3")
    _, b = _oracle(synth, "tiny-qwen3")
    rng = np.random.default_rng(5)
    p1 = rng.integers(0, w.spec.vocab, 10).tolist()
    q = p1[:4] + rng.integers(0, w.spec.vocab, 5).tolist()
    a.generate(p1, 4)
    assert a.generate(q, 5) == b.generate(q, 5)
    assert a.position == b.position


def test_gpt2_loop_runs_the_last_id_and_resumes(synth):
    """generateGptWgsl also runs the last generated id (:228-245); its result is
    cachedNextId, so an empty suffix continues one token later than the llama loop."""
    w, a = _oracle(synth, "tiny-gpt2")
    _, b = _oracle(synth, "tiny-gpt2")
    p1 = np.random.default_rng(6).integers(0, w.spec.vocab, 7).tolist()
    g = a.generate(p1, 4)
    assert a.position == len(p1) + len(g)
    h = a.generate(p1 + g, 3)
    long = b.generate(p1, 7)
    assert long[:4] == g and h == long[4:]


def _bitrev8(i: int) -> int:
    return int(f"{i & 255:08b}"[::-1], 2)


def test_gpt2_argmax_without_ties_is_argmax():
    rng = np.random.default_rng(7)
    for vocab in (1, 200, 256, 257, 5000, 50257, 65536):
        lg = rng.standard_normal(vocab).astype(np.float32)
        assert orc.argmax_gpt(lg)[0] == int(np.argmax(lg))


def test_gpt2_argmax_ties_follow_the_tree():
    rng = np.random.default_rng(8)
    for _ in range(200):
        vocab = 256
        lg = rng.standard_normal(vocab).astype(np.float32)
        ids = rng.choice(vocab, size=int(rng.integers(2, 6)), replace=False)
        lg[ids] = 9.0
        want = min(ids, key=_bitrev8)
        tok, pairs = orc.argmax_gpt(lg)
        assert tok == want, (sorted(ids), tok, want)
        assert pairs.view(np.uint32)[1] == want
    # across groups: the stage-2 tree over group winners breaks ties the same way
    for _ in range(100):
        groups = int(rng.integers(5, 40))
        lg = rng.standard_normal(groups * 256).astype(np.float32)
        gsel = rng.choice(groups, size=int(rng.integers(2, 5)), replace=False)
        ids = [g * 256 + int(rng.integers(0, 256)) for g in gsel]
        lg[ids] = 9.0
        want = min(ids, key=lambda i: _bitrev8(i // 256))
        assert orc.argmax_gpt(lg)[0] == want
    # the lowest-id rule of the llama runtime differs on such cases
    lg = np.zeros(256, dtype=np.float32)
    lg[[1, 2]] = 1.0
    assert orc.argmax_gpt(lg)[0] == 2 and orc.argmax(lg)[0] == 1


def test_gpt2_argmax_nan_and_padding():
    lg = np.linspace(-1, 1, 300).astype(np.float32)
    lg[0] = np.nan
    tok, pairs = orc.argmax_gpt(lg)
    v = pairs.view(np.float32)[0::2]
    i = pairs.view(np.uint32)[1::2]
    assert math.isnan(v[0]) and i[0] == 0  # NaN in slot 0 is never replaced
    assert tok == 0  # and the NaN group wins stage 2 from slot 0 as well
    lg[0] = -5.0
    lg[100] = np.nan  # a NaN elsewhere never wins
    tok, pairs = orc.argmax_gpt(lg)
    assert tok == 299
    # a group whose real entries all lose to the padding value keeps index 0
    short = np.full(3, -np.inf, dtype=np.float32)
    tok, pairs = orc.argmax_gpt(short)
    assert pairs.view(np.uint32)[1] == 0 and tok == 0


@pytest.mark.parametrize("rp", [0.8, 1.3])
def test_gpt2_argmax_penalty_whenever_not_one(rp):
    rng = np.random.default_rng(9)
    lg = rng.standard_normal(3000).astype(np.float32)
    pen_ids = rng.choice(3000, size=50, replace=False).tolist()
    p = np.float32(math.floor(rp * 1000 + 0.5) / 1000)
    want = lg.copy()
    sel = np.array(pen_ids)
    want[sel] = np.where(want[sel] > 0, want[sel] / p, want[sel] * p)
    assert orc.argmax_gpt(lg, pen_ids, rp)[0] == int(np.argmax(want))
    assert orc.argmax_gpt(lg, pen_ids, 1.0)[0] == int(np.argmax(lg))


def _expected_distribution(vals, ids, temperature, top_k, top_p):
    order = sorted(range(len(vals)), key=lambda j: -vals[j])  # stable, as Array.prototype.sort
    if top_k > 0:
        order = order[:top_k]
    v = np.array([vals[j] for j in order], dtype=np.float64)
    p = np.exp((v - v[0]) / temperature)
    if top_p < 1:
        cdf = np.cumsum(p / p.sum())
        cut = int(np.argmax(cdf >= top_p)) + 1 if np.any(cdf >= top_p) else len(p)
        p = p[:cut]
        order = order[:cut]
    return {ids[j]: float(q) for j, q in zip(order, p / p.sum())}


@pytest.mark.parametrize("temperature,top_k,top_p", [(0.8, 40, 1.0), (1.0, 0, 1.0), (0.5, 10, 0.9), (2.0, 5, 0.5)])
def test_sampler_distribution(temperature, top_k, top_p):
    rng = np.random.default_rng(int(temperature * 100) + top_k)
    groups = 120
    vals = (rng.standard_normal(groups) * 1.5).astype(np.float32)
    ids = (np.arange(groups) * 256 + rng.integers(0, 256, groups)).astype(np.uint32)
    pairs = np.empty(groups * 2, dtype=np.uint32)
    pairs[0::2] = vals.view(np.uint32)
    pairs[1::2] = ids
    want = _expected_distribution(vals.astype(np.float64).tolist(), ids.tolist(), temperature, top_k, top_p)
    N = 20000
    counts: dict[int, int] = {}
    for k in range(N):
        u = (k + 0.5) / N
        t = orc.sample_candidates(pairs.view(np.uint8), temperature, top_p, top_k, 1.0, [], u)
        counts[t] = counts.get(t, 0) + 1
    assert set(counts) <= set(want)
    for tok, q in want.items():
        assert abs(counts.get(tok, 0) / N - q) <= 2.0 / N + 1e-9, (tok, counts.get(tok, 0) / N, q)
