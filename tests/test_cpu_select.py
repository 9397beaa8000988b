"""Token selection in the oracle: argmax stage 1/2 and the candidate sampler.

Argmax (llama-wgsl-runtime.ts:3645-3791): ties go to the lowest id, NaN never
wins, and the repetition penalty divides positive / multiplies negative
logits by round(p * 1000) / 1000. The sampler is checked against a
line-by-line Python reading of sampleFromCandidateBuffer
(src/lib/sampling.ts:23-76) with the uniform draw given explicitly.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import oracle as orc


def pairs_of(buf: np.ndarray):
    v = buf.view(np.float32)[0::2]
    i = buf.view(np.uint32)[1::2]
    return v, i


def test_argmax_is_first_maximum():
    rng = np.random.default_rng(0)
    for vocab in (1, 255, 256, 257, 1000, 49152, 151936):
        lg = rng.standard_normal(vocab).astype(np.float32)
        tok, _ = orc.argmax(lg)
        assert tok == int(np.argmax(lg))


def test_argmax_ties_go_to_lowest_id():
    lg = np.zeros(5000, dtype=np.float32)
    for ids in ([4999, 17, 300], [3000, 2999], [256, 255]):
        x = lg.copy()
        x[ids] = 7.0
        assert orc.argmax(x)[0] == min(ids)


def test_argmax_nan_never_wins():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal(3000).astype(np.float32)
    best = int(np.argmax(lg))
    lg[[0, 5, best + 1 if best + 1 < lg.size else 0]] = np.nan
    assert orc.argmax(lg)[0] == best
    lg2 = np.full(600, np.nan, dtype=np.float32)
    lg2[333] = -1e30
    assert orc.argmax(lg2)[0] == 333


def test_group_candidates_are_group_maxima():
    rng = np.random.default_rng(2)
    lg = rng.standard_normal(1000).astype(np.float32)
    lg[512:768] = 3.0  # a tied group: lowest id wins
    _, buf = orc.argmax(lg)
    v, i = pairs_of(buf)
    for g in range(4):
        seg = lg[256 * g:256 * (g + 1)]
        assert i[g] == 256 * g + int(np.argmax(seg))
        assert v[g] == seg.max()


@pytest.mark.parametrize("rp", [1.3, 1.1234, 2.0])
def test_repetition_penalty_rule(rp):
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(2000).astype(np.float32)
    pen = [int(np.argmax(lg)), 5, 77, 1999]
    lg[5] = -0.5
    p = np.float32(round(rp * 1000)) / np.float32(1000)
    want = lg.copy()
    for t in pen:
        want[t] = want[t] / p if want[t] > 0 else want[t] * p
    tok, buf = orc.argmax(lg, pen, rp)
    assert tok == int(np.argmax(want))
    v, i = pairs_of(buf)
    for g in range(len(v)):
        seg = want[256 * g:256 * (g + 1)]
        assert i[g] == 256 * g + int(np.argmax(seg)) and v[g] == np.float32(seg.max())


def sample_reference_reading(values, ids, temperature, top_p, top_k, repetition_penalty, seen, u):
    """sampleFromCandidateBuffer (sampling.ts:23-76), Math.random() -> u."""
    seen = set(seen)
    rp = max(repetition_penalty, 1e-6)
    cands = []
    for val, idx in zip(values, ids):
        val = float(val)
        if not math.isfinite(val) or idx == 0xFFFFFFFF:
            continue
        if rp != 1 and int(idx) in seen:
            val = val / rp if val > 0 else val * rp
        cands.append((val, int(idx)))
    cands = sorted(cands, key=lambda c: -c[0])  # stable, like Array.prototype.sort
    k = max(0, int(math.floor(top_k))) if top_k is not None else 0
    lim = cands[:min(k, len(cands))] if k > 0 else cands
    if temperature <= 0:
        return lim[0][1] if lim else (cands[0][1] if cands else 0)
    top_p = min(max(top_p, 0.0), 1.0)
    mx = lim[0][0] if lim else 0.0
    probs = [math.exp((c[0] - mx) / temperature) for c in lim]
    total = 0.0
    for p in probs:
        total += p
    cutoff = len(lim)
    if top_p < 1 and total > 0:
        cdf = 0.0
        for j, p in enumerate(probs):
            cdf += p / total
            if cdf >= top_p:
                cutoff = j + 1
                break
    st = 0.0
    for j in range(cutoff):
        st += probs[j]
    r = u * st
    for j in range(cutoff):
        r -= probs[j]
        if r <= 0:
            return lim[j][1]
    return lim[max(0, cutoff - 1)][1] if lim else 0


@pytest.mark.parametrize("case", range(40))
def test_sampler_matches_reference_reading(case):
    rng = np.random.default_rng(100 + case)
    groups = int(rng.integers(1, 1100))
    vals = (rng.standard_normal(groups) * rng.uniform(0.5, 8)).astype(np.float32)
    vals[rng.random(groups) < 0.05] = np.float32(rng.choice([np.inf, -np.inf, np.nan]))
    if case % 5 == 0:
        vals[: groups // 2] = vals[0]  # ties keep their order
    ids = (np.arange(groups) * 256 + rng.integers(0, 256, groups)).astype(np.uint32)
    ids[rng.random(groups) < 0.02] = 0xFFFFFFFF
    buf = np.empty(groups * 2, dtype=np.uint32)
    buf[0::2] = vals.view(np.uint32)
    buf[1::2] = ids
    temperature = [0.0, 0.3, 0.8, 1.0, 1.7][case % 5]
    top_p = [1.0, 0.9, 0.5, 0.0][case % 4]
    top_k = [0, 1, 40, 5000][case % 4 if case % 3 else 0]
    rp = [1.0, 1.3][case % 2]
    seen = [int(x) for x in rng.choice(ids, size=min(20, groups), replace=False)]
    for j in range(6):
        u = orc.uniform(case, j)
        want = sample_reference_reading(vals, ids, temperature, top_p, top_k, rp, seen, u)
        got = orc.sample_candidates(buf, temperature, top_p, top_k, rp, seen, u)
        assert got == want, (case, j, u)


def test_uniform_draws_are_in_unit_interval_and_spread():
    u = np.array([orc.uniform(s, t) for s in range(20) for t in range(50)])
    assert (u >= 0).all() and (u < 1).all()
    assert abs(u.mean() - 0.5) < 0.03 and abs(u.var() - 1 / 12) < 0.01


def test_top_k_one_is_greedy_over_candidates():
    rng = np.random.default_rng(9)
    lg = rng.standard_normal(3000).astype(np.float32)
    tok, buf = orc.argmax(lg)
    for j in range(10):
        assert orc.sample_candidates(buf, 1.0, 1.0, 1, 1.0, [], orc.uniform(1, j)) == tok
