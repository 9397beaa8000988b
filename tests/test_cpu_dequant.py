"""Oracle block decode and matvec, pinned without a GPU.

* Known-answer blocks (tests/golden/dequant_kat.npz, written by
  tests/golden/make_dequant_kat.py from per-element closed forms): bit-exact.
* An independent vectorised numpy decoder (tests/ggufpy.py) on random blocks,
  including zero / subnormal / negative-zero / large f16 scales: bit-exact.
* Matvec against float64 dot products of the decoded rows: the oracle
  accumulates in fp32 in the WGSL order, so it agrees to ~1e-6 relative.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc
from tests import ggufpy
from tests.blocks import TYPES, random_blocks
from tests.conftest import rel_err

KAT = np.load(Path(__file__).parent / "golden" / "dequant_kat.npz")


def same_bits(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


@pytest.mark.parametrize("tname", list(TYPES))
def test_known_answer_blocks(tname):
    t = TYPES[tname]
    blocks, want = KAT[f"blocks_{t}"], KAT[f"values_{t}"]
    got = orc.dequant(t, blocks, want.size)
    bad = np.flatnonzero(~same_bits(got, want))
    assert bad.size == 0, f"{tname}: elements {bad[:8]} got {got[bad[:8]]} want {want[bad[:8]]}"


@pytest.mark.parametrize("tname", list(TYPES))
def test_known_answers_agree_with_numpy_decoder(tname):
    # the two restatements that pin the oracle agree with each other
    t = TYPES[tname]
    blocks, want = KAT[f"blocks_{t}"], KAT[f"values_{t}"]
    with np.errstate(all="ignore"):
        alt = ggufpy.dequantize(t, blocks.tobytes(), want.size)
    assert same_bits(alt, want).all()


@pytest.mark.parametrize("special", [False, True])
@pytest.mark.parametrize("tname", list(TYPES))
def test_random_blocks_match_numpy_decoder(tname, special):
    t = TYPES[tname]
    rng = np.random.default_rng(7 * t + special)
    be = orc.BLOCK[t][0]
    n = 64 * be
    blocks = random_blocks(t, n, rng, special)
    got = orc.dequant(t, blocks, n)
    with np.errstate(all="ignore"):
        want = ggufpy.dequantize(t, blocks.tobytes(), n)
    assert same_bits(got, want).all()


def test_f32_f16_passthrough():
    x = np.array([0.0, -0.0, 1.5, -2.25, 65504.0, 6.1e-5, 5.96e-8], dtype=np.float32)
    assert same_bits(orc.dequant(0, x.view(np.uint8), x.size), x).all()
    h = x.astype(np.float16)
    assert same_bits(orc.dequant(1, h.view(np.uint8), h.size), h.astype(np.float32)).all()


@pytest.mark.parametrize("tname,n_rows,row_len", [("Q4_K", 96, 1024), ("Q6_K", 64, 768), ("Q8_0", 80, 576),
                                                  ("Q5_0", 72, 640), ("Q5_1", 40, 96), ("Q5_K", 33, 512)])
def test_matvec_matches_float64(tname, n_rows, row_len):
    t = TYPES[tname]
    rng = np.random.default_rng(n_rows + row_len)
    blocks = random_blocks(t, n_rows * row_len, rng)
    x = rng.standard_normal(row_len).astype(np.float32)
    w = ggufpy.dequantize(t, blocks.tobytes(), n_rows * row_len).reshape(n_rows, row_len).astype(np.float64)
    want = w @ x.astype(np.float64)
    got = orc.matvec(t, blocks, n_rows, row_len, x, threads=4)
    assert rel_err(got, want) <= 2e-6


def test_matvec_row_independence():
    # every row is its own dot product: permuting rows permutes outputs exactly
    t, n, k = TYPES["Q4_K"], 32, 512
    rng = np.random.default_rng(3)
    blocks = random_blocks(t, n * k, rng).reshape(n, -1)
    x = rng.standard_normal(k).astype(np.float32)
    perm = rng.permutation(n)
    y = orc.matvec(t, blocks.reshape(-1), n, k, x)
    yp = orc.matvec(t, blocks[perm].reshape(-1), n, k, x)
    assert np.array_equal(y[perm], yp)
