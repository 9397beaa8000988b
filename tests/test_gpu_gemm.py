"""GPU parity of the batched pass's dequant-fused MFMA GEMM against the oracle.

Y[T,N] = X[T,K] W[N,K]^T with W the oracle's bit-exact block decode
(oracle.dequant, pinned by the golden vectors) and the product taken in
float64 on the host. The GEMM splits both operands into fp16 hi + lo halves
and accumulates in fp32 on the matrix cores; the bar is the matvec's:
max|y - y_ref| / max|y_ref| <= 1e-4 (the contract is 1e-3), for every token
row. Shapes cover K not a multiple of the 128-wide stage, N and T not
multiples of the 64-wide tiles, and a single row.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from chonklm_amd._lib import check, lib
from oracle import oracle as orc
from tests.blocks import TYPES, random_blocks

pytestmark = pytest.mark.gpu


def gpu_gemm(type_id: int, blocks: np.ndarray, n_rows: int, row_len: int, x: np.ndarray, reps: int = 0):
    t = x.shape[0]
    y = np.empty((t, n_rows), dtype=np.float32)
    us = C.c_double()
    xc = np.ascontiguousarray(x, dtype=np.float32)
    check(lib().chonk_gemm(0, type_id, blocks.ctypes.data, n_rows, row_len, xc.ctypes.data_as(C.POINTER(C.c_float)), t,
                           y.ctypes.data_as(C.POINTER(C.c_float)), reps, C.byref(us)))
    return y, us.value


GEMM_SHAPES = [
    ("Q4_K", 1024, 1024, 64), ("Q4_K", 1000, 2048, 100), ("Q4_K", 3072, 1024, 1), ("Q4_K", 256, 3072, 130),
    ("Q6_K", 1024, 3072, 37), ("Q6_K", 999, 256, 64),
    ("Q8_0", 576, 576, 65), ("Q8_0", 192, 608, 3),
    ("Q5_0", 1536, 576, 70), ("Q5_0", 333, 96, 17),
    ("Q5_1", 640, 640, 33), ("Q5_K", 512, 1024, 80),
    # passes over 512 rows take the 128-row tiles: ragged token and weight-row counts
    ("Q4_K", 1000, 2048, 700), ("Q6_K", 999, 768, 601), ("Q8_0", 576, 576, 530),
    ("Q5_0", 333, 96, 515), ("Q5_1", 640, 640, 513), ("Q5_K", 512, 1024, 520),
]


@pytest.mark.parametrize("tname,n_rows,row_len,n_tok", GEMM_SHAPES)
def test_gemm_matches_oracle(tname, n_rows, row_len, n_tok):
    type_id = TYPES[tname]
    rng = np.random.default_rng(n_rows * 17 + row_len * 3 + n_tok + type_id)
    blocks = random_blocks(type_id, n_rows * row_len, rng)
    w = orc.dequant(type_id, blocks, n_rows * row_len).reshape(n_rows, row_len).astype(np.float64)
    x = rng.standard_normal((n_tok, row_len)).astype(np.float32)
    x[0] *= 300.0  # rows of very different scale share the tile
    got, _ = gpu_gemm(type_id, blocks, n_rows, row_len, x)
    want = x.astype(np.float64) @ w.T
    for t in range(n_tok):
        err = np.max(np.abs(got[t] - want[t])) / max(np.max(np.abs(want[t])), 1e-30)
        assert err <= 1e-4, f"{tname} {n_rows}x{row_len} row {t}: rel err {err:.3e}"


def test_gemm_zero_and_tiny_rows():
    type_id = TYPES["Q4_K"]
    rng = np.random.default_rng(3)
    n_rows, row_len = 128, 512
    blocks = random_blocks(type_id, n_rows * row_len, rng)
    w = orc.dequant(type_id, blocks, n_rows * row_len).reshape(n_rows, row_len).astype(np.float64)
    x = rng.standard_normal((3, row_len)).astype(np.float32)
    x[1] = 0.0
    x[2] *= 1e-20
    got, _ = gpu_gemm(type_id, blocks, n_rows, row_len, x)
    assert np.all(got[1] == 0.0)
    want = x[2].astype(np.float64) @ w.T
    assert np.max(np.abs(got[2] - want)) <= 1e-4 * np.max(np.abs(want))
