"""GPU parity of the dequant and dequant-matvec kernels against the oracle.

Block decode must be bit-exact (the reference WGSL decode order,
llama-wgsl-runtime.ts:2202-2613); the matvec must agree within fp32
reduction-order differences: max|y_gpu - y_ref| / max|y_ref| <= 1e-4 (the
contract is 1e-3).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from chonklm_amd._lib import check, lib
from oracle import oracle as orc
from tests.blocks import TYPES, random_blocks
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

BLOCK = orc.BLOCK


def gpu_dequant(type_id: int, blocks: np.ndarray, n_rows: int, row_len: int) -> np.ndarray:
    out = np.empty(n_rows * row_len, dtype=np.float32)
    check(lib().chonk_dequant(0, type_id, blocks.ctypes.data, n_rows, row_len,
                              out.ctypes.data_as(C.POINTER(C.c_float))))
    return out


def gpu_matvec(type_id: int, blocks: np.ndarray, n_rows: int, row_len: int, x: np.ndarray, reps: int = 0):
    y = np.empty(n_rows, dtype=np.float32)
    us = C.c_double()
    check(lib().chonk_matvec(0, type_id, blocks.ctypes.data, n_rows, row_len,
                             x.ctypes.data_as(C.POINTER(C.c_float)), y.ctypes.data_as(C.POINTER(C.c_float)), reps,
                             C.byref(us)))
    return y, us.value


@pytest.mark.parametrize("tname", list(TYPES))
@pytest.mark.parametrize("special", [False, True])
def test_dequant_bit_exact(tname, special):
    type_id = TYPES[tname]
    rng = np.random.default_rng(100 + type_id + (7 if special else 0))
    n_rows, row_len = 7, 768 if BLOCK[type_id][0] == 256 else 352
    blocks = random_blocks(type_id, n_rows * row_len, rng, special)
    got = gpu_dequant(type_id, blocks, n_rows, row_len)
    want = orc.dequant(type_id, blocks, n_rows * row_len)
    both_nan = np.isnan(got) & np.isnan(want)
    same = (got.view(np.uint32) == want.view(np.uint32)) | both_nan
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{tname}: {bad.size} elements differ, first {bad[:5]} {got[bad[:5]]} vs {want[bad[:5]]}"


MATVEC_SHAPES = [
    ("Q4_K", 2048, 1024), ("Q4_K", 3072, 1024), ("Q4_K", 1024, 3072), ("Q4_K", 1000, 2048),
    ("Q6_K", 1024, 3072), ("Q6_K", 1024, 1024), ("Q6_K", 999, 256),
    ("Q8_0", 576, 576), ("Q8_0", 192, 576), ("Q8_0", 1024, 640),
    ("Q5_0", 1536, 576), ("Q5_0", 576, 576), ("Q5_0", 2048, 640), ("Q5_0", 333, 96),
    ("Q5_1", 640, 640), ("Q5_K", 512, 1024),
]


@pytest.mark.parametrize("tname,n_rows,row_len", MATVEC_SHAPES)
def test_matvec_matches_oracle(tname, n_rows, row_len):
    type_id = TYPES[tname]
    rng = np.random.default_rng(n_rows * 31 + row_len + type_id)
    blocks = random_blocks(type_id, n_rows * row_len, rng)
    x = rng.standard_normal(row_len).astype(np.float32)
    got, _ = gpu_matvec(type_id, blocks, n_rows, row_len, x)
    want = orc.matvec(type_id, blocks, n_rows, row_len, x)
    assert rel_err(got, want) <= 1e-4, f"{tname} {n_rows}x{row_len}: rel err {rel_err(got, want):.3e}"


@pytest.mark.parametrize("tname,n_rows,row_len", [("Q6_K", 151936, 1024), ("Q8_0", 49152, 576)])
def test_matvec_lm_head_shapes(tname, n_rows, row_len):
    type_id = TYPES[tname]
    rng = np.random.default_rng(5)
    blocks = random_blocks(type_id, n_rows * row_len, rng)
    x = rng.standard_normal(row_len).astype(np.float32)
    got, _ = gpu_matvec(type_id, blocks, n_rows, row_len, x)
    want = orc.matvec(type_id, blocks, n_rows, row_len, x, threads=16)
    assert rel_err(got, want) <= 1e-4
