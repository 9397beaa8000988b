"""Writes dequant_kat.npz: hand-built GGUF blocks and their decoded values.

Known-answer blocks for every block type on the decode path (Q5_0, Q5_1,
Q8_0, Q4_K, Q5_K, Q6_K; the layouts of llama.cpp's ggml-common.h as read by
the reference's src/lib/gguf.ts:103-130 and decoded by
src/lib/llama-wgsl-runtime.ts:2202-2613). The expected values come from the
per-element closed forms below, one element at a time in plain Python
floats rounded to float32 after each operation (the fp32 op order of
llama.cpp's dequantize_row_*), independent of the oracle and of the numpy
decoder in tests/ggufpy.py.

Cases per type: zero block, d = 0, every quant value in order, sign and
high-bit packing (Q4_K/Q5_K scale index j >= 4, Q6_K negative int8 scales,
Q5 high bits), subnormal / negative-zero / infinite f16 scales.

Run: python tests/golden/make_dequant_kat.py  (rewrites the .npz next to it)
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

F32 = np.float32


def f16(x: float) -> bytes:
    return np.array([x], dtype=np.float16).tobytes()


def h(b: bytes, off: int) -> float:
    return float(np.frombuffer(b[off:off + 2], dtype=np.float16)[0])


def r(x) -> float:
    return float(F32(x))


def mul(a, b):
    return r(F32(a) * F32(b))


def sub(a, b):
    return r(F32(a) - F32(b))


def add(a, b):
    return r(F32(a) + F32(b))


# ---- closed forms, element by element -------------------------------------

def dec_q8_0(b: bytes):
    d = h(b, 0)
    return [mul(struct.unpack_from("b", b, 2 + i)[0], d) for i in range(32)]


def dec_q5(b: bytes, with_min: bool):
    d = h(b, 0)
    m = h(b, 2) if with_min else 0.0
    qh_at = 4 if with_min else 2
    qh = struct.unpack_from("<I", b, qh_at)[0]
    qs = b[qh_at + 4:qh_at + 20]
    out = [0.0] * 32
    for j in range(16):
        hb0 = (qh >> j) & 1
        hb1 = (qh >> (j + 16)) & 1
        v0 = (qs[j] & 0xF) | (hb0 << 4)
        v1 = (qs[j] >> 4) | (hb1 << 4)
        if with_min:
            out[j] = add(mul(v0, d), m)
            out[j + 16] = add(mul(v1, d), m)
        else:
            out[j] = mul(v0 - 16, d)
            out[j + 16] = mul(v1 - 16, d)
    return out


def scale_min_k4(j: int, q: bytes):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def dec_qk(b: bytes, five: bool):
    d, dmin = h(b, 0), h(b, 2)
    scales = b[4:16]
    qh = b[16:48] if five else None
    ql = b[48:176] if five else b[16:144]
    out = []
    for step in range(4):  # 64 elements: two sub-blocks of 32
        sc0, m0 = scale_min_k4(2 * step, scales)
        sc1, m1 = scale_min_k4(2 * step + 1, scales)
        d1, mn1 = mul(d, sc0), mul(dmin, m0)
        d2, mn2 = mul(d, sc1), mul(dmin, m1)
        q = ql[32 * step:32 * step + 32]
        for l in range(32):
            v = q[l] & 0xF
            if five and (qh[l] >> (2 * step)) & 1:
                v += 16
            out.append(sub(mul(d1, v), mn1))
        for l in range(32):
            v = q[l] >> 4
            if five and (qh[l] >> (2 * step + 1)) & 1:
                v += 16
            out.append(sub(mul(d2, v), mn2))
    return out


def dec_q6_k(b: bytes):
    ql, qh = b[0:128], b[128:192]
    sc = struct.unpack_from("16b", b, 192)
    d = h(b, 208)
    out = [0.0] * 256
    for half in range(2):
        L, H, S = ql[64 * half:], qh[32 * half:], sc[8 * half:]
        for l in range(32):
            isub = l // 16
            q1 = ((L[l] & 0xF) | (((H[l] >> 0) & 3) << 4)) - 32
            q2 = ((L[l + 32] & 0xF) | (((H[l] >> 2) & 3) << 4)) - 32
            q3 = ((L[l] >> 4) | (((H[l] >> 4) & 3) << 4)) - 32
            q4 = ((L[l + 32] >> 4) | (((H[l] >> 6) & 3) << 4)) - 32
            base = 128 * half
            for k, q in enumerate((q1, q2, q3, q4)):
                out[base + 32 * k + l] = mul(mul(d, S[isub + 2 * k]), q)
    return out


# ---- hand-built blocks ----------------------------------------------------

SPECIAL = [0.0, -0.0, 5.96e-8, 6.1e-5, 1.0, -2.5, 65504.0, float("inf")]


def blocks_q8_0(rng):
    out = [f16(0.0) + bytes(32), f16(0.0) + bytes(range(32)),
           f16(0.5) + np.arange(-16, 16, dtype=np.int8).tobytes(),
           f16(-1.0) + np.array([-128, 127] * 16, dtype=np.int8).tobytes()]
    for s in SPECIAL:
        out.append(f16(s) + rng.integers(-128, 128, 32).astype(np.int8).tobytes())
    return out


def blocks_q5(rng, with_min):
    head = (lambda d, m: f16(d) + f16(m)) if with_min else (lambda d, m: f16(d))
    out = [head(0.0, 0.0) + bytes(20),
           head(1.0, 0.0) + struct.pack("<I", 0) + bytes((j | (j << 4)) & 0xFF for j in range(16)),
           head(1.0, -3.0) + struct.pack("<I", 0xFFFFFFFF) + bytes([0xFF] * 16),
           head(0.25, 0.5) + struct.pack("<I", 0xA5A5F00F) + rng.integers(0, 256, 16).astype(np.uint8).tobytes()]
    for s in SPECIAL:
        out.append(head(s, -s if with_min else 0.0) + rng.integers(0, 256, 20).astype(np.uint8).tobytes())
    return out


def blocks_qk(rng, five):
    nq = 176 - 16 if five else 144 - 16
    out = [f16(0.0) + f16(0.0) + bytes(12) + bytes(nq)]
    # every nibble value, unit scales (6-bit fields all 1), no mins
    sc = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])
    ql = bytes(((i % 16) | (((i + 7) % 16) << 4)) for i in range(128))
    qh = bytes((i * 37) & 0xFF for i in range(32)) if five else b""
    out.append(f16(1.0) + f16(0.0) + sc + qh + ql)
    # high-bit packing of scale index j >= 4: top two bits of bytes 0..7 in use
    sc = bytes([0xC5, 0x83, 0x41, 0xFF, 0xC2, 0x7F, 0x80, 0x3F, 0x9A, 0x5B, 0xE1, 0x0F])
    out.append(f16(0.01) + f16(0.02) + sc + (rng.integers(0, 256, 32).astype(np.uint8).tobytes() if five else b"")
               + rng.integers(0, 256, 128).astype(np.uint8).tobytes())
    for s in SPECIAL:
        out.append(f16(s) + f16(abs(s) / 3) + rng.integers(0, 256, 12 + nq).astype(np.uint8).tobytes())
    return out


def blocks_q6_k(rng):
    out = [bytes(208) + f16(0.0)]
    ql = bytes(((i % 16) | (((i + 3) % 16) << 4)) for i in range(128))
    qh = bytes((i * 29) & 0xFF for i in range(64))
    sc = np.array([1, -1, 2, -2, 127, -128, 3, -3, 5, -7, 11, -13, 64, -64, 0, 1], dtype=np.int8).tobytes()
    out.append(ql + qh + sc + f16(1.0))
    for s in SPECIAL:
        out.append(rng.integers(0, 256, 192).astype(np.uint8).tobytes()
                   + rng.integers(-128, 128, 16).astype(np.int8).tobytes() + f16(s))
    return out


def main() -> None:
    rng = np.random.default_rng(20261201)
    cases = {
        8: (blocks_q8_0(rng), dec_q8_0),
        6: (blocks_q5(rng, False), lambda b: dec_q5(b, False)),
        7: (blocks_q5(rng, True), lambda b: dec_q5(b, True)),
        12: (blocks_qk(rng, False), lambda b: dec_qk(b, False)),
        13: (blocks_qk(rng, True), lambda b: dec_qk(b, True)),
        14: (blocks_q6_k(rng), dec_q6_k),
    }
    arrays = {}
    for t, (blocks, dec) in cases.items():
        arrays[f"blocks_{t}"] = np.frombuffer(b"".join(blocks), dtype=np.uint8)
        arrays[f"values_{t}"] = np.array([v for b in blocks for v in dec(b)], dtype=np.float32)
    np.savez(Path(__file__).with_name("dequant_kat.npz"), **arrays)
    print({k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
