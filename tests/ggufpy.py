"""Test-side GGUF reader and block decoders in numpy.

Written independently of the oracle and of the product: the header parser
follows the GGUF v3 layout, and the block decoders follow llama.cpp's
dequantize_row_{q8_0,q5_0,q5_1,q4_K,q5_K,q6_K} loop structure (whole blocks,
scale pairs per 64 elements) rather than the reference WGSL's per-element
index arithmetic, so an index mistake in either shows up as a mismatch.
Arithmetic is numpy float32 (IEEE, no fused multiply-add), matching the
reference op order (d*sc)*q - (dmin*m).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

TYPE_BLOCK = {0: (1, 4), 1: (1, 2), 6: (32, 22), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176),
              14: (256, 210)}


@dataclass
class Tensor:
    name: str
    shape: list
    type: int
    offset: int
    n_bytes: int


@dataclass
class Gguf:
    version: int
    kv: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)
    data_offset: int = 0
    raw: bytes = b""

    def tensor_bytes(self, name: str) -> bytes:
        t = self.tensors[name]
        start = self.data_offset + t.offset
        return self.raw[start:start + t.n_bytes]


def read_gguf(path: str) -> Gguf:
    raw = open(path, "rb").read()
    off = 0

    def take(fmt):
        nonlocal off
        v = struct.unpack_from("<" + fmt, raw, off)
        off += struct.calcsize("<" + fmt)
        return v[0]

    def string():
        nonlocal off
        n = take("Q")
        s = raw[off:off + n].decode()
        off += n
        return s

    scalar = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

    def value(t):
        if t in scalar:
            return take(scalar[t])
        if t == 8:
            return string()
        if t == 9:
            it = take("I")
            n = take("Q")
            return [value(it) for _ in range(n)]
        raise ValueError(f"bad metadata type {t}")

    assert take("I") == 0x46554747, "bad magic"
    g = Gguf(version=take("I"), raw=raw)
    nt, nkv = take("Q"), take("Q")
    for _ in range(nkv):
        k = string()
        g.kv[k] = value(take("I"))
    for _ in range(nt):
        name = string()
        nd = take("I")
        shape = [take("Q") for _ in range(nd)]
        ttype = take("I")
        toff = take("Q")
        n = int(np.prod(shape))
        be, bb = TYPE_BLOCK[ttype]
        g.tensors[name] = Tensor(name, shape, ttype, toff, n // be * bb)
    g.data_offset = (off + 31) // 32 * 32
    return g


def _f16(b: np.ndarray) -> np.ndarray:
    return b.copy().view(np.float16).astype(np.float32)


def _scale_min_k4(scales: np.ndarray, j: int):
    # scales: [nb, 12] uint8
    if j < 4:
        return (scales[:, j] & 63).astype(np.float32), (scales[:, j + 4] & 63).astype(np.float32)
    sc = (scales[:, j + 4] & 0xF) | ((scales[:, j - 4] >> 6) << 4)
    m = (scales[:, j + 4] >> 4) | ((scales[:, j] >> 6) << 4)
    return sc.astype(np.float32), m.astype(np.float32)


def dequantize(type_id: int, data: bytes, n: int) -> np.ndarray:
    be, bb = TYPE_BLOCK[type_id]
    raw = np.frombuffer(data, dtype=np.uint8)[: n // be * bb]
    if type_id == 0:
        return raw.view(np.float32).copy()
    if type_id == 1:
        return raw.view(np.float16).astype(np.float32)
    blk = raw.reshape(-1, bb)
    nb = blk.shape[0]
    f32 = np.float32
    if type_id == 8:  # Q8_0
        d = _f16(blk[:, 0:2])
        qs = blk[:, 2:34].view(np.int8).astype(np.float32)
        return (qs * d).reshape(-1)
    if type_id in (6, 7):  # Q5_0 / Q5_1
        d = _f16(blk[:, 0:2])
        qh_at, qs_at = (2, 6) if type_id == 6 else (4, 8)
        qh = blk[:, qh_at:qh_at + 4].copy().view(np.uint32)[:, 0]
        qs = blk[:, qs_at:qs_at + 16].astype(np.uint32)
        j = np.arange(16, dtype=np.uint32)
        xh0 = ((qh[:, None] >> j) << 4) & 0x10
        xh1 = (qh[:, None] >> (j + 12)) & 0x10
        lo = (qs & 0x0F) | xh0
        hi = (qs >> 4) | xh1
        y = np.empty((nb, 32), dtype=np.float32)
        if type_id == 6:
            y[:, :16] = (lo.astype(np.int32) - 16).astype(f32) * d
            y[:, 16:] = (hi.astype(np.int32) - 16).astype(f32) * d
        else:
            m = _f16(blk[:, 2:4])
            y[:, :16] = lo.astype(f32) * d + m
            y[:, 16:] = hi.astype(f32) * d + m
        return y.reshape(-1)
    if type_id in (12, 13):  # Q4_K / Q5_K
        d = _f16(blk[:, 0:2])[:, 0]
        dmin = _f16(blk[:, 2:4])[:, 0]
        scales = blk[:, 4:16]
        if type_id == 12:
            ql = blk[:, 16:144]
            qh = None
        else:
            qh = blk[:, 16:48]
            ql = blk[:, 48:176]
        y = np.empty((nb, 256), dtype=np.float32)
        for step in range(4):
            sc0, m0 = _scale_min_k4(scales, 2 * step)
            sc1, m1 = _scale_min_k4(scales, 2 * step + 1)
            d1, mm1 = d * sc0, dmin * m0
            d2, mm2 = d * sc1, dmin * m1
            q = ql[:, 32 * step:32 * step + 32]
            lo = (q & 0xF).astype(np.float32)
            hi = (q >> 4).astype(np.float32)
            if qh is not None:
                lo = lo + np.where(qh & (1 << (2 * step)), 16, 0).astype(np.float32)
                hi = hi + np.where(qh & (2 << (2 * step)), 16, 0).astype(np.float32)
            y[:, 64 * step:64 * step + 32] = d1[:, None] * lo - mm1[:, None]
            y[:, 64 * step + 32:64 * step + 64] = d2[:, None] * hi - mm2[:, None]
        return y.reshape(-1)
    if type_id == 14:  # Q6_K
        ql = blk[:, 0:128].astype(np.int32)
        qh = blk[:, 128:192].astype(np.int32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float32)
        d = _f16(blk[:, 208:210])[:, 0]
        y = np.empty((nb, 256), dtype=np.float32)
        for half in range(2):
            L = ql[:, 64 * half:64 * half + 64]
            H = qh[:, 32 * half:32 * half + 32]
            S = sc[:, 8 * half:8 * half + 8]
            lidx = np.arange(32)
            isub = lidx // 16
            q1 = ((L[:, :32] & 0xF) | (((H >> 0) & 3) << 4)) - 32
            q2 = ((L[:, 32:] & 0xF) | (((H >> 2) & 3) << 4)) - 32
            q3 = ((L[:, :32] >> 4) | (((H >> 4) & 3) << 4)) - 32
            q4 = ((L[:, 32:] >> 4) | (((H >> 6) & 3) << 4)) - 32
            base = 128 * half
            for k, q in enumerate((q1, q2, q3, q4)):
                s = S[:, isub + 2 * k]
                y[:, base + 32 * k:base + 32 * k + 32] = (d[:, None] * s) * q.astype(np.float32)
        return y.reshape(-1)
    raise ValueError(f"unsupported type {type_id}")


def matrix(g: Gguf, name: str) -> np.ndarray:
    t = g.tensors[name]
    n = int(np.prod(t.shape))
    w = dequantize(t.type, g.tensor_bytes(name), n)
    if len(t.shape) == 1:
        return w
    return w.reshape(t.shape[1], t.shape[0])
