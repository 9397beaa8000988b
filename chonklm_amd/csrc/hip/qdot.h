// Per-type 32-element unit decode for the striped layout (device_common.h).
//
// For every GGUF type there is
//   * Frag<T>            the raw bytes of one unit (loaded with vector loads),
//   * load_unit<T>()     issues the loads for (row, unit),
//   * load_xu<T>() / dot_q<T>()  sum_i x[k_i] * w_i over the unit's 32 elements
//                        against the integer-digit form of x (XqView),
//   * dequant_unit<T>()  the 32 weights, bit-exact with the reference decode.
//
// Element placement inside a unit, and the exact fp32 operation order used by
// dequant_unit, follow the reference's WGSL weight helpers
// (src/lib/llama-wgsl-runtime.ts: q5_0 :2230-2246, q5_1 :2280-2289,
// q8_0 :2321-2327, q4_k :2378-2410, q5_k :2479-2495, q6_k :2560-2580), which
// in turn follow llama.cpp's dequantize_row_* block formats. dot_q uses the
// factored form d*sc*sum(x*q) - dmin*m*sum(x) and is only required to match
// within fp32 rounding.
#pragma once

#include "device_common.h"

namespace chonk {

__device__ __forceinline__ uint32_t byte_of3(uint32_t w0, uint32_t w1, uint32_t w2, int j) {
  const uint32_t w = j < 4 ? w0 : (j < 8 ? w1 : w2);
  return (w >> (8 * (j & 3))) & 0xffu;
}

// scale_min_k4 over the 12 packed scale bytes held in three words.
__device__ __forceinline__ void scale_min(int j, uint32_t w0, uint32_t w1, uint32_t w2, uint32_t* sc, uint32_t* m) {
  if (j < 4) {
    *sc = byte_of3(w0, w1, w2, j) & 63u;
    *m = byte_of3(w0, w1, w2, j + 4) & 63u;
  } else {
    *sc = (byte_of3(w0, w1, w2, j + 4) & 15u) | ((byte_of3(w0, w1, w2, j - 4) >> 6) << 4);
    *m = (byte_of3(w0, w1, w2, j + 4) >> 4) | ((byte_of3(w0, w1, w2, j) >> 6) << 4);
  }
}

__device__ __forceinline__ float nib_lo(uint32_t w, int i) { return (float)((w >> (8 * i)) & 15u); }
__device__ __forceinline__ float nib_hi(uint32_t w, int i) { return (float)((w >> (8 * i + 4)) & 15u); }

template <int T>
struct Frag;

template <>
struct Frag<QT_Q4_K> {
  uint4 qs;
  uint4 hdr;
};
template <>
struct Frag<QT_Q5_K> {
  uint4 qs;
  uint4 hdr;
  uint4 qh;
};
template <>
struct Frag<QT_Q6_K> {
  uint2 qa, qb, qh, sc;
  uint32_t d;
};
template <>
struct Frag<QT_Q8_0> {
  uint4 q0, q1;
  uint32_t d;
};
template <>
struct Frag<QT_Q5_0> {
  uint4 qs;
  uint32_t qh;
  uint32_t d;
};
template <>
struct Frag<QT_Q5_1> {
  uint4 qs;
  uint32_t qh;
  uint32_t d, m;
};

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *gbl((const unsigned short*)p); }

template <int T>
__device__ __forceinline__ Frag<T> load_unit(const QMat& w, int row, int u);

template <>
__device__ __forceinline__ Frag<QT_Q4_K> load_unit<QT_Q4_K>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  Frag<QT_Q4_K> f;
  f.qs = ldg4(w.s0 + row * (K / 2) + 16 * u);
  f.hdr = ldg4(w.s1 + row * (K / 16) + 16 * (u >> 3));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_K> load_unit<QT_Q5_K>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  Frag<QT_Q5_K> f;
  f.qs = ldg4(w.s0 + row * (K / 2) + 16 * u);
  f.hdr = ldg4(w.s1 + row * (K / 16) + 16 * (u >> 3));
  const int hh = u & 1;
  f.qh = ldg4(w.s2 + row * (K / 8) + 32 * (u >> 3) + 16 * hh);
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q6_K> load_unit<QT_Q6_K>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  const int sb = u >> 3, c = u & 7, h = c >> 2, b = c & 3;
  Frag<QT_Q6_K> f;
  const uint8_t* ql = w.s0 + row * (K / 2) + 128 * sb + 64 * h + 8 * b;
  f.qa = ldg2(ql);
  f.qb = ldg2(ql + 32);
  f.qh = ldg2(w.s1 + row * (K / 4) + 64 * sb + 32 * h + 8 * b);
  f.sc = ldg2(w.s2 + row * (K / 16) + 16 * sb + 8 * h);
  f.d = ld_u16(w.s3 + 2 * (row * (K / 256) + sb));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q8_0> load_unit<QT_Q8_0>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  Frag<QT_Q8_0> f;
  const uint8_t* q = w.s0 + row * K + 32 * u;
  f.q0 = ldg4(q);
  f.q1 = ldg4(q + 16);
  f.d = ld_u16(w.s1 + 2 * (row * (K / 32) + u));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_0> load_unit<QT_Q5_0>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  Frag<QT_Q5_0> f;
  f.qs = ldg4(w.s0 + row * (K / 2) + 16 * u);
  f.qh = ldg1(w.s1 + 4 * (row * (K / 32) + u));
  f.d = ld_u16(w.s2 + 2 * (row * (K / 32) + u));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_1> load_unit<QT_Q5_1>(const QMat& w, int row, int u) {
  const size_t K = (size_t)w.k;
  Frag<QT_Q5_1> f;
  f.qs = ldg4(w.s0 + row * (K / 2) + 16 * u);
  f.qh = ldg1(w.s1 + 4 * (row * (K / 32) + u));
  f.d = ld_u16(w.s2 + 2 * (row * (K / 32) + u));
  f.m = ld_u16(w.s3 + 2 * (row * (K / 32) + u));
  return f;
}

// ---- lane-interleaved copy (the lm_head's row-per-lane layout) ----------------
// Rows in blocks of 64 (one per lane of a wave); per (block, unit) the 64 rows'
// unit bytes lie side by side, and per (block, super-block) the 64 rows'
// super-block scales, so that a wave's load of one unit is one contiguous run
// (1 KiB of Q6_K ql) instead of 64 rows' strided pieces, and a K-quant lane
// loads its super-block scales once per 8 units. Streams (R = 64 rows, U = K/32
// units, SB = K/256 super-blocks, i = (blk*U + u)*R + lane, j = (blk*SB + sb)*R + lane):
//   Q6_K  s0 [i][16] ql (the unit's two 8-byte runs)  s1 [i][8] qh  s2 [j][16] scales  s3 [j][2] d
//   Q8_0  s0 [i][32] qs                                s1 [i][2] d
//   Q4_K  s0 [i][16] qs                                s1 [j][16] header (d, dmin, scales)
// The bytes are those of the GGUF blocks (rows padded with zero blocks to a
// multiple of 256).
template <int T>
struct LaneFrag;  // one unit of one row
template <int T>
struct LaneHead;  // one super-block's scales of one row (K-quants)
template <>
struct LaneFrag<QT_Q6_K> {
  uint4 ql;
  uint2 qh;
};
template <>
struct LaneHead<QT_Q6_K> {
  uint4 sc;
  uint32_t d;
};
template <>
struct LaneFrag<QT_Q4_K> {
  uint4 qs;
};
template <>
struct LaneHead<QT_Q4_K> {
  uint4 hdr;
};
template <>
struct LaneFrag<QT_Q8_0> {
  uint4 q0, q1;
  uint32_t d;
};
template <>
struct LaneHead<QT_Q8_0> {};

template <int T>
__device__ __forceinline__ LaneFrag<T> load_lane_frag(const QMat& w, int blk, int u, int lane) {
  const size_t i = ((size_t)blk * (size_t)(w.k >> 5) + u) * 64 + lane;
  LaneFrag<T> f;
  if constexpr (T == QT_Q6_K) {
    f.ql = ldg4(w.s0 + 16 * i);
    f.qh = ldg2(w.s1 + 8 * i);
  } else if constexpr (T == QT_Q4_K) {
    f.qs = ldg4(w.s0 + 16 * i);
  } else {
    f.q0 = ldg4(w.s0 + 32 * i);
    f.q1 = ldg4(w.s0 + 32 * i + 16);
    f.d = ld_u16(w.s1 + 2 * i);
  }
  return f;
}

template <int T>
__device__ __forceinline__ LaneHead<T> load_lane_head(const QMat& w, int blk, int sb, int lane) {
  const size_t j = ((size_t)blk * (size_t)(w.k >> 8) + sb) * 64 + lane;
  LaneHead<T> h;
  if constexpr (T == QT_Q6_K) {
    h.sc = ldg4(w.s2 + 16 * j);
    h.d = ld_u16(w.s3 + 2 * j);
  } else if constexpr (T == QT_Q4_K) {
    h.hdr = ldg4(w.s1 + 16 * j);
  }
  (void)j;
  return h;
}

// ---- element index of unit-local element e (0..31) within the row ----------
// Q4_K/Q5_K: e<16 -> low nibble of qs byte e; e>=16 -> high nibble of byte e-16.
// Q6_K: e = 8*qd + i (quarter qd, i<8).  Q8_0/Q5_x: e is the block element.
template <int T>
__device__ __forceinline__ int unit_col(int u, int e) {
  if (T == QT_Q4_K || T == QT_Q5_K) {
    const int sb = u >> 3, c = u & 7, g = c >> 1, hh = c & 1;
    return sb * 256 + 64 * g + 16 * hh + (e < 16 ? e : 32 + (e - 16));
  } else if (T == QT_Q6_K) {
    const int sb = u >> 3, c = u & 7, h = c >> 2, b = c & 3;
    return sb * 256 + 128 * h + 32 * (e >> 3) + 8 * b + (e & 7);
  } else {
    return 32 * u + e;
  }
}

// ---- dot products --------------------------------------------------------------
// The matvec input x is re-expressed per aligned 32-element block as integers
// q = rint(x * 2^sh) with |q| <= 2^22, sh chosen from the block's largest |x|,
// held as three planes of balanced base-256 digits (q = d0 + 256 d1 + 65536 d2,
// each digit an int8). Dot products of the integer weight codes with the digit
// planes are exact in int32 (v_dot4_i32_i8, four products per instruction);
// one conversion per 8-16 elements brings them back to fp32. The representation
// error is <= 2^-22 of the block's largest |x|, the order of fp32 rounding of
// the reference's own sum.
struct XqView {
  const int8_t* plane;  // digit plane p at plane + p * k
  const float* bsc;     // [k/32] 2^-sh of each block
  const float* xs16;    // [k/16] fp32 sums of x over aligned 16-element runs
  const float* xs8;     // [k/8]  fp32 sums of x over aligned 8-element runs
  int k;
};

// x for one 32-element unit: digit words w[plane][word] (4 elements per word,
// in the order the type's dot consumes them) and per-run scales and sums.
struct XU {
  int w[3][8];
  float b[4];  // 2^-sh of the runs' blocks
  float s[4];  // fp32 sums of x over the runs
};

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// d0 + 256 d1 + 65536 d2 in fp32 (|d1 * 256 + d0| stays far inside int32)
__device__ __forceinline__ float digits_f(int a0, int a1, int a2) {
  return fmaf((float)a2, 65536.0f, (float)(a1 * 256 + a0));
}

__device__ __forceinline__ void ld_words4(const int8_t* p, int k, int off, XU& x, int at) {
#pragma unroll
  for (int pl = 0; pl < 3; ++pl) {
    const int4 v = *(const int4*)(p + pl * k + off);
    x.w[pl][at] = v.x;
    x.w[pl][at + 1] = v.y;
    x.w[pl][at + 2] = v.z;
    x.w[pl][at + 3] = v.w;
  }
}
__device__ __forceinline__ void ld_words2(const int8_t* p, int k, int off, XU& x, int at) {
#pragma unroll
  for (int pl = 0; pl < 3; ++pl) {
    const int2 v = *(const int2*)(p + pl * k + off);
    x.w[pl][at] = v.x;
    x.w[pl][at + 1] = v.y;
  }
}

template <int T>
__device__ __forceinline__ void load_xu(const XqView& x, int u, XU& r) {
  if constexpr (T == QT_Q4_K || T == QT_Q5_K) {
    // elements base + [0,16) (sub-block 2g) and base + 32 + [0,16) (sub-block 2g+1)
    const int sb = u >> 3, c = u & 7, g = c >> 1, hh = c & 1;
    const int base = sb * 256 + 64 * g + 16 * hh;
    ld_words4(x.plane, x.k, base, r, 0);
    ld_words4(x.plane, x.k, base + 32, r, 4);
    r.b[0] = x.bsc[base >> 5];
    r.b[1] = x.bsc[(base >> 5) + 1];
    r.s[0] = x.xs16[base >> 4];
    r.s[1] = x.xs16[(base >> 4) + 2];
  } else if constexpr (T == QT_Q6_K) {
    // four 8-element runs base + 32 qd + [0,8)
    const int sb = u >> 3, c = u & 7, h = c >> 2, b = c & 3;
    const int base = sb * 256 + 128 * h + 8 * b;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      ld_words2(x.plane, x.k, base + 32 * qd, r, 2 * qd);
      r.b[qd] = x.bsc[(base + 32 * qd) >> 5];
      r.s[qd] = x.xs8[(base + 32 * qd) >> 3];
    }
  } else {
    // Q8_0 / Q5_0 / Q5_1: the 32 elements of block u
    ld_words4(x.plane, x.k, 32 * u, r, 0);
    ld_words4(x.plane, x.k, 32 * u + 16, r, 4);
    r.b[0] = x.bsc[u];
    r.s[0] = x.xs16[2 * u] + x.xs16[2 * u + 1];
  }
}

// sum over the unit of x * w (w dequantized), for the unit's fragment
template <int T>
__device__ __forceinline__ float dot_q(const Frag<T>& f, int u, const XU& x);

template <>
__device__ __forceinline__ float dot_q<QT_Q4_K>(const Frag<QT_Q4_K>& f, int u, const XU& x) {
  const int g = (u & 7) >> 1;
  const int q[4] = {(int)f.qs.x, (int)f.qs.y, (int)f.qs.z, (int)f.qs.w};
  int l0 = 0, l1 = 0, l2 = 0, h0 = 0, h1 = 0, h2 = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int wl = q[v] & 0x0f0f0f0f, wh = (q[v] >> 4) & 0x0f0f0f0f;
    l0 = sdot4(wl, x.w[0][v], l0);
    l1 = sdot4(wl, x.w[1][v], l1);
    l2 = sdot4(wl, x.w[2][v], l2);
    h0 = sdot4(wh, x.w[0][4 + v], h0);
    h1 = sdot4(wh, x.w[1][4 + v], h1);
    h2 = sdot4(wh, x.w[2][4 + v], h2);
  }
  const float lo = digits_f(l0, l1, l2) * x.b[0], hi = digits_f(h0, h1, h2) * x.b[1];
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * x.s[0] + (float)m1 * x.s[1]);
}

template <>
__device__ __forceinline__ float dot_q<QT_Q5_K>(const Frag<QT_Q5_K>& f, int u, const XU& x) {
  const int g = (u & 7) >> 1;
  const int q[4] = {(int)f.qs.x, (int)f.qs.y, (int)f.qs.z, (int)f.qs.w};
  const int h[4] = {(int)f.qh.x, (int)f.qh.y, (int)f.qh.z, (int)f.qh.w};
  int l0 = 0, l1 = 0, l2 = 0, h0 = 0, h1 = 0, h2 = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int wl = (q[v] & 0x0f0f0f0f) | (((h[v] >> (2 * g)) & 0x01010101) << 4);
    const int wh = ((q[v] >> 4) & 0x0f0f0f0f) | (((h[v] >> (2 * g + 1)) & 0x01010101) << 4);
    l0 = sdot4(wl, x.w[0][v], l0);
    l1 = sdot4(wl, x.w[1][v], l1);
    l2 = sdot4(wl, x.w[2][v], l2);
    h0 = sdot4(wh, x.w[0][4 + v], h0);
    h1 = sdot4(wh, x.w[1][4 + v], h1);
    h2 = sdot4(wh, x.w[2][4 + v], h2);
  }
  const float lo = digits_f(l0, l1, l2) * x.b[0], hi = digits_f(h0, h1, h2) * x.b[1];
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * x.s[0] + (float)m1 * x.s[1]);
}

template <>
__device__ __forceinline__ float dot_q<QT_Q6_K>(const Frag<QT_Q6_K>& f, int u, const XU& x) {
  // codes 0..63 (the -32 offset is applied through the run sums)
  const int b = (u & 7) & 3;
  const int qa[2] = {(int)f.qa.x, (int)f.qa.y}, qb[2] = {(int)f.qb.x, (int)f.qb.y};
  const int qh[2] = {(int)f.qh.x, (int)f.qh.y};
  float acc = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const int* src = (qd & 1) ? qb : qa;
    const int shift = qd < 2 ? 0 : 4;
    int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int w = ((src[half] >> shift) & 0x0f0f0f0f) | (((qh[half] >> (2 * qd)) & 0x03030303) << 4);
      a0 = sdot4(w, x.w[0][2 * qd + half], a0);
      a1 = sdot4(w, x.w[1][2 * qd + half], a1);
      a2 = sdot4(w, x.w[2][2 * qd + half], a2);
    }
    const float s = digits_f(a0, a1, a2) * x.b[qd] - 32.0f * x.s[qd];
    // sc[8h + (l>>4) + 2qd] with l>>4 == b>>1; f.sc holds sc[8h .. 8h+7]
    const int si = (b >> 1) + 2 * qd;
    const uint32_t sw = si < 4 ? f.sc.x : f.sc.y;
    acc += (float)(int8_t)((sw >> (8 * (si & 3))) & 0xffu) * s;
  }
  return h2f(f.d) * acc;
}

template <>
__device__ __forceinline__ float dot_q<QT_Q8_0>(const Frag<QT_Q8_0>& f, int u, const XU& x) {
  const int q[8] = {(int)f.q0.x, (int)f.q0.y, (int)f.q0.z, (int)f.q0.w,
                    (int)f.q1.x, (int)f.q1.y, (int)f.q1.z, (int)f.q1.w};
  int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    a0 = sdot4(q[v], x.w[0][v], a0);
    a1 = sdot4(q[v], x.w[1][v], a1);
    a2 = sdot4(q[v], x.w[2][v], a2);
  }
  (void)u;
  return h2f(f.d) * (digits_f(a0, a1, a2) * x.b[0]);
}

// Q5_0 / Q5_1 codes 0..31: low nibbles (elements 0..15) and high nibbles
// (16..31) of qs, fifth bit from qh; returns sum(x * code)
__device__ __forceinline__ float dot_q5_codes(const uint4 qs, uint32_t qh, const XU& x) {
  const int q[4] = {(int)qs.x, (int)qs.y, (int)qs.z, (int)qs.w};
  int a0 = 0, a1 = 0, a2 = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    // bits 4v..4v+3 of qh (and 16+4v..) spread to bit 4 of bytes 0..3
    const int hl = (int)((((qh >> (4 * v)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
    const int hh = (int)((((qh >> (16 + 4 * v)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
    const int wl = (q[v] & 0x0f0f0f0f) | hl, wh = ((q[v] >> 4) & 0x0f0f0f0f) | hh;
    a0 = sdot4(wl, x.w[0][v], a0);
    a1 = sdot4(wl, x.w[1][v], a1);
    a2 = sdot4(wl, x.w[2][v], a2);
    a0 = sdot4(wh, x.w[0][4 + v], a0);
    a1 = sdot4(wh, x.w[1][4 + v], a1);
    a2 = sdot4(wh, x.w[2][4 + v], a2);
  }
  return digits_f(a0, a1, a2) * x.b[0];
}

template <>
__device__ __forceinline__ float dot_q<QT_Q5_0>(const Frag<QT_Q5_0>& f, int u, const XU& x) {
  (void)u;
  return h2f(f.d) * (dot_q5_codes(f.qs, f.qh, x) - 16.0f * x.s[0]);
}

template <>
__device__ __forceinline__ float dot_q<QT_Q5_1>(const Frag<QT_Q5_1>& f, int u, const XU& x) {
  (void)u;
  return h2f(f.d) * dot_q5_codes(f.qs, f.qh, x) + h2f(f.m) * x.s[0];
}

// ---- fp32 activation form (decode row kernels) ----------------------------------
// The row kernels keep x in fp32 and skip the integer-digit conversion, whose
// per-workgroup cost (every workgroup converts the whole vector) dominates a
// decode matvec. Layout in LDS, U = K/32 units, unit-local element order
// e = 0..31 as in unit_col:
//   X[v * U + u]  float4: elements 4v .. 4v+3 of unit u (v = 0..7)
//   S[u]          float4: sums of x over the unit's 8-element runs e in [8k, 8k+8)
// Lanes of a row group read consecutive units, so every 16-byte LDS read of a
// wave touches consecutive slots. The sums give each type's factored offset
// term (Q4_K/Q5_K halves, Q6_K quarters, Q8_0/Q5_x whole blocks).

// Unit u and unit-local element e of row column c (inverse of unit_col).
template <int T>
__device__ __forceinline__ void unit_of_col(int c, int& u, int& e) {
  if constexpr (T == QT_Q4_K || T == QT_Q5_K) {
    const int r = c & 255, r2 = r & 63, r3 = r2 & 31;
    u = (c >> 8) * 8 + 2 * (r >> 6) + (r3 >> 4);
    e = (r2 >> 5) * 16 + (r3 & 15);
  } else if constexpr (T == QT_Q6_K) {
    const int r = c & 255, r2 = r & 127, r3 = r2 & 31;
    u = (c >> 8) * 8 + 4 * (r >> 7) + (r3 >> 3);
    e = 8 * (r2 >> 5) + (r3 & 7);
  } else {
    u = c >> 5;
    e = c & 31;
  }
}

// x for one unit: the eight float4 and the four run sums.
struct XF {
  float4 x[8];
  float4 s;
};

__device__ __forceinline__ void load_xf(const float4* X, const float4* S, int U, int u, XF& r) {
#pragma unroll
  for (int v = 0; v < 8; ++v) r.x[v] = X[v * U + u];
  r.s = S[u];
}

__device__ __forceinline__ float ub(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ float sb(uint32_t w, int i) { return (float)(int)(int8_t)((w >> (8 * i)) & 0xffu); }
__device__ __forceinline__ float dot4u(float4 a, uint32_t w) {
  return (a.x * ub(w, 0) + a.y * ub(w, 1)) + (a.z * ub(w, 2) + a.w * ub(w, 3));
}

// sum over the unit of x * w (w dequantized) in fp32, factored as the
// integer-digit dot_q: d * sc * sum(x * q) - dmin * m * sum(x) and the like.
template <int T>
__device__ __forceinline__ float dot_f(const Frag<T>& f, int u, const XF& x);

template <>
__device__ __forceinline__ float dot_f<QT_Q4_K>(const Frag<QT_Q4_K>& f, int u, const XF& x) {
  const int g = (u & 7) >> 1;
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    lo += dot4u(x.x[v], q[v] & 0x0f0f0f0fu);
    hi += dot4u(x.x[4 + v], (q[v] >> 4) & 0x0f0f0f0fu);
  }
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * (x.s.x + x.s.y) + (float)m1 * (x.s.z + x.s.w));
}

template <>
__device__ __forceinline__ float dot_f<QT_Q5_K>(const Frag<QT_Q5_K>& f, int u, const XF& x) {
  const int g = (u & 7) >> 1;
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  const uint32_t h[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t wl = (q[v] & 0x0f0f0f0fu) | (((h[v] >> (2 * g)) & 0x01010101u) << 4);
    const uint32_t wh = ((q[v] >> 4) & 0x0f0f0f0fu) | (((h[v] >> (2 * g + 1)) & 0x01010101u) << 4);
    lo += dot4u(x.x[v], wl);
    hi += dot4u(x.x[4 + v], wh);
  }
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * (x.s.x + x.s.y) + (float)m1 * (x.s.z + x.s.w));
}

template <>
__device__ __forceinline__ float dot_f<QT_Q6_K>(const Frag<QT_Q6_K>& f, int u, const XF& x) {
  // codes 0..63, the -32 offset through the run sums
  const int b = u & 3;
  const uint32_t qa[2] = {f.qa.x, f.qa.y}, qb[2] = {f.qb.x, f.qb.y}, qh[2] = {f.qh.x, f.qh.y};
  const float sr[4] = {x.s.x, x.s.y, x.s.z, x.s.w};
  float acc = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const uint32_t* src = (qd & 1) ? qb : qa;
    const int shift = qd < 2 ? 0 : 4;
    float s = 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t w = ((src[half] >> shift) & 0x0f0f0f0fu) | (((qh[half] >> (2 * qd)) & 0x03030303u) << 4);
      s += dot4u(x.x[2 * qd + half], w);
    }
    s -= 32.0f * sr[qd];
    const int si = (b >> 1) + 2 * qd;
    const uint32_t sw = si < 4 ? f.sc.x : f.sc.y;
    acc += (float)(int8_t)((sw >> (8 * (si & 3))) & 0xffu) * s;
  }
  return h2f(f.d) * acc;
}

template <>
__device__ __forceinline__ float dot_f<QT_Q8_0>(const Frag<QT_Q8_0>& f, int u, const XF& x) {
  const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int v = 0; v < 8; v += 2) {
    a0 += (x.x[v].x * sb(q[v], 0) + x.x[v].y * sb(q[v], 1)) + (x.x[v].z * sb(q[v], 2) + x.x[v].w * sb(q[v], 3));
    a1 += (x.x[v + 1].x * sb(q[v + 1], 0) + x.x[v + 1].y * sb(q[v + 1], 1)) +
          (x.x[v + 1].z * sb(q[v + 1], 2) + x.x[v + 1].w * sb(q[v + 1], 3));
  }
  (void)u;
  return h2f(f.d) * (a0 + a1);
}

// Q5_0 / Q5_1 codes 0..31 (fifth bit from qh): sum(x * code)
__device__ __forceinline__ float dot_q5f_codes(const uint4 qs, uint32_t qh, const XF& x) {
  const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const uint32_t hl = ((((qh >> (4 * v)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
    const uint32_t hh = ((((qh >> (16 + 4 * v)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
    lo += dot4u(x.x[v], (q[v] & 0x0f0f0f0fu) | hl);
    hi += dot4u(x.x[4 + v], ((q[v] >> 4) & 0x0f0f0f0fu) | hh);
  }
  return lo + hi;
}

template <>
__device__ __forceinline__ float dot_f<QT_Q5_0>(const Frag<QT_Q5_0>& f, int u, const XF& x) {
  (void)u;
  const float s = (x.s.x + x.s.y) + (x.s.z + x.s.w);
  return h2f(f.d) * (dot_q5f_codes(f.qs, f.qh, x) - 16.0f * s);
}

template <>
__device__ __forceinline__ float dot_f<QT_Q5_1>(const Frag<QT_Q5_1>& f, int u, const XF& x) {
  (void)u;
  const float s = (x.s.x + x.s.y) + (x.s.z + x.s.w);
  return h2f(f.d) * dot_q5f_codes(f.qs, f.qh, x) + h2f(f.m) * s;
}

// acc + sum over unit c of a super-block (any unit for Q8_0) of x * w for the
// row-per-lane lm_head. x is in the unit-major layout XU[u * 9 + v] (float4 v
// = elements 4v .. 4v+3 of unit u in the unit's own element order, then the
// four 8-element run sums), so that every lane of a wave reads the same
// 144-byte unit (broadcast reads). The dot_f arithmetic as one fma chain per
// run (4 cvt + 4 fma per 4 weights).
template <int T>
__device__ __forceinline__ float acc_lane(const LaneFrag<T>& f, const LaneHead<T>& h, int c, const float4* xu,
                                          float acc);

__device__ __forceinline__ float fma4u(float4 a, uint32_t w, float s) {
  s = fmaf(a.x, ub(w, 0), s);
  s = fmaf(a.y, ub(w, 1), s);
  s = fmaf(a.z, ub(w, 2), s);
  return fmaf(a.w, ub(w, 3), s);
}

__device__ __forceinline__ uint32_t word4(const uint4 v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

template <>
__device__ __forceinline__ float acc_lane<QT_Q6_K>(const LaneFrag<QT_Q6_K>& f, const LaneHead<QT_Q6_K>& h, int c,
                                                   const float4* xu, float acc) {
  // unit c: half hh = c / 4, run b = c % 4; scale byte 8 hh + (b >> 1) + 2 qd
  const int hh = c >> 2, b = c & 3;
  const float4 s4 = xu[8];
  const float sr[4] = {s4.x, s4.y, s4.z, s4.w};
  const uint32_t qa[2] = {f.ql.x, f.ql.y}, qb[2] = {f.ql.z, f.ql.w}, qh[2] = {f.qh.x, f.qh.y};
  float su = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const uint32_t* src = (qd & 1) ? qb : qa;
    const int shift = qd < 2 ? 0 : 4;
    float s = -32.0f * sr[qd];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t w = ((src[half] >> shift) & 0x0f0f0f0fu) | (((qh[half] >> (2 * qd)) & 0x03030303u) << 4);
      s = fma4u(xu[2 * qd + half], w, s);
    }
    const int si = 8 * hh + (b >> 1) + 2 * qd;
    su = fmaf((float)(int8_t)((word4(h.sc, si >> 2) >> (8 * (si & 3))) & 0xffu), s, su);
  }
  return fmaf(h2f(h.d), su, acc);
}

template <>
__device__ __forceinline__ float acc_lane<QT_Q8_0>(const LaneFrag<QT_Q8_0>& f, const LaneHead<QT_Q8_0>& h, int c,
                                                   const float4* xu, float acc) {
  (void)h;
  (void)c;
  const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const float4 a = xu[v];
    s = fmaf(a.x, sb(q[v], 0), s);
    s = fmaf(a.y, sb(q[v], 1), s);
    s = fmaf(a.z, sb(q[v], 2), s);
    s = fmaf(a.w, sb(q[v], 3), s);
  }
  return fmaf(h2f(f.d), s, acc);
}

template <>
__device__ __forceinline__ float acc_lane<QT_Q4_K>(const LaneFrag<QT_Q4_K>& f, const LaneHead<QT_Q4_K>& h, int c,
                                                   const float4* xu, float acc) {
  const int g = c >> 1;
  const float4 s4 = xu[8];
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    lo = fma4u(xu[v], q[v] & 0x0f0f0f0fu, lo);
    hi = fma4u(xu[4 + v], (q[v] >> 4) & 0x0f0f0f0fu, hi);
  }
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, h.hdr.y, h.hdr.z, h.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, h.hdr.y, h.hdr.z, h.hdr.w, &sc1, &m1);
  const float d = h2f(h.hdr.x), dmin = h2f(h.hdr.x >> 16);
  const float pos = fmaf((float)sc1, hi, (float)sc0 * lo);
  const float neg = fmaf((float)m1, s4.z + s4.w, (float)m0 * (s4.x + s4.y));
  return fmaf(d, pos, fmaf(-dmin, neg, acc));
}

// ---- exact dequantization ------------------------------------------------------
// out[e] for unit-local element e (placement per unit_col), computed with the
// reference's fp32 operation order and no contraction. `pow2` (a power of two)
// scales the unit's factors, which scales every result exactly: out[e] is the
// unscaled value times pow2 bit for bit (normal-range values).
template <int T>
__device__ __forceinline__ void dequant_unit(const Frag<T>& f, int u, float out[32], float pow2 = 1.0f);

template <>
__device__ __forceinline__ void dequant_unit<QT_Q4_K>(const Frag<QT_Q4_K>& f, int u, float out[32], float pow2) {
  const int g = (u & 7) >> 1;
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x) * pow2, dmin = h2f(f.hdr.x >> 16) * pow2;
  const float a0 = __fmul_rn(d, (float)sc0), b0 = __fmul_rn(dmin, (float)m0);
  const float a1 = __fmul_rn(d, (float)sc1), b1 = __fmul_rn(dmin, (float)m1);
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    out[e] = __fsub_rn(__fmul_rn(a0, nib_lo(q[e >> 2], e & 3)), b0);
    out[16 + e] = __fsub_rn(__fmul_rn(a1, nib_hi(q[e >> 2], e & 3)), b1);
  }
}

template <>
__device__ __forceinline__ void dequant_unit<QT_Q5_K>(const Frag<QT_Q5_K>& f, int u, float out[32], float pow2) {
  const int g = (u & 7) >> 1;
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x) * pow2, dmin = h2f(f.hdr.x >> 16) * pow2;
  const float a0 = __fmul_rn(d, (float)sc0), b0 = __fmul_rn(dmin, (float)m0);
  const float a1 = __fmul_rn(d, (float)sc1), b1 = __fmul_rn(dmin, (float)m1);
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  const uint32_t h[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const uint32_t qb = (q[e >> 2] >> (8 * (e & 3))) & 0xffu;
    const uint32_t hb = (h[e >> 2] >> (8 * (e & 3))) & 0xffu;
    const uint32_t ql = (qb & 15u) + (((hb >> (2 * g)) & 1u) << 4);
    const uint32_t qhh = (qb >> 4) + (((hb >> (2 * g + 1)) & 1u) << 4);
    out[e] = __fsub_rn(__fmul_rn(a0, (float)ql), b0);
    out[16 + e] = __fsub_rn(__fmul_rn(a1, (float)qhh), b1);
  }
}

template <>
__device__ __forceinline__ void dequant_unit<QT_Q6_K>(const Frag<QT_Q6_K>& f, int u, float out[32], float pow2) {
  const int b = (u & 7) & 3;
  const float d = h2f(f.d) * pow2;
  const uint32_t qa[2] = {f.qa.x, f.qa.y}, qb[2] = {f.qb.x, f.qb.y}, qh[2] = {f.qh.x, f.qh.y};
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const int si = (b >> 1) + 2 * qd;
    const uint32_t sw = si < 4 ? f.sc.x : f.sc.y;
    const float ds = __fmul_rn(d, (float)(int8_t)((sw >> (8 * (si & 3))) & 0xffu));
    const uint32_t* src = (qd & 1) ? qb : qa;
    const int shift = qd < 2 ? 0 : 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lo = (src[i >> 2] >> (8 * (i & 3) + shift)) & 15u;
      const uint32_t hb = (qh[i >> 2] >> (8 * (i & 3) + 2 * qd)) & 3u;
      out[8 * qd + i] = __fmul_rn(ds, (float)((int)(lo | (hb << 4)) - 32));
    }
  }
}

template <>
__device__ __forceinline__ void dequant_unit<QT_Q8_0>(const Frag<QT_Q8_0>& f, int u, float out[32], float pow2) {
  const float d = h2f(f.d) * pow2;
  const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
#pragma unroll
  for (int e = 0; e < 32; ++e) out[e] = __fmul_rn((float)(int8_t)((q[e >> 2] >> (8 * (e & 3))) & 0xffu), d);
}

template <int T, typename F>
__device__ __forceinline__ void dequant_q5x(const F& f, float out[32], float pow2) {
  const float d = h2f(f.d) * pow2;
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const int j = e & 15;
    const uint32_t qb = (q[j >> 2] >> (8 * (j & 3))) & 0xffu;
    const uint32_t low4 = e >= 16 ? qb >> 4 : qb & 15u;
    const uint32_t qv = low4 | (((f.qh >> e) & 1u) << 4);
    if constexpr (T == QT_Q5_0) {
      out[e] = __fmul_rn(d, (float)((int)qv - 16));
    } else {
      out[e] = __fadd_rn(__fmul_rn(d, (float)qv), h2f(f.m) * pow2);
    }
  }
}

template <>
__device__ __forceinline__ void dequant_unit<QT_Q5_0>(const Frag<QT_Q5_0>& f, int u, float out[32], float pow2) {
  dequant_q5x<QT_Q5_0>(f, out, pow2);
}
template <>
__device__ __forceinline__ void dequant_unit<QT_Q5_1>(const Frag<QT_Q5_1>& f, int u, float out[32], float pow2) {
  dequant_q5x<QT_Q5_1>(f, out, pow2);
}

// Dispatch helper: calls fn.template operator()<T>() for the runtime type.
template <typename Fn>
__device__ __forceinline__ void with_type(int type, Fn&& fn) {
  switch (type) {
    case QT_Q4_K: fn.template operator()<QT_Q4_K>(); break;
    case QT_Q6_K: fn.template operator()<QT_Q6_K>(); break;
    case QT_Q8_0: fn.template operator()<QT_Q8_0>(); break;
    case QT_Q5_0: fn.template operator()<QT_Q5_0>(); break;
    case QT_Q5_1: fn.template operator()<QT_Q5_1>(); break;
    case QT_Q5_K: fn.template operator()<QT_Q5_K>(); break;
    default: break;
  }
}

}  // namespace chonk
