// Per-type 32-element unit decode for the striped layout (device_common.h).
//
// For every GGUF type there is
//   * Frag<T>            the raw bytes of one unit (loaded with vector loads),
//   * load_unit<T>()     issues the loads for (row, unit),
//   * dot_unit<T>()      sum_i x[k_i] * w_i over the unit's 32 elements,
//   * dequant_unit<T>()  the 32 weights, bit-exact with the reference decode.
//
// Element placement inside a unit, and the exact fp32 operation order used by
// dequant_unit, follow the reference's WGSL weight helpers
// (src/lib/llama-wgsl-runtime.ts: q5_0 :2230-2246, q5_1 :2280-2289,
// q8_0 :2321-2327, q4_k :2378-2410, q5_k :2479-2495, q6_k :2560-2580), which
// in turn follow llama.cpp's dequantize_row_* block formats. dot_unit uses the
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

// ---- dot products ------------------------------------------------------------
// xs: activations in LDS; xs16: sums of xs over aligned 16-element runs.
template <int T>
__device__ __forceinline__ float dot_unit(const Frag<T>& f, int u, const float* xs, const float* xs16);

template <>
__device__ __forceinline__ float dot_unit<QT_Q4_K>(const Frag<QT_Q4_K>& f, int u, const float* xs,
                                                   const float* xs16) {
  const int sb = u >> 3, c = u & 7, g = c >> 1, hh = c & 1;
  const int base = sb * 256 + 64 * g + 16 * hh;
  const float4* xl = (const float4*)(xs + base);
  const float4* xh = (const float4*)(xs + base + 32);
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float4 a = xl[v], b = xh[v];
    lo += a.x * nib_lo(q[v], 0) + a.y * nib_lo(q[v], 1) + a.z * nib_lo(q[v], 2) + a.w * nib_lo(q[v], 3);
    hi += b.x * nib_hi(q[v], 0) + b.y * nib_hi(q[v], 1) + b.z * nib_hi(q[v], 2) + b.w * nib_hi(q[v], 3);
  }
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  const float s_lo = xs16[base >> 4], s_hi = xs16[(base >> 4) + 2];
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * s_lo + (float)m1 * s_hi);
}

template <>
__device__ __forceinline__ float dot_unit<QT_Q5_K>(const Frag<QT_Q5_K>& f, int u, const float* xs,
                                                   const float* xs16) {
  const int sb = u >> 3, c = u & 7, g = c >> 1, hh = c & 1;
  const int base = sb * 256 + 64 * g + 16 * hh;
  const float4* xl = (const float4*)(xs + base);
  const float4* xh = (const float4*)(xs + base + 32);
  const uint32_t q[4] = {f.qs.x, f.qs.y, f.qs.z, f.qs.w};
  const uint32_t h[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
  float lo = 0.f, hi = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float4 a = xl[v], b = xh[v];
    float ql[4], qhv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hb = (h[v] >> (8 * i)) & 0xffu;
      ql[i] = (float)(((q[v] >> (8 * i)) & 15u) + (((hb >> (2 * g)) & 1u) << 4));
      qhv[i] = (float)(((q[v] >> (8 * i + 4)) & 15u) + (((hb >> (2 * g + 1)) & 1u) << 4));
    }
    lo += a.x * ql[0] + a.y * ql[1] + a.z * ql[2] + a.w * ql[3];
    hi += b.x * qhv[0] + b.y * qhv[1] + b.z * qhv[2] + b.w * qhv[3];
  }
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
  const float s_lo = xs16[base >> 4], s_hi = xs16[(base >> 4) + 2];
  return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * s_lo + (float)m1 * s_hi);
}

template <>
__device__ __forceinline__ float dot_unit<QT_Q6_K>(const Frag<QT_Q6_K>& f, int u, const float* xs,
                                                   const float* xs16) {
  const int sb = u >> 3, c = u & 7, h = c >> 2, b = c & 3;
  const int base = sb * 256 + 128 * h + 8 * b;
  const uint32_t qa[2] = {f.qa.x, f.qa.y}, qb[2] = {f.qb.x, f.qb.y}, qh[2] = {f.qh.x, f.qh.y};
  float acc = 0.f;
#pragma unroll
  for (int qd = 0; qd < 4; ++qd) {
    const uint32_t* src = (qd & 1) ? qb : qa;
    const int shift = qd < 2 ? 0 : 4;
    const float4* xv = (const float4*)(xs + base + 32 * qd);
    float s = 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const float4 x4 = xv[half];
      const uint32_t lo = src[half] >> shift, hb = qh[half] >> (2 * qd);
      const float q0 = (float)((int)(((lo >> 0) & 15u) | (((hb >> 0) & 3u) << 4)) - 32);
      const float q1 = (float)((int)(((lo >> 8) & 15u) | (((hb >> 8) & 3u) << 4)) - 32);
      const float q2 = (float)((int)(((lo >> 16) & 15u) | (((hb >> 16) & 3u) << 4)) - 32);
      const float q3 = (float)((int)(((lo >> 24) & 15u) | (((hb >> 24) & 3u) << 4)) - 32);
      s += x4.x * q0 + x4.y * q1 + x4.z * q2 + x4.w * q3;
    }
    // sc[8h + (l>>4) + 2qd] with l>>4 == b>>1; f.sc holds sc[8h .. 8h+7]
    const int si = (b >> 1) + 2 * qd;
    const uint32_t sw = si < 4 ? f.sc.x : f.sc.y;
    const float scv = (float)(int8_t)((sw >> (8 * (si & 3))) & 0xffu);
    acc += scv * s;
  }
  (void)xs16;
  return h2f(f.d) * acc;
}

template <>
__device__ __forceinline__ float dot_unit<QT_Q8_0>(const Frag<QT_Q8_0>& f, int u, const float* xs,
                                                   const float* xs16) {
  const float4* xv = (const float4*)(xs + 32 * u);
  const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const float4 a = xv[v];
    s += a.x * (float)(int8_t)(q[v] & 0xffu) + a.y * (float)(int8_t)((q[v] >> 8) & 0xffu) +
         a.z * (float)(int8_t)((q[v] >> 16) & 0xffu) + a.w * (float)(int8_t)(q[v] >> 24);
  }
  (void)xs16;
  return h2f(f.d) * s;
}

template <int T>
__device__ __forceinline__ float dot_q5x(const uint4 qs, uint32_t qh, int u, const float* xs) {
  const float4* xv = (const float4*)(xs + 32 * u);
  const uint32_t q[4] = {qs.x, qs.y, qs.z, qs.w};
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const float4 a = xv[v], b = xv[v + 4];
    float lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * v + i;
      lo[i] = (float)((int)(((q[v] >> (8 * i)) & 15u) | (((qh >> j) & 1u) << 4)) - (T == QT_Q5_0 ? 16 : 0));
      hi[i] = (float)((int)(((q[v] >> (8 * i + 4)) & 15u) | (((qh >> (j + 16)) & 1u) << 4)) - (T == QT_Q5_0 ? 16 : 0));
    }
    s += a.x * lo[0] + a.y * lo[1] + a.z * lo[2] + a.w * lo[3];
    s += b.x * hi[0] + b.y * hi[1] + b.z * hi[2] + b.w * hi[3];
  }
  return s;
}

template <>
__device__ __forceinline__ float dot_unit<QT_Q5_0>(const Frag<QT_Q5_0>& f, int u, const float* xs,
                                                   const float* xs16) {
  (void)xs16;
  return h2f(f.d) * dot_q5x<QT_Q5_0>(f.qs, f.qh, u, xs);
}

template <>
__device__ __forceinline__ float dot_unit<QT_Q5_1>(const Frag<QT_Q5_1>& f, int u, const float* xs,
                                                   const float* xs16) {
  const float sx = xs16[2 * u] + xs16[2 * u + 1];
  return h2f(f.d) * dot_q5x<QT_Q5_1>(f.qs, f.qh, u, xs) + h2f(f.m) * sx;
}

// ---- exact dequantization ------------------------------------------------------
// out[e] for unit-local element e (placement per unit_col), computed with the
// reference's fp32 operation order and no contraction.
template <int T>
__device__ __forceinline__ void dequant_unit(const Frag<T>& f, int u, float out[32]);

template <>
__device__ __forceinline__ void dequant_unit<QT_Q4_K>(const Frag<QT_Q4_K>& f, int u, float out[32]) {
  const int g = (u & 7) >> 1;
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
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
__device__ __forceinline__ void dequant_unit<QT_Q5_K>(const Frag<QT_Q5_K>& f, int u, float out[32]) {
  const int g = (u & 7) >> 1;
  uint32_t sc0, m0, sc1, m1;
  scale_min(2 * g, f.hdr.y, f.hdr.z, f.hdr.w, &sc0, &m0);
  scale_min(2 * g + 1, f.hdr.y, f.hdr.z, f.hdr.w, &sc1, &m1);
  const float d = h2f(f.hdr.x), dmin = h2f(f.hdr.x >> 16);
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
__device__ __forceinline__ void dequant_unit<QT_Q6_K>(const Frag<QT_Q6_K>& f, int u, float out[32]) {
  const int b = (u & 7) & 3;
  const float d = h2f(f.d);
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
__device__ __forceinline__ void dequant_unit<QT_Q8_0>(const Frag<QT_Q8_0>& f, int u, float out[32]) {
  const float d = h2f(f.d);
  const uint32_t q[8] = {f.q0.x, f.q0.y, f.q0.z, f.q0.w, f.q1.x, f.q1.y, f.q1.z, f.q1.w};
#pragma unroll
  for (int e = 0; e < 32; ++e) out[e] = __fmul_rn((float)(int8_t)((q[e >> 2] >> (8 * (e & 3))) & 0xffu), d);
}

template <int T, typename F>
__device__ __forceinline__ void dequant_q5x(const F& f, float out[32]) {
  const float d = h2f(f.d);
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
      out[e] = __fadd_rn(__fmul_rn(d, (float)qv), h2f(f.m));
    }
  }
}

template <>
__device__ __forceinline__ void dequant_unit<QT_Q5_0>(const Frag<QT_Q5_0>& f, int u, float out[32]) {
  dequant_q5x<QT_Q5_0>(f, out);
}
template <>
__device__ __forceinline__ void dequant_unit<QT_Q5_1>(const Frag<QT_Q5_1>& f, int u, float out[32]) {
  dequant_q5x<QT_Q5_1>(f, out);
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
