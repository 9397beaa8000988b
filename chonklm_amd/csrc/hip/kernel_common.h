// Device helpers shared by the decode kernels (kernels.hip, attn_decode.hip, prefill.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.h"
#include "qdot.h"

// Optional trace point inside the attention phases (k = 1, 2, 3 after B, C, D);
// empty unless a profiling build defines it.
#ifndef CHONK_ATTN_STAMP
#define CHONK_ATTN_STAMP(k)
#endif
// Optional trace points of the matvec kernels: CHONK_MV_T(tr, k) records phase
// k of this workgroup into the uint64_t tr[8], CHONK_MV_TRACE_END(tr, tag)
// publishes them; both empty unless a profiling build defines them.
#ifndef CHONK_MV_T
#define CHONK_MV_T(tr, k) (void)(tr)
#endif
#ifndef CHONK_MV_TRACE_END
#define CHONK_MV_TRACE_END(tr, tag) (void)(tr)
#endif

namespace chonk {
namespace {

constexpr float kNegBig = -3.402823e38f;  // the WGSL literal -3.402823e38

// Touches every 64-byte line of the kernel arguments' first BYTES bytes with
// one round of scalar loads (awaited once), so that the argument loads that
// depend on each other (a segment's fields after the segment index) find their
// lines in the scalar cache instead of each round going to memory.
template <int BYTES>
__device__ __forceinline__ void warm_kernarg() {
  static_assert(BYTES <= 16 * 64, "at most 16 lines");
  const uint32_t* ka = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  uint32_t v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = i * 64 < BYTES ? ld_scalar(ka + i * 16) : 0u;
  asm volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]), "s"(v[8]),
               "s"(v[9]), "s"(v[10]), "s"(v[11]), "s"(v[12]), "s"(v[13]), "s"(v[14]), "s"(v[15]));
  __builtin_amdgcn_sched_barrier(0);
}


// Cross-lane steps without the LDS crossbar: DPP quad/row permutations inside
// 16-lane rows, then gfx950's permlane swaps across the rows of a 32-lane half
// (v_permlane16_swap) and across the halves (v_permlane32_swap) — VALU ops,
// where a ds_swizzle would take a trip through the LDS unit. Every lane of an
// aligned group of N lanes ends with the same value. Lanes of a group must be
// active together.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
}
// (a, b) = (v of this lane, v of lane ^ 16) and (v of this lane, v of lane ^ 32)
// as the two halves of one swap (each lane receives both)
__device__ __forceinline__ void swap16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float lane_of(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (N >= 2) v += dpp<0xb1>(v);   // quad_perm 1,0,3,2
  if constexpr (N >= 4) v += dpp<0x4e>(v);   // quad_perm 2,3,0,1
  if constexpr (N >= 8) v += dpp<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp<0x140>(v); // row_mirror
  if constexpr (N >= 32) {
    float a, b;
    swap16(v, a, b);
    v = a + b;
  }
  if constexpr (N >= 64) {
    float a, b;
    swap32(v, a, b);
    v = a + b;
  }
  return v;
}
template <int N>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (N >= 2) v = fmaxf(v, dpp<0xb1>(v));
  if constexpr (N >= 4) v = fmaxf(v, dpp<0x4e>(v));
  if constexpr (N >= 8) v = fmaxf(v, dpp<0x141>(v));
  if constexpr (N >= 16) v = fmaxf(v, dpp<0x140>(v));
  if constexpr (N >= 32) {
    float a, b;
    swap16(v, a, b);
    v = fmaxf(a, b);
  }
  if constexpr (N >= 64) {
    float a, b;
    swap32(v, a, b);
    v = fmaxf(a, b);
  }
  return v;
}
// runtime group width (power of two in [1, 64])
__device__ __forceinline__ float group_sum_n(float v, int n) {
  switch (n) {
    case 2: return group_sum<2>(v);
    case 4: return group_sum<4>(v);
    case 8: return group_sum<8>(v);
    case 16: return group_sum<16>(v);
    case 32: return group_sum<32>(v);
    case 64: return group_sum<64>(v);
    default: return v;
  }
}
__device__ __forceinline__ float group_max_n(float v, int n) {
  switch (n) {
    case 2: return group_max<2>(v);
    case 4: return group_max<4>(v);
    case 8: return group_max<8>(v);
    case 16: return group_max<16>(v);
    case 32: return group_max<32>(v);
    case 64: return group_max<64>(v);
    default: return v;
  }
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

// Sum over the position groups of a wave whose lanes are (group, dim pair):
// lanes that differ only in the bits at and above log2(DW) (DW = 8 or 16
// lanes per group). Every lane ends with its dim pair's total.
template <int DW>
__device__ __forceinline__ float pg_sum(float v) {
  if constexpr (DW <= 8) v += dpp<0x128>(v);  // row_ror:8 = lane ^ 8 inside a 16-lane row
  float a, b;
  swap16(v, a, b);
  v = a + b;
  swap32(v, a, b);
  return a + b;
}

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// Sum over the 256 threads; red must hold 4 floats. Callable repeatedly.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  if (v != v) return false;
  if (bv != bv) return true;
  return (v > bv) || ((v == bv) && (i < bi));
}

__device__ __forceinline__ bool bit_test(const uint32_t* bits, uint32_t id) {
  return (*gbl(bits + (id >> 5)) >> (id & 31u)) & 1u;
}

__device__ __forceinline__ void st_relaxed(float* p, float v) {
  __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_relaxed(const float* p) {
  return __uint_as_float(__hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  if (x != x) return 0.0f;
  if (x > 10.0f) return x;
  if (x < -10.0f) return 0.0f;
  const float c = 0.7978845608028654f;
  const float cube = __fmul_rn(__fmul_rn(__fmul_rn(0.044715f, x), x), x);
  const float t = __fadd_rn(1.0f, tanhf(__fmul_rn(c, __fadd_rn(x, cube))));
  return __fmul_rn(__fmul_rn(0.5f, x), t);
}

// ---------------------------------------------------------------------------
// matvec: activation staging, weight streaming, epilogues.

typedef __attribute__((address_space(1))) void gmem_void;
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate that waits until at most n vector memory operations of
// the wave are outstanding (gfx9 encoding: vmcnt bits 3:0 and 15:14; expcnt
// and lgkmcnt left at their maxima, i.e. not waited for).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// A workgroup barrier that orders LDS accesses only: no wait for the global
// loads in flight (__syncthreads waits for every outstanding memory access).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Copies n floats from global memory into LDS with the CDNA3/4 direct-to-LDS
// loads (16 bytes per lane, no registers); completion is awaited with
// s_waitcnt vmcnt(0) + a barrier by the caller.
__device__ __forceinline__ void lds_dma(const float* src, float* dst, int n) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int base = wave * 256; base < n; base += 4 * 256) {
    const int idx = base + lane * 4;
    if (idx < n) __builtin_amdgcn_global_load_lds((gmem_void*)(src + idx), (lds_void*)(dst + base), 16, 0, 0);
  }
}

// One matvec segment as a kernel sees it (fields picked individually from the
// argument block).
struct SegView {
  QMat w;
  const uint8_t *u0, *u1, *u2, *u3;  // GLU up-matrix streams
  float* out;
  const float* add;
  const float* bias;
  int n_out, tile, lpr, wg_begin, tag_div;
};

// ---- matvec core (k_mv_*) -----------------------------------------------

// LDS of the integer-digit form of x at `base`: three digit planes of K bytes,
// then bsc[K/32] and xs8[K/8] (3.625 K bytes in all); xs16[K/16] lies apart.
__device__ __forceinline__ XqView xq_view(void* base, float* xs16, int K) {
  XqView v;
  v.plane = (const int8_t*)base;
  v.bsc = (const float*)((char*)base + 3 * K);
  v.xs8 = v.bsc + K / 32;
  v.xs16 = xs16;
  v.k = K;
  return v;
}

// Digit planes, block scale and run sums of the four elements 4*i4 .. 4*i4+3
// of x. The 8 consecutive threads that hold one 32-element block call it
// together (their lanes must be active together).
__device__ __forceinline__ void quantize4(const float4 v, int i4, int K, void* base, float* xs16) {
  int8_t* plane = (int8_t*)base;
  float* bsc = (float*)((char*)base + 3 * K);
  float* xs8 = bsc + K / 32;
  {
    const float m = group_max<8>(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    int e = 0;
    (void)frexpf(m, &e);  // m < 2^e, so |x| * 2^(22-e) < 2^22
    const int sh = min(22 - e, 126);
    const float vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = (int)rintf(ldexpf(vv[i], sh));
      const int d0 = (int)(int8_t)q;
      const int r1 = (q - d0) >> 8;
      const int d1 = (int)(int8_t)r1;
      const int d2 = (r1 - d1) >> 8;  // |d2| <= 65
      w0 |= ((uint32_t)d0 & 255u) << (8 * i);
      w1 |= ((uint32_t)d1 & 255u) << (8 * i);
      w2 |= ((uint32_t)d2 & 255u) << (8 * i);
    }
    reinterpret_cast<uint32_t*>(plane)[i4] = w0;
    reinterpret_cast<uint32_t*>(plane + K)[i4] = w1;
    reinterpret_cast<uint32_t*>(plane + 2 * K)[i4] = w2;
    const float s4 = (v.x + v.y) + (v.z + v.w);
    const float s8 = s4 + dpp<0xb1>(s4);
    const float s16 = s8 + dpp<0x4e>(s8);
    if ((i4 & 1) == 0) xs8[i4 >> 1] = s8;
    if ((i4 & 3) == 0) xs16[i4 >> 2] = s16;
    // a non-finite block poisons its products as the fp32 sum would
    if ((i4 & 7) == 0) bsc[i4 >> 3] = __builtin_isfinite(m) ? ldexpf(1.0f, -sh) : __int_as_float(0x7fc00000);
  }
}

// Fills the digit planes, block scales and run sums of x (fp32 in LDS, K a
// multiple of 32). Called by all threads after a barrier that follows the last
// write of x; a barrier must separate it from the first read of the planes.
__device__ __forceinline__ void quantize_x(const float* xs, int K, void* base, float* xs16) {
  // 8 consecutive threads cover one 32-element block (K / 4 is a multiple of 8)
  for (int i4 = threadIdx.x; i4 < (K >> 2); i4 += kWg)
    quantize4(reinterpret_cast<const float4*>(xs)[i4], i4, K, base, xs16);
}

// Stores elements 4*i4 .. 4*i4+3 of x into the fp32 unit layout of type T
// (qdot.h: X[v * U + u], run sums S[u]). Lane pairs hold consecutive i4 (the
// caller's threads cover i4 in order, K a multiple of 32), and both lanes of a
// pair call it together: the even lane stores the pair's 8-element sum.
template <int T>
__device__ __forceinline__ void xf_put(const float4 v, int i4, int U, float4* X, float* S) {
  int u, e;
  unit_of_col<T>(4 * i4, u, e);
  X[(e >> 2) * U + u] = v;
  const float s4 = (v.x + v.y) + (v.z + v.w);
  const float s8 = s4 + dpp<0xb1>(s4);
  if ((i4 & 1) == 0) S[4 * u + (e >> 3)] = s8;
}

// The same from the fp32 vector xs[K] in LDS. All threads call it after a
// barrier that follows the last write of xs; a barrier must separate it from
// the first read of X / S.
template <int T>
__device__ __forceinline__ void xf_build(const float* xs, int K, float4* X, float* S) {
  for (int i4 = threadIdx.x; i4 < (K >> 2); i4 += kWg) xf_put<T>(reinterpret_cast<const float4*>(xs)[i4], i4, K >> 5, X, S);
}

// The same into the unit-major layout of the row-per-lane lm_head (qdot.h,
// acc_lane): XU[u * 9 + v] = float4 v of unit u, XU[u * 9 + 8] = its run sums.
template <int T>
__device__ __forceinline__ void xu_build(const float* xs, int K, float4* XU) {
  for (int i4 = threadIdx.x; i4 < (K >> 2); i4 += kWg) {
    const float4 v = reinterpret_cast<const float4*>(xs)[i4];
    int u, e;
    unit_of_col<T>(4 * i4, u, e);
    XU[9 * u + (e >> 2)] = v;
    const float s4 = (v.x + v.y) + (v.z + v.w);
    const float s8 = s4 + dpp<0xb1>(s4);
    if ((i4 & 1) == 0) reinterpret_cast<float*>(XU + 9 * u + 8)[e >> 3] = s8;
  }
}

// A lane's share of a matvec task: lane group lg (of ng groups of lpr lanes)
// owns virtual rows lg, lg + ng, ... (GLU: even rows gate, odd rows up); lane
// li owns units li, li + lpr, ... of each row.
struct MvLane {
  int U, lpr, ng, lg, li, rows, ucount, t0;
  bool glu;
};

__device__ __forceinline__ MvLane mv_lane(const SegView& g, int t0, int nt, bool glu) {
  MvLane m;
  m.U = g.w.k >> 5;
  m.lpr = g.lpr;
  const int shift = __builtin_ctz((unsigned)m.lpr);
  m.ng = kWg >> shift;
  m.lg = threadIdx.x >> shift;
  m.li = threadIdx.x & (m.lpr - 1);
  const int nv = nt > 0 ? (glu ? 2 * nt : nt) : 0;
  m.rows = m.lg < nv ? (nv - m.lg + m.ng - 1) / m.ng : 0;
  m.ucount = (m.U + m.lpr - 1) / m.lpr;
  m.t0 = t0;
  m.glu = glu;
  return m;
}

// The lane walks its rows in batches of RB rows x UC units; the UC units' x
// stays in registers for all rows. Fragments of the next batch are in flight
// while the current one is reduced.
template <int T, int UC>
struct MvShape {
  static constexpr int kPf = sizeof(Frag<T>) > 40 ? 2 : 4;
  static constexpr int RB = kPf / UC > 0 ? kPf / UC : 1;
  static constexpr int N = RB * UC;
};

// units held in registers per lane: 1 or 2 (more are walked in blocks of 2)
__device__ __forceinline__ int mv_uc(const SegView& g) { return (g.w.k >> 5) <= g.lpr ? 1 : 2; }

// Issues the weight loads of batch b (unit block jb, rows [rb*RB, rb*RB+RB)).
template <int T, int UC>
__device__ __forceinline__ void mv_fetch(const SegView& g, const MvLane& m, int b, Frag<T> (&f)[MvShape<T, UC>::N]) {
  constexpr int RB = MvShape<T, UC>::RB;
  const int nrb = max(1, (m.rows + RB - 1) / RB);
  const int jb = b / nrb, rb = b - jb * nrb;
#pragma unroll
  for (int rr = 0; rr < RB; ++rr) {
    const int r = rb * RB + rr;
    const int v = m.lg + r * m.ng;
#pragma unroll
    for (int j = 0; j < UC; ++j) {
      // past the last batch u >= U, so nothing is loaded
      const int u = m.li + (jb * UC + j) * m.lpr;
      if (r < m.rows && u < m.U) {
        QMat w = g.w;
        if (m.glu && (v & 1)) {
          w.s0 = g.u0;
          w.s1 = g.u1;
          w.s2 = g.u2;
          w.s3 = g.u3;
        }
        f[rr * UC + j] = load_unit<T>(w, m.t0 + (m.glu ? (v >> 1) : v), u);
      }
    }
  }
}

// Dot products of the lane's rows once the digit planes are ready; cur holds
// batch 0 (issued by mv_fetch before the input was). Row r's sum lands in
// res[lg + r * ng]. AHEAD batches are in flight while one is reduced (two for
// long row streams such as the lm_head, whose batches would otherwise wait
// on memory one at a time).
template <int T, int UC, int AHEAD = 1>
__device__ __forceinline__ void mv_stream(const SegView& g, const MvLane& m, const XqView& x, float* res,
                                          Frag<T> (&cur)[MvShape<T, UC>::N]) {
  constexpr int RB = MvShape<T, UC>::RB, N = MvShape<T, UC>::N;
  const int nrb = max(1, (m.rows + RB - 1) / RB);
  const int nb = m.rows > 0 ? nrb * ((m.ucount + UC - 1) / UC) : 0;
  XU xr[UC];
  Frag<T> ahead[AHEAD > 1 ? AHEAD - 1 : 1][N];  // batches b + 1 .. b + AHEAD - 1
#pragma unroll
  for (int a = 0; a + 1 < AHEAD; ++a) mv_fetch<T, UC>(g, m, 1 + a, ahead[a]);
  for (int b = 0; b < nb; ++b) {
    const int jb = b / nrb, rb = b - jb * nrb;
    if (rb == 0) {
#pragma unroll
      for (int j = 0; j < UC; ++j) {
        const int u = m.li + (jb * UC + j) * m.lpr;
        if (u < m.U) load_xu<T>(x, u, xr[j]);
      }
    }
    Frag<T> nxt[N];
    mv_fetch<T, UC>(g, m, b + AHEAD, nxt);
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int r = rb * RB + rr;
      if (r < m.rows) {  // uniform in the lane group
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < UC; ++j) {
          const int u = m.li + (jb * UC + j) * m.lpr;
          if (u < m.U) acc += dot_q<T>(cur[rr * UC + j], u, xr[j]);
        }
        acc = group_sum_n(acc, m.lpr);
        if (m.li == 0) {
          float* d = res + m.lg + r * m.ng;
          *d = jb == 0 ? acc : *d + acc;
        }
      }
    }
    if constexpr (AHEAD > 1) {
#pragma unroll
      for (int q = 0; q < N; ++q) cur[q] = ahead[0][q];
#pragma unroll
      for (int a = 0; a + 2 < AHEAD; ++a)
#pragma unroll
        for (int q = 0; q < N; ++q) ahead[a][q] = ahead[a + 1][q];
#pragma unroll
      for (int q = 0; q < N; ++q) ahead[AHEAD - 2][q] = nxt[q];
    } else {
#pragma unroll
      for (int q = 0; q < N; ++q) cur[q] = nxt[q];
    }
  }
}

constexpr int kMaxG = 8;

__host__ __device__ constexpr int attn_tpp(int hd) { return hd / 64 > 2 ? hd / 64 : 2; }

template <bool KV16>
__device__ __forceinline__ void load_v(const void* tile, int idx, int dpl, float* v) {
  if constexpr (KV16) {
    const __half* h = (const __half*)tile + idx;
    if (dpl == 1) {
      v[0] = __half2float(h[0]);
    } else if (dpl == 2) {
      const uint32_t w = *(const uint32_t*)h;
      v[0] = h2f(w);
      v[1] = h2f(w >> 16);
    } else {
      const uint2 w = *(const uint2*)h;
      v[0] = h2f(w.x);
      v[1] = h2f(w.x >> 16);
      v[2] = h2f(w.y);
      v[3] = h2f(w.y >> 16);
    }
  } else {
    const float* f = (const float*)tile + idx;
    if (dpl == 1) {
      v[0] = f[0];
    } else if (dpl == 2) {
      const float2 w = *(const float2*)f;
      v[0] = w.x;
      v[1] = w.y;
    } else {
      const float4 w = *(const float4*)f;
      v[0] = w.x;
      v[1] = w.y;
      v[2] = w.z;
      v[3] = w.w;
    }
  }
}

// s[g] += q_g[my dims] . k[my dims] for this thread's NV 16-byte K vectors.
template <int G, bool KV16, int NV>
__device__ __forceinline__ void score_dot(const uint4* kreg, const float* qbase, int hd, float (&s)[G]) {
  constexpr int per = KV16 ? 8 : 4;  // elements per vector
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float kf[8];
    if constexpr (KV16) {
      const uint32_t w4[4] = {kreg[v].x, kreg[v].y, kreg[v].z, kreg[v].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kf[2 * i] = h2f(w4[i]);
        kf[2 * i + 1] = h2f(w4[i] >> 16);
      }
    } else {
      kf[0] = __uint_as_float(kreg[v].x);
      kf[1] = __uint_as_float(kreg[v].y);
      kf[2] = __uint_as_float(kreg[v].z);
      kf[3] = __uint_as_float(kreg[v].w);
    }
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const float4* qq = (const float4*)(qbase + gg * hd + v * per);
      const float4 q0 = qq[0];
      float s4 = (q0.x * kf[0] + q0.y * kf[1]) + (q0.z * kf[2] + q0.w * kf[3]);
      if constexpr (per == 8) {
        const float4 q1 = qq[1];
        s4 += (q1.x * kf[4] + q1.y * kf[5]) + (q1.z * kf[6] + q1.w * kf[7]);
      }
      s[gg] += s4;
    }
  }
}

// o[g][0..DPL) += sum over positions p in [pa, pb) of w_g(p) * V[p][d0..d0+DPL),
// where w_g(p) sits in lane (p - w0) * tpp of e[g]; eight positions per pass
// so that the LDS reads of a pass overlap.
template <int G, bool KV16, int DPL>
__device__ __forceinline__ void v_walk(const void* tile, int hd, int d0, int pa, int pb, int w0, int tpp,
                                       const float (&e)[G], float (&o)[G][4]) {
  int p = pa;
  for (; p + 8 <= pb; p += 8) {
    float vv[8][4];
#pragma unroll
    for (int u = 0; u < 8; ++u) load_v<KV16>(tile, (p + u) * hd + d0, DPL, vv[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int sel = (p + u - w0) * tpp;
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const float wgt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[gg]), sel));
#pragma unroll
        for (int k = 0; k < DPL; ++k) o[gg][k] += wgt * vv[u][k];
      }
    }
  }
  for (; p < pb; ++p) {
    float vv[4];
    load_v<KV16>(tile, p * hd + d0, DPL, vv);
    const int sel = (p - w0) * tpp;
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const float wgt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[gg]), sel));
#pragma unroll
      for (int k = 0; k < DPL; ++k) o[gg][k] += wgt * vv[k];
    }
  }
}

// LDS layout of the decode attention (floats): q_s[G][hd] | k_new[hd] |
// v_new[hd] | qn[hd] | kn[hd] | inv[hd] | wpart[4][G][hd] | wml[4][kMaxG][2] |
// wts[G][ncp] | cpart[rowf] | tile (V rows, later merge staging).

// Phases B-D of the decode attention for (kv head kv, chunk c) at position
// pos, once the group's q heads, the new k/v, the norm weights and the rotary
// table are in LDS, the chunk's valid V rows are in the LDS tile and this
// thread's K slice is in kreg (layout of k_attention). Leaves the chunk
// partial in cpart: for head g at g * (hd + 2), [max, sum, acc[hd]].
template <int G, bool KV16>
__device__ __forceinline__ void attn_chunk(const AttnArgs& a, float* sm, int kv, int c, int pos,
                                           uint4 (&kreg)[KV16 ? 8 : 16], const float* inv_in = nullptr,
                                           const float* qn_in = nullptr, const float* kn_in = nullptr,
                                           void* vtile = nullptr) {
  const int hd = a.hd, half = hd / 2, CH = a.chunk;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tpp = a.tpp, P = 64 / tpp;
  const int my_p = tid / tpp, my_j = tid & (tpp - 1);
  const int dpt = hd / tpp;
  const int t_lo = c * CH;
  constexpr int kElem = KV16 ? 2 : 4;
  constexpr int kVec = KV16 ? 8 : 16;
  const int nvec = dpt * kElem / 16;
  const int ncp = (a.nchunk + 3) & ~3;
  float* q_s = sm;
  float* k_new = q_s + G * hd;
  float* v_new = k_new + hd;
  float* qn = v_new + hd;
  float* kn = qn + hd;
  float* inv = kn + hd;
  float* wpart = inv + hd;
  float* wml = wpart + 4 * G * hd;
  float* wts = wml + 8 * kMaxG;
  float* cpart = wts + G * ncp;
  // the rotary table, norm weights and V rows come from sm, or from the
  // caller's copies when it passes them
  float* tile = vtile ? (float*)vtile : cpart + attn_rowf(G, hd);
  if (inv_in) inv = (float*)inv_in;
  if (qn_in) qn = (float*)qn_in;
  if (kn_in) kn = (float*)kn_in;
  const size_t head_base = (size_t)kv * a.ctx * hd;
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_hi = pos / CH;
  const int p_begin = max(start - t_lo, 0);
  const int p_end = min(pos + 1 - t_lo, CH);
  const int p_new = pos - t_lo;
  const bool own_new = (c == c_hi);
  (void)P;

  // B: per-head RMSNorm + rotary, one wave per head; the new k/v to the cache
  {
    const int nh = G + (own_new ? 1 : 0);
    const size_t row = head_base + (size_t)pos * hd;
    for (int hh = wave; hh < nh; hh += 4) {
      const bool is_k = hh == G;
      float* x = is_k ? k_new : q_s + hh * hd;
      float r = 1.0f;
      if (a.qn_w) {
        float ss = 0.f;
        for (int d = lane; d < hd; d += 64) ss += x[d] * x[d];
        ss = wave_sum(ss);
        r = 1.0f / sqrtf(ss / (float)hd + a.eps);
      }
      const float* w = is_k ? kn : qn;
      for (int d = lane; d < half; d += 64) {
        const int ia = a.interleaved ? 2 * d : d;
        const int ib = a.interleaved ? 2 * d + 1 : d + half;
        float x0 = x[ia], x1 = x[ib];
        if (a.qn_w) {
          x0 = __fmul_rn(__fmul_rn(x0, r), w[ia]);
          x1 = __fmul_rn(__fmul_rn(x1, r), w[ib]);
        }
        const float ang = __fmul_rn((float)pos, inv[d]);
        const float co = cosf(ang), si = sinf(ang);
        float y0 = __fsub_rn(__fmul_rn(x0, co), __fmul_rn(x1, si));
        float y1 = __fadd_rn(__fmul_rn(x0, si), __fmul_rn(x1, co));
        if (is_k) {
          if constexpr (KV16) {
            const __half h0 = __float2half_rn(y0), h1 = __float2half_rn(y1);
            *gblw((unsigned short*)a.kc + row + ia) = __half_as_ushort(h0);
            *gblw((unsigned short*)a.kc + row + ib) = __half_as_ushort(h1);
            y0 = __half2float(h0);
            y1 = __half2float(h1);
          } else {
            *gblw((float*)a.kc + row + ia) = y0;
            *gblw((float*)a.kc + row + ib) = y1;
          }
        }
        x[ia] = y0;
        x[ib] = y1;
      }
      if (is_k) {
        for (int d = lane; d < hd; d += 64) {
          if constexpr (KV16) {
            const __half vh = __float2half_rn(v_new[d]);
            *gblw((unsigned short*)a.vc + row + d) = __half_as_ushort(vh);
            ((__half*)tile)[p_new * hd + d] = vh;
          } else {
            *gblw((float*)a.vc + row + d) = v_new[d];
            tile[p_new * hd + d] = v_new[d];
          }
        }
      }
    }
    __syncthreads();
  }
  CHONK_ATTN_STAMP(1);

  // C: scores, wave-local softmax statistics, weighted V
  {
    const bool valid = my_p < CH && my_p >= p_begin && my_p < p_end;
    if (own_new && my_p == p_new) {
      // the new position's k (already rounded to the cache type) into the K registers
      const float* kk = k_new + my_j * dpt;
#pragma unroll
      for (int v = 0; v < kVec; ++v) {
        if (v < nvec) {
          if constexpr (KV16) {
            uint32_t w4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              w4[i] = (uint32_t)__half_as_ushort(__float2half_rn(kk[v * 8 + 2 * i])) |
                      ((uint32_t)__half_as_ushort(__float2half_rn(kk[v * 8 + 2 * i + 1])) << 16);
            kreg[v] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          } else {
            kreg[v] = make_uint4(__float_as_uint(kk[v * 4]), __float_as_uint(kk[v * 4 + 1]),
                                 __float_as_uint(kk[v * 4 + 2]), __float_as_uint(kk[v * 4 + 3]));
          }
        }
      }
    }
    float s[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) s[gg] = 0.f;
    {
      const float* qbase = q_s + my_j * dpt;
      switch (nvec) {
        case 1: score_dot<G, KV16, 1>(kreg, qbase, hd, s); break;
        case 2: score_dot<G, KV16, 2>(kreg, qbase, hd, s); break;
        case 4: score_dot<G, KV16, 4>(kreg, qbase, hd, s); break;
        case 8: score_dot<G, KV16, 8>(kreg, qbase, hd, s); break;
        default:
          if constexpr (!KV16) score_dot<G, KV16, 16>(kreg, qbase, hd, s);
          break;
      }
    }
    float e[G], m[G], l[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      s[gg] = group_sum_n(s[gg], tpp);
      const float sv = valid ? s[gg] * a.scale : -INFINITY;
      m[gg] = wave_max(sv);
      e[gg] = valid ? expf(sv - m[gg]) : 0.0f;
      l[gg] = wave_sum(my_j == 0 ? e[gg] : 0.0f);
    }
    // V: lane -> dims [d0, d0 + dpl); positions of this wave in order
    const int dpl = hd >= 64 ? hd / 64 : 1;
    const int d0 = (lane * dpl) % hd;
    const int w0 = wave * P;
    const int pa = max(p_begin, w0), pb = min(p_end, w0 + P);
    float o[G][4];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int k = 0; k < 4; ++k) o[gg][k] = 0.f;
    if (dpl == 1)
      v_walk<G, KV16, 1>(tile, hd, d0, pa, pb, w0, tpp, e, o);
    else if (dpl == 2)
      v_walk<G, KV16, 2>(tile, hd, d0, pa, pb, w0, tpp, e, o);
    else
      v_walk<G, KV16, 4>(tile, hd, d0, pa, pb, w0, tpp, e, o);
    if (lane * dpl < hd) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (k < dpl) wpart[(wave * G + gg) * hd + d0 + k] = o[gg][k];
    }
    if (lane == 0) {
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        wml[(wave * kMaxG + gg) * 2] = m[gg];
        wml[(wave * kMaxG + gg) * 2 + 1] = l[gg];
      }
    }
  }
  __syncthreads();
  CHONK_ATTN_STAMP(2);

  // D: chunk partial = the four wave partials rescaled to the chunk maximum
  for (int i = tid; i < G * hd; i += kWg) {
    const int gg = i / hd, d = i - gg * hd;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * kMaxG + gg) * 2]);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = wml[(w * kMaxG + gg) * 2];
      if (mw != -INFINITY) acc += wpart[(w * G + gg) * hd + d] * expf(mw - M);
    }
    cpart[gg * (hd + 2) + 2 + d] = acc;
  }
  if (tid < G) {
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * kMaxG + tid) * 2]);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = wml[(w * kMaxG + tid) * 2];
      if (mw != -INFINITY) L += wml[(w * kMaxG + tid) * 2 + 1] * expf(mw - M);
    }
    cpart[tid * (hd + 2)] = M;
    cpart[tid * (hd + 2) + 1] = L;
  }
  __syncthreads();
  CHONK_ATTN_STAMP(3);
}

// attn_chunk, then the chunk partial to uncached memory; the last chunk of the
// head to arrive (arrival counter a.cnt[kv]) merges all of them and stores
// output element i of the group (i = g * hd + d) with out(i, value).
template <int G, bool KV16, class Out>
__device__ __forceinline__ void attn_compute(const AttnArgs& a, float* sm, int kv, int c, int pos,
                                             uint4 (&kreg)[KV16 ? 8 : 16], uint32_t* s_last, Out out) {
  attn_chunk<G, KV16>(a, sm, kv, c, pos, kreg);
  const int hd = a.hd, CH = a.chunk;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncp = (a.nchunk + 3) & ~3;
  float* wml = sm + (5 * G + 5) * hd;
  float* wts = wml + 8 * kMaxG;
  const float* cpart = wts + G * ncp;
  float* tile = (float*)cpart + attn_rowf(G, hd);
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_lo = start / CH, c_hi = pos / CH;
  const int rowf = attn_rowf(G, hd);  // floats per chunk partial, 16-byte multiple
  float* part = a.part + (size_t)(kv * a.nchunk + c) * rowf;
  for (int i = tid; i < G * (hd + 2); i += kWg) *gblw(part + i) = cpart[i];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(gblw(&a.cnt[kv]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = (old == (uint32_t)(c_hi - c_lo)) ? 1u : 0u;
  }
  __syncthreads();
  if (!*s_last) return;

  // merge (last chunk): chunk weights w[g][c] = exp(m_c - M_g) once, then the
  // acc rows, staged into LDS in batches, weighted and summed
  const int nact = c_hi - c_lo + 1;
  const float* rows0 = a.part + (size_t)(kv * a.nchunk + c_lo) * rowf;
  float* stage = tile;
  const int per_batch = max(1, a.merge_floats / rowf);
  lds_dma(rows0, stage, min(per_batch, nact) * rowf);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int gg = wave; gg < G; gg += 4) {
    float M = -INFINITY;
    for (int cc = lane; cc < nact; cc += 64) {
      const float mv = cc < per_batch ? stage[cc * rowf + gg * (hd + 2)] : *gbl(rows0 + (size_t)cc * rowf + gg * (hd + 2));
      M = fmaxf(M, mv);
    }
    M = wave_max(M);
    float L = 0.f;
    for (int cc = lane; cc < nact; cc += 64) {
      const float* pp = cc < per_batch ? stage + cc * rowf + gg * (hd + 2) : rows0 + (size_t)cc * rowf + gg * (hd + 2);
      const float f = expf(pp[0] - M);
      wts[gg * ncp + cc] = f;
      L += pp[1] * f;
    }
    L = wave_sum(L);
    if (lane == 0) wml[2 * gg] = 1.0f / L;
  }
  __syncthreads();
  float o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = 0.f;
  for (int b0 = 0; b0 < nact; b0 += per_batch) {
    const int nb = min(per_batch, nact - b0);
    if (b0 > 0) {
      __syncthreads();  // previous batch consumed
      lds_dma(rows0 + (size_t)b0 * rowf, stage, nb * rowf);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = tid + q * kWg;
      if (i < G * hd) {
        const int gg = i / hd, d = i - gg * hd;
        const float* src = stage + gg * (hd + 2) + 2 + d;
        const float* wv = wts + gg * ncp + b0;
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        int cc = 0;
        for (; cc + 4 <= nb; cc += 4) {
          acc0 += src[cc * rowf] * wv[cc];
          acc1 += src[(cc + 1) * rowf] * wv[cc + 1];
          acc2 += src[(cc + 2) * rowf] * wv[cc + 2];
          acc3 += src[(cc + 3) * rowf] * wv[cc + 3];
        }
        for (; cc < nb; ++cc) acc0 += src[cc * rowf] * wv[cc];
        o[q] += (acc0 + acc1) + (acc2 + acc3);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = tid + q * kWg;
    if (i < G * hd) {
      const int gg = i / hd, d = i - gg * hd;
      out(gg * hd + d, o[q] * wml[2 * gg]);
    }
  }
  if (tid == 0) __hip_atomic_store(gblw(&a.cnt[kv]), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Token selection: ARGMAX_STAGE2 or the candidate sampler; bookkeeping.
constexpr int kMaxGroups = 4096;

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// sort order: valid before invalid, then value descending, then group ascending
__device__ __forceinline__ bool before(double va, uint32_t ga, double vb, uint32_t gb) {
  const bool oka = !(ga >> 31), okb = !(gb >> 31);
  if (oka != okb) return oka;
  if (va != vb) return va > vb;
  return (ga & 0x7fffffffu) < (gb & 0x7fffffffu);
}

constexpr int kSelectWorkspaceBytes = kMaxGroups * 12 + kWg * 8 + 16;

// Selects the next token from the group candidates and updates the
// bookkeeping (history, generated ids, stop flag, position). `ws` is LDS of
// kSelectWorkspaceBytes bytes; all kWg threads of the workgroup take part.
__device__ __forceinline__ void select_token(const SelArgs& a, uint8_t* ws) {
  DevState* st = a.st;
  const DevSampling& s = *a.samp;
  const int tid = threadIdx.x;
  double* sv = (double*)ws;                             // [kMaxGroups]
  uint32_t* sg = (uint32_t*)(sv + kMaxGroups);          // [kMaxGroups]
  float* vals = (float*)(sg + kMaxGroups);              // [kWg]
  uint32_t* idx = (uint32_t*)(vals + kWg);              // [kWg]
  int* s_int = (int*)(idx + kWg);                       // [4]
  int token = 0;
  const int groups = a.groups;

  if (s.sample_mode == 0 && a.gpt_argmax) {
    // the GPT-2 runtime's ARGMAX_STAGE2 (gpt-wgsl-runtime.ts:1961-2004): one
    // slot per group (at most 256), padding (-3.402823e38, 0), a tree that
    // keeps the left slot unless the right one is strictly greater
    if (tid < groups) {
      const Candidate c = a.cand[tid];
      vals[tid] = c.value;
      idx[tid] = c.index;
    } else {
      vals[tid] = kNegBig;
      idx[tid] = 0u;
    }
    __syncthreads();
    for (int stride = 128; stride >= 1; stride >>= 1) {
      if (tid < stride && vals[tid + stride] > vals[tid]) {
        vals[tid] = vals[tid + stride];
        idx[tid] = idx[tid + stride];
      }
      __syncthreads();
    }
    token = (int)idx[0];
  } else if (s.sample_mode == 0) {
    float bv = kNegBig;
    uint32_t bi = 0xffffffffu;
    for (int g = tid; g < groups; g += kWg) {
      const Candidate c = a.cand[g];
      if (better(c.value, c.index, bv, bi)) {
        bv = c.value;
        bi = c.index;
      }
    }
    vals[tid] = bv;
    idx[tid] = bi;
    __syncthreads();
    for (int stride = 128; stride >= 1; stride >>= 1) {
      if (tid < stride && better(vals[tid + stride], idx[tid + stride], vals[tid], idx[tid])) {
        vals[tid] = vals[tid + stride];
        idx[tid] = idx[tid + stride];
      }
      __syncthreads();
    }
    token = (int)idx[0];
  } else {
    int n2 = 1;
    while (n2 < groups) n2 <<= 1;
    // load + second penalty (sampling.ts:35-43)
    int cnt = 0;
    for (int i = tid; i < n2; i += kWg) {
      double v = 0.0;
      bool ok = false;
      if (i < groups) {
        const Candidate c = a.cand[i];
        ok = isfinite(c.value) && c.index != 0xffffffffu;
        v = (double)c.value;
        if (ok && s.seen_penalty && c.index < (uint32_t)a.vocab && bit_test(a.seen_bits, c.index))
          v = v > 0 ? v / s.repetition_penalty : v * s.repetition_penalty;
      }
      sv[i] = ok ? v : 0.0;
      sg[i] = (uint32_t)i | (ok ? 0u : 0x80000000u);
      cnt += ok ? 1 : 0;
    }
    vals[tid] = (float)cnt;
    __syncthreads();
    for (int stride = 128; stride >= 1; stride >>= 1) {
      if (tid < stride) vals[tid] += vals[tid + stride];
      __syncthreads();
    }
    const int n_valid = (int)vals[0];
    // bitonic sort (stable via the group index key)
    for (int k = 2; k <= n2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < n2; i += kWg) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const bool asc = (i & k) == 0;
            const bool swap = asc ? before(sv[ixj], sg[ixj], sv[i], sg[i]) : before(sv[i], sg[i], sv[ixj], sg[ixj]);
            if (swap) {
              const double tv = sv[i];
              sv[i] = sv[ixj];
              sv[ixj] = tv;
              const uint32_t tg = sg[i];
              sg[i] = sg[ixj];
              sg[ixj] = tg;
            }
          }
        }
        __syncthreads();
      }
    }
    const int lim = s.top_k > 0 ? min(s.top_k, n_valid) : n_valid;
    auto id_at = [&](int i) -> int { return (int)a.cand[sg[i] & 0x7fffffffu].index; };
    if (s.temperature <= 0.0) {
      token = n_valid > 0 ? id_at(0) : 0;
    } else {
      // sampling.ts:53-75: probabilities in parallel, the running sums
      // sequentially in the reference's order.
      const double maxv = lim > 0 ? sv[0] : 0.0;
      __syncthreads();
      for (int i = tid; i < lim; i += kWg) sv[i] = exp((sv[i] - maxv) / s.temperature);
      __syncthreads();
      if (tid == 0) {
        double total = 0.0;
        for (int i = 0; i < lim; ++i) total += sv[i];
        int cutoff = lim;
        if (s.top_p < 1.0 && total > 0.0) {
          double cdf = 0.0;
          for (int i = 0; i < lim; ++i) {
            cdf += sv[i] / total;
            if (cdf >= s.top_p) {
              cutoff = i + 1;
              break;
            }
          }
        }
        double sample_total = 0.0;
        for (int i = 0; i < cutoff; ++i) sample_total += sv[i];
        const uint64_t z = mix64(s.seed + 0x9e3779b97f4a7c15ull * (uint64_t)(st->pos + 1));
        const double u = (double)(z >> 11) * (1.0 / 9007199254740992.0);
        double r = u * sample_total;
        int pick = -1;
        for (int i = 0; i < cutoff; ++i) {
          r -= sv[i];
          if (r <= 0) {
            pick = i;
            break;
          }
        }
        if (pick < 0) pick = max(0, cutoff - 1);
        s_int[2] = lim > 0 ? id_at(pick) : 0;
      }
      __syncthreads();
      token = s_int[2];
    }
  }

  if (tid == 0) {
    const int pos = st->pos;
    st->last_token = token;
    if (pos + 1 <= a.ctx) a.hist[pos + 1] = token;
    if (st->generating) {
      const int ng = st->n_generated;
      if (ng <= a.ctx) a.gen[ng] = token;
      st->n_generated = ng + 1;
      if (token >= 0 && token < a.vocab) {
        a.pen_bits[token >> 5] |= 1u << (token & 31);
        a.seen_bits[token >> 5] |= 1u << (token & 31);
      }
      bool eos = false;
      for (int i = 0; i < s.n_eos && i < 16; ++i) eos |= (s.eos[i] == token);
      if (eos || ng + 1 >= st->max_generated) st->stopped = 1;
    }
    st->pos = pos + 1;
  }
}

}  // namespace
}  // namespace chonk
