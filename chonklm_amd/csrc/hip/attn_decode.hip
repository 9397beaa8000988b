// Decode attention over the fp16 K/V cache for one new token (the reference's
// qkNormRopeStore + attention score/value passes, src/lib/llama-wgsl-runtime.ts
// :1467-1509, :1548-1570, WGSL :2868-3490), laid out for latency on gfx950.
//
// One workgroup per (kv head, chunk of 64 positions); each wave owns 16
// positions of the chunk and keeps them in registers:
//   A  the position by a scalar load, then every load of the workgroup: the
//      wave's K rows (four lanes per position, HD/4 dims each) and V rows
//      (HD/64 dims of each of the 16 positions per lane) into registers, q
//      heads of the group, new k/v and norm weights into LDS, and the rotary
//      (cos, sin) of the position from the engine's table.
//   B  every wave does the q RMSNorm + rotary of the group into its own LDS
//      copy (no workgroup barrier).
//   C  scores by quads of lanes, softmax statistics over the wave's 16
//      positions, weights through LDS (broadcast reads), V walked from
//      registers — over the cached positions [start, pos); the new position
//      is not in the cache yet.
//   D  the four wave partials rescale to the chunk maximum and go to the
//      chunk's row as tagged words {f32, u32 tag} (no wait); then every active
//      chunk merges a slice of the output dims: it polls the rows' (max, sum)
//      words and its dims' acc words until all carry this launch's tag, forms
//      the weights exp(m_c - M) once per (head, chunk) with the lanes of one
//      wave, and writes one weighted sum per output element. The new position
//      joins every merge as one more term: while the rows travel, each chunk
//      normalises, rotates and rounds k (and rounds v) itself, and the
//      newest chunk stores both to the cache — so no chunk does more work
//      than another before its row is out. The chunks of a
//      launch wait for each other, so the engine uses this kernel only when
//      its whole grid fits on the device at once; every wait is also bounded
//      in time (DevState.error = 4 past the bound).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "kernel_common.h"
#include "kernels.h"

namespace chonk {
namespace {

constexpr int kDecChunk = 64;  // positions per workgroup
constexpr int kDecWave = 16;   // positions per wave

// DPL consecutive halves of one V row held by a lane.
template <int DPL>
struct VRow;
template <>
struct VRow<1> {
  uint32_t w;
  __device__ void load(const __half* p) { w = (uint32_t)*gbl((const uint16_t*)p); }
  __device__ void get(float* f) const { f[0] = __half2float(__ushort_as_half((unsigned short)w)); }
};
template <>
struct VRow<2> {
  uint32_t w;
  __device__ void load(const __half* p) { w = ldg1(p); }
  __device__ void get(float* f) const {
    f[0] = __half2float(__ushort_as_half((unsigned short)(w & 0xffffu)));
    f[1] = __half2float(__ushort_as_half((unsigned short)(w >> 16)));
  }
};
template <>
struct VRow<4> {
  uint2 w;
  __device__ void load(const __half* p) { w = ldg2(p); }
  __device__ void get(float* f) const {
    f[0] = __half2float(__ushort_as_half((unsigned short)(w.x & 0xffffu)));
    f[1] = __half2float(__ushort_as_half((unsigned short)(w.x >> 16)));
    f[2] = __half2float(__ushort_as_half((unsigned short)(w.y & 0xffffu)));
    f[3] = __half2float(__ushort_as_half((unsigned short)(w.y >> 16)));
  }
};

__device__ __forceinline__ float2 ldg2f(const float2* p) {
  const uint2 v = ldg2(p);
  return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
}

// A load through the scalar unit (own wait counter). For values that do not
// change while the kernel reads them: written by an earlier kernel, or (the
// epoch) advanced only after every workgroup that uses it has read it.
template <class T>
__device__ __forceinline__ T ld_scalar(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

__device__ __forceinline__ void halves8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __half2float(__ushort_as_half((unsigned short)(w[i] & 0xffffu)));
    f[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
  }
}

// Two floats that are exact fp16 values, packed (truncating conversion).
__device__ __forceinline__ uint32_t pkrtz(float a, float b) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(a, b);
  uint32_t u;
  __builtin_memcpy(&u, &h, 4);
  return u;
}

// A wait for chunk rows is bounded (wall clock, 100 MHz): past the bound the
// merge gives up, reports DevState.error = 4 and leaves.
constexpr uint64_t kDecPollTicks = 20ull * 100000ull;  // 20 ms

__device__ __forceinline__ void tag_put(tagged_t* p, float v, uint32_t tag) {
  __hip_atomic_store(gblw(p), ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tag_get(const tagged_t* p) {
  return __hip_atomic_load(gbl(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float tag_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

// LDS (floats): q_s[G][HD] (raw) | kx[HD] | vx[HD] | nq[HD] | nk[HD] |
// qw[4][G][HD] (each wave's normalised, rotated q) | ew[4][G][16] |
// wml[4][G][2] | area: wave partials [4][G][HD], later the merge weights [G][ncp].
//
// Chunk rows (a.tpart, [kv][nchunk][rowf] tagged words): per head [max, sum,
// acc[HD]], each word {f32, u32 tag}; the tag of a launch is the kv head's
// epoch a.cnt[kv], which the merging workgroup advances when it is done.
template <int G, int HD>
__global__ __launch_bounds__(kWg) void k_attn_dec(const AttnArgs a) {
  extern __shared__ __align__(16) float sm[];
  constexpr int HALF = HD / 2;
  constexpr int DPT = HD / 4;       // K dims per lane (four lanes per position)
  constexpr int NKV = DPT / 8;      // 16-byte K vectors per lane
  constexpr int DPL = HD / 64;      // V dims per lane
  constexpr int NPR = (HALF + 63) / 64;  // rotary pairs per lane
  const int kv = blockIdx.x, c = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* q_s = sm;
  float* kx = q_s + G * HD;
  float* vx = kx + HD;
  float* nq = vx + HD;
  float* nk = nq + HD;
  float* qw = nk + HD + wave * G * HD;
  float* ew = nk + HD + 4 * G * HD;
  float* wml = ew + 4 * G * kDecWave;
  float* area = wml + 8 * G;
  uint64_t tr[8];
  CHONK_MV_T(tr, 0);

  // A: the position, stop flag and epoch by scalar loads (their own counter,
  // so nothing below waits on them early), then the vector loads: the rotary
  // frequencies, the wave's K/V rows, the LDS copies — with the rotary cos/sin
  // computed while they are in flight
  DevState* st = a.st;
  const int pos = ld_scalar(&st->pos);
  const int stopped = ld_scalar(&st->stopped);
  const uint32_t tag = ld_scalar(&a.cnt[kv]);
  const int t_lo = c * kDecChunk;
  const int kp = kDecWave * wave + (lane >> 2);  // this lane's K position in the chunk
  const int kd0 = (lane & 3) * DPT;
  const __half* kc = (const __half*)a.kc + (size_t)kv * a.ctx * HD;
  const __half* vc = (const __half*)a.vc + (size_t)kv * a.ctx * HD;
  uint4 kr[NKV];
  VRow<DPL> vr[kDecWave];
  auto load_kv = [&]() {
    const int tk = min(t_lo + kp, a.ctx - 1);
#pragma unroll
    for (int v = 0; v < NKV; ++v) kr[v] = ldg4(kc + (size_t)tk * HD + kd0 + 8 * v);
#pragma unroll
    for (int p = 0; p < kDecWave; ++p) {
      const int tv = min(t_lo + kDecWave * wave + p, a.ctx - 1);
      vr[p].load(vc + (size_t)tv * HD + lane * DPL);
    }
  };
  if (a.spec_kv) load_kv();
  lds_dma(a.qkv + (size_t)kv * G * HD, q_s, G * HD);
  lds_dma(a.qkv + (size_t)a.heads * HD + (size_t)kv * HD, kx, HD);
  lds_dma(a.qkv + (size_t)(a.heads + a.kv_heads) * HD + (size_t)kv * HD, vx, HD);
  if (a.qn_w) {
    lds_dma(a.qn_w, nq, HD);
    lds_dma(a.kn_w, nk, HD);
  }
  // rotary (cos, sin) of the lane's pairs at the position
  float co[NPR], si[NPR];
  {
    const int pc = min(pos, a.ctx - 1);
#pragma unroll
    for (int j = 0; j < NPR; ++j) {
      const float2 v = ldg2f(a.rope_cs + (size_t)pc * HALF + min(lane + 64 * j, HALF - 1));
      co[j] = v.x;
      si[j] = v.y;
    }
  }
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_lo = start / kDecChunk, c_hi = pos / kDecChunk;
  const bool active = !stopped && pos < a.ctx && c >= c_lo && c <= c_hi;
  if (active && !a.spec_kv) load_kv();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  CHONK_MV_T(tr, 1);
  if (stopped) return;
  if (pos >= a.ctx) {
    if (tid == 0) st->error = 1;
    return;
  }
  if (!active) return;

  // B: every wave normalises and rotates the group's q heads into its own copy
  // (all heads in one pass, so the reductions overlap)
  int ia[NPR], ib[NPR];
#pragma unroll
  for (int j = 0; j < NPR; ++j) {
    const int d = min(lane + 64 * j, HALF - 1);
    ia[j] = a.interleaved ? 2 * d : d;
    ib[j] = a.interleaved ? 2 * d + 1 : d + HALF;
  }
  {
    float x0[G][NPR], x1[G][NPR];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < NPR; ++j) {
        x0[h][j] = q_s[h * HD + ia[j]];
        x1[h][j] = q_s[h * HD + ib[j]];
      }
    if (a.qn_w) {
      float ss[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        ss[h] = 0.f;
#pragma unroll
        for (int j = 0; j < NPR; ++j)
          if (lane + 64 * j < HALF) ss[h] += x0[h][j] * x0[h][j] + x1[h][j] * x1[h][j];
      }
#pragma unroll
      for (int h = 0; h < G; ++h) ss[h] = wave_sum(ss[h]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float r = 1.0f / sqrtf(ss[h] / (float)HD + a.eps);
#pragma unroll
        for (int j = 0; j < NPR; ++j) {
          x0[h][j] = __fmul_rn(__fmul_rn(x0[h][j], r), nq[ia[j]]);
          x1[h][j] = __fmul_rn(__fmul_rn(x1[h][j], r), nq[ib[j]]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int j = 0; j < NPR; ++j)
        if (lane + 64 * j < HALF) {
          qw[h * HD + ia[j]] = __fsub_rn(__fmul_rn(x0[h][j], co[j]), __fmul_rn(x1[h][j], si[j]));
          qw[h * HD + ib[j]] = __fadd_rn(__fmul_rn(x0[h][j], si[j]), __fmul_rn(x1[h][j], co[j]));
        }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's q copy is in LDS
  __builtin_amdgcn_wave_barrier();

  // C: scores, the wave's softmax statistics, weighted V
  const int tk = t_lo + kp;
  // the new position is not in the registers (its row is written by this
  // launch): the merge adds it
  const bool kvalid = tk >= start && tk < pos;
  float s[G];
#pragma unroll
  for (int g = 0; g < G; ++g) s[g] = 0.f;
#pragma unroll
  for (int v = 0; v < NKV; ++v) {
    float kf[8];
    halves8(kr[v], kf);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float4 q0 = *(const float4*)(qw + g * HD + kd0 + 8 * v);
      const float4 q1 = *(const float4*)(qw + g * HD + kd0 + 8 * v + 4);
      s[g] += ((q0.x * kf[0] + q0.y * kf[1]) + (q0.z * kf[2] + q0.w * kf[3])) +
              ((q1.x * kf[4] + q1.y * kf[5]) + (q1.z * kf[6] + q1.w * kf[7]));
    }
  }
  float m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float sc = group_sum<4>(s[g]);
    const float sv = kvalid ? sc * a.scale : -INFINITY;
    m[g] = wave_max(sv);
    const float e = kvalid ? expf(sv - m[g]) : 0.f;
    l[g] = wave_sum((lane & 3) == 0 ? e : 0.f);
    if ((lane & 3) == 0) ew[(wave * G + g) * kDecWave + (lane >> 2)] = e;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's weights are in LDS
  __builtin_amdgcn_wave_barrier();
  float o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int k = 0; k < DPL; ++k) o[g][k] = 0.f;
  const int p0 = t_lo + kDecWave * wave;
#pragma unroll
  for (int p4 = 0; p4 < kDecWave / 4; ++p4) {
    float4 w4[G];
#pragma unroll
    for (int g = 0; g < G; ++g) w4[g] = *(const float4*)(ew + (wave * G + g) * kDecWave + 4 * p4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = 4 * p4 + i;
      float vf[DPL];
      vr[p].get(vf);
      // positions outside [start, pos) carry weight 0; their (possibly
      // unwritten) rows must not reach the sum
      const bool ok = p0 + p >= start && p0 + p < pos;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float wt = i == 0 ? w4[g].x : i == 1 ? w4[g].y : i == 2 ? w4[g].z : w4[g].w;
#pragma unroll
        for (int k = 0; k < DPL; ++k) o[g][k] += ok ? wt * vf[k] : 0.f;
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int k = 0; k < DPL; ++k) area[(wave * G + g) * HD + lane * DPL + k] = o[g][k];
    if (lane == 0) {
      wml[(wave * G + g) * 2] = m[g];
      wml[(wave * G + g) * 2 + 1] = l[g];
    }
  }
  __syncthreads();
  CHONK_MV_T(tr, 2);

  // D: chunk partial [max, sum, acc[HD]] per head, to the chunk's row
  const int rowf = attn_rowf(G, HD);
  tagged_t* row = a.tpart + (size_t)(kv * a.nchunk + c) * rowf;
  for (int i = tid; i < G * HD; i += kWg) {
    const int g = i / HD, d = i - g * HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * G + g) * 2]);
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = wml[(w * G + g) * 2];
      if (mw != -INFINITY) acc += area[(w * G + g) * HD + d] * expf(mw - M);
    }
    tag_put(row + g * (HD + 2) + 2 + d, acc, tag);
  }
  if (tid < G) {
    float M = -INFINITY, L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, wml[(w * G + tid) * 2]);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = wml[(w * G + tid) * 2];
      if (mw != -INFINITY) L += wml[(w * G + tid) * 2 + 1] * expf(mw - M);
    }
    tag_put(row + tid * (HD + 2), M, tag);
    tag_put(row + tid * (HD + 2) + 1, L, tag);
  }

  CHONK_MV_T(tr, 3);
  // merge, shared by the active chunks: chunk ci merges dims [ci*SD, ci*SD+SD)
  // of every head of the group. It polls the (max, sum) words of every row and
  // its dims' acc words until all carry this launch's tag (one pass costs one
  // memory round trip), then weights exp(m_c - M) per (head, chunk) by the
  // lanes of one wave, then one weighted sum per output element.
  const int nact = c_hi - c_lo + 1, ci = c - c_lo;
  const int SD = (HD + nact - 1) / nact;
  const int d_lo = min(ci * SD, HD), nd = min(SD, HD - d_lo);
  const tagged_t* rows0 = a.tpart + (size_t)(kv * a.nchunk + c_lo) * rowf;
  __syncthreads();  // area (the wave partials) is reused
  float* ml = area;                  // [G][nact][2]
  float* colv = ml + 2 * G * nact;   // [G][nd][nact]
  float* wts = colv + G * SD * nact; // [G][nact], then 1/L per head in wml
  const int n_ml = 2 * G * nact, n_col = G * nd * nact, total = n_ml + n_col;
  // the new position, while the rows are on their way: wave 0 normalises,
  // rotates and rounds k, wave 1 rounds v (the newest chunk also stores both
  // to the cache); every chunk adds the position to its merge
  const size_t kv_row = ((size_t)kv * a.ctx + pos) * HD;
  if (wave == 0) {
    float x0[NPR], x1[NPR];
#pragma unroll
    for (int j = 0; j < NPR; ++j) {
      x0[j] = kx[ia[j]];
      x1[j] = kx[ib[j]];
    }
    if (a.qn_w) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NPR; ++j)
        if (lane + 64 * j < HALF) ss += x0[j] * x0[j] + x1[j] * x1[j];
      ss = wave_sum(ss);
      const float r = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
      for (int j = 0; j < NPR; ++j) {
        x0[j] = __fmul_rn(__fmul_rn(x0[j], r), nk[ia[j]]);
        x1[j] = __fmul_rn(__fmul_rn(x1[j], r), nk[ib[j]]);
      }
    }
#pragma unroll
    for (int j = 0; j < NPR; ++j)
      if (lane + 64 * j < HALF) {
        const __half h0 = __float2half_rn(__fsub_rn(__fmul_rn(x0[j], co[j]), __fmul_rn(x1[j], si[j])));
        const __half h1 = __float2half_rn(__fadd_rn(__fmul_rn(x0[j], si[j]), __fmul_rn(x1[j], co[j])));
        if (c == c_hi) {
          *gblw((unsigned short*)a.kc + kv_row + ia[j]) = __half_as_ushort(h0);
          *gblw((unsigned short*)a.kc + kv_row + ib[j]) = __half_as_ushort(h1);
        }
        kx[ia[j]] = __half2float(h0);
        kx[ib[j]] = __half2float(h1);
      }
  } else if (wave == 1) {
#pragma unroll
    for (int d = lane; d < HD; d += 64) {
      const __half vh = __float2half_rn(vx[d]);
      if (c == c_hi) *gblw((unsigned short*)a.vc + kv_row + d) = __half_as_ushort(vh);
      vx[d] = __half2float(vh);
    }
  }
  CHONK_MV_T(tr, 4);
  constexpr int NW = 4;  // words per thread per pass
  const uint64_t t0 = wall_clock64();
  bool late = false;
  for (int base = 0; base < total && !late; base += NW * kWg) {
    for (uint32_t it = 0;; ++it) {
      uint64_t w[NW];
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int e = min(base + tid + k * kWg, total - 1);
        const tagged_t* src;
        if (e < n_ml) {
          const int g = e / (2 * nact), r = e - g * 2 * nact;
          src = rows0 + (size_t)(r >> 1) * rowf + g * (HD + 2) + (r & 1);
        } else {
          const int f = e - n_ml;
          const int g = f / (nd * nact), r = f - g * nd * nact;
          const int dd = r / nact, cc = r - dd * nact;
          src = rows0 + (size_t)cc * rowf + g * (HD + 2) + 2 + d_lo + dd;
        }
        w[k] = tag_get(src);
      }
      int stale = 0;
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const int e = base + tid + k * kWg;
        if (e < total) {
          stale |= !tag_is(w[k], tag);
          if (e < n_ml)
            ml[e] = tag_val(w[k]);
          else
            colv[e - n_ml] = tag_val(w[k]);
        }
      }
      if (!__syncthreads_or(stale)) break;
      if ((it & 3) == 3) {
        const int t_out = tid == 0 && wall_clock64() - t0 > kDecPollTicks;
        if (__syncthreads_or(t_out)) {
          late = true;
          break;
        }
      }
    }
  }
  CHONK_MV_T(tr, 5);
  // (the poll's barriers also publish the rounded k and v)
  for (int g = wave; g < G; g += 4) {
    // the new position's score with the wave's own copy of q head g
    float sn = 0.f;
#pragma unroll
    for (int d = lane; d < HD; d += 64) sn += qw[g * HD + d] * kx[d];
    sn = wave_sum(sn) * a.scale;
    float mv[2], lv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cc = lane + 64 * j;
      mv[j] = cc < nact ? ml[(g * nact + cc) * 2] : -INFINITY;
      lv[j] = cc < nact ? ml[(g * nact + cc) * 2 + 1] : 0.f;
    }
    const float M = fmaxf(wave_max(fmaxf(mv[0], mv[1])), sn);
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int cc = lane + 64 * j;
      const float f = mv[j] == -INFINITY ? 0.f : expf(mv[j] - M);
      if (cc < nact) wts[g * nact + cc] = f;
      L += lv[j] * f;
    }
    const float fn = expf(sn - M);
    L = wave_sum(L) + fn;
    if (lane == 0) {
      wml[2 * g] = 1.0f / L;
      wml[2 * g + 1] = fn;
    }
  }
  __syncthreads();
  // the weighted sum over the chunks of each output element of the slice, by
  // tpi lanes per element (every tpi-th chunk each, then a DPP sum): the
  // workgroup's lanes spread over the G * nd elements
  const int n_el = G * nd;
  int tpi = 1;
  while (tpi < 64 && 2 * tpi * n_el <= kWg && tpi < nact) tpi *= 2;
  for (int base = 0; base < n_el * tpi; base += kWg) {
    const int q = base + tid;
    const int i = q / tpi, sub = q & (tpi - 1);
    if (i < n_el) {
      const int g = i / nd, dd = i - g * nd;
      const float* src = colv + (size_t)(g * nd + dd) * nact;
      const float* wv = wts + g * nact;
      float a0 = 0.f, a1 = 0.f;
      int cc = sub;
      for (; cc + tpi < nact; cc += 2 * tpi) {
        a0 += src[cc] * wv[cc];
        a1 += src[cc + tpi] * wv[cc + tpi];
      }
      if (cc < nact) a0 += src[cc] * wv[cc];
      const float sum = group_sum_n(a0 + a1, tpi);
      if (sub == 0) {
        const float acc = sum + wml[2 * g + 1] * vx[d_lo + dd];
        a.out[(size_t)kv * G * HD + g * HD + d_lo + dd] = acc * wml[2 * g];
      }
    }
  }
  if (late && tid == 0) st->error = 4;
  CHONK_MV_T(tr, 6);
  CHONK_MV_TRACE_END(tr, 7 * 65536);
  // every producer of this launch has read the tag once all rows carry it:
  // the newest chunk advances the epoch for the next launch
  if (c != c_hi) return;
  if (tid == 0) __hip_atomic_store(gblw(&a.cnt[kv]), tag + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool attn_dec_supported(int group, int hd, int ctx, int kv_f16) {
  // (group 8 at head_dim 256 would spill its score operands)
  return kv_f16 && (hd == 64 || hd == 128 || hd == 256) && group >= 1 && group <= 8 && group * hd <= 1536 &&
         (ctx + kDecChunk - 1) / kDecChunk <= 128;
}

int attn_dec_chunk() { return kDecChunk; }

size_t attn_dec_shared_bytes(int group, int hd, int nchunk) {
  // merge buffers: (max, sum) and weights per (head, chunk), the acc words of
  // ceil(hd / nact) dims per head and chunk (at most hd + nact per head)
  const size_t merge = (size_t)group * (3 * (size_t)nchunk + hd + nchunk);
  const size_t area = std::max((size_t)4 * group * hd, merge);
  return sizeof(float) * ((size_t)(group + 4) * hd + (size_t)4 * group * hd + 4 * group * kDecWave + 8 * group + area);
}

namespace {
// cs[p][d] = (cos, sin) of the rotary angle p * inv[d], the expression the
// decode and prompt kernels evaluate inline.
__global__ __launch_bounds__(kWg) void k_rope_cs(const float* inv, int half, int ctx, float2* cs) {
  const int64_t i = (int64_t)blockIdx.x * kWg + threadIdx.x;
  if (i >= (int64_t)ctx * half) return;
  const int p = (int)(i / half), d = (int)(i % half);
  const float ang = __fmul_rn((float)p, inv[d]);
  cs[i] = make_float2(cosf(ang), sinf(ang));
}

template <int G, int HD>
const void* dec_fn() {
  return (const void*)k_attn_dec<G, HD>;
}
const void* dec_kernel(int group, int hd) {
#define CHONK_DEC_FN(GG)                              \
  if (group == GG) {                                  \
    if (hd == 64) return dec_fn<GG, 64>();            \
    if (hd == 128) return dec_fn<GG, 128>();          \
    if (hd == 256) return dec_fn<GG, 256>();          \
  }
  CHONK_DEC_FN(1)
  CHONK_DEC_FN(2)
  CHONK_DEC_FN(3)
  CHONK_DEC_FN(4)
  CHONK_DEC_FN(5)
  CHONK_DEC_FN(6)
  CHONK_DEC_FN(7)
  CHONK_DEC_FN(8)
#undef CHONK_DEC_FN
  return nullptr;
}
}  // namespace

int attn_dec_resident(int device, int group, int hd, size_t shmem) {
  const void* f = dec_kernel(group, hd);
  if (!f) return 0;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, kWg, shmem) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return per_cu * cus;
}

hipError_t launch_rope_cs(const float* inv, int half, int ctx, float2* cs, hipStream_t s) {
  const int64_t n = (int64_t)ctx * half;
  hipLaunchKernelGGL(k_rope_cs, dim3((unsigned)((n + kWg - 1) / kWg)), dim3(kWg), 0, s, inv, half, ctx, cs);
  return hipGetLastError();
}

hipError_t launch_attn_dec(const AttnArgs& a, size_t shmem, hipStream_t s) {
  const int group = a.heads / a.kv_heads;
  const dim3 grid(a.kv_heads, a.nchunk);
#define CHONK_DEC_CASE(GG, HH) \
  if (group == GG && a.hd == HH) { hipLaunchKernelGGL((k_attn_dec<GG, HH>), grid, dim3(kWg), shmem, s, a); return hipGetLastError(); }
#define CHONK_DEC_G(GG) CHONK_DEC_CASE(GG, 64) CHONK_DEC_CASE(GG, 128) CHONK_DEC_CASE(GG, 256)
  CHONK_DEC_G(1)
  CHONK_DEC_G(2)
  CHONK_DEC_G(3)
  CHONK_DEC_G(4)
  CHONK_DEC_G(5)
  CHONK_DEC_G(6)
  CHONK_DEC_G(7)
  CHONK_DEC_G(8)
#undef CHONK_DEC_G
#undef CHONK_DEC_CASE
  return hipErrorInvalidValue;
}

}  // namespace chonk
