// Decode-step kernels for gfx950 (wave64, 256-thread workgroups).
//
// Reference semantics (src/lib/llama-wgsl-runtime.ts):
//   RMSNorm / add+RMSNorm       :1910-1992   out = (in * rsqrt(mean(in^2) + eps)) * w
//   GGUF dequant-matvec         :2202-2613   y[n] = sum_k x[k] * w(n, k)
//   embedding gather            :2615-2866   out[k] = w(token, k) * EMBEDDING_SCALE
//   qk-norm + RoPE + K/V store  :2868-3383   angle = pos * theta^(-2d/hd); split or interleaved pairs
//   attention score / value     :3385-3490   softmax(q.K * 1/sqrt(hd)) . V over [start, pos]
//   add / add-clamp / SiLU / GELU-tanh :3492-3599
//   argmax stage 1 / 2          :3645-3791   ties -> lower id, NaN never wins, penalty on listed ids
// and the candidate sampler of src/lib/sampling.ts:23-76.
//
// The work decomposition is our own: weights are streamed as 32-element units
// by lane groups holding the activation vector in LDS; attention is split over
// 'chunk'-position slices of the context with a last-arriver combine; the
// final group argmax is fused into the lm_head matvec epilogue.
#include <hip/hip_runtime.h>

#include <cmath>

#include "kernels.h"
#include "qdot.h"

namespace chonk {

namespace {

constexpr float kNegBig = -3.402823e38f;  // the WGSL literal -3.402823e38

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

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
  return (bits[id >> 5] >> (id & 31u)) & 1u;
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
// matvec prologue: activation vector into LDS (xs) plus 16-element run sums.
__device__ void mv_prologue(const MvArgs& a, float* xs, float* xs16, float* red) {
  const int K = a.k, tid = threadIdx.x;
  if (a.pro == PRO_PLAIN || a.pro == PRO_NORM) {
    for (int i = tid; i < K; i += kWg) xs[i] = a.in[i];
  } else if (a.pro == PRO_EMBED_NORM) {
    int tok = a.hist[a.st->pos];
    if (tok < 0 || tok >= a.vocab) {
      if (tid == 0 && blockIdx.x == 0) a.st->error = 2;
      tok = 0;
    }
    const int U = K / 32;
    with_type(a.embed.type, [&]<int T>() {
      for (int u = tid; u < U; u += kWg) {
        const Frag<T> f = load_unit<T>(a.embed, tok, u);
        float v[32];
        dequant_unit<T>(f, u, v);
#pragma unroll
        for (int e = 0; e < 32; ++e) xs[unit_col<T>(u, e)] = __fmul_rn(v[e], a.embed_scale);
      }
    });
  } else {  // PRO_RES_NORM
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) {
      const float d = a.delta[i];
      ss += d * d;
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) {
      const float nd = __fmul_rn(__fmul_rn(a.delta[i], inv), a.w_delta[i]);
      const float r = __fadd_rn(a.in[i], nd);
      xs[i] = fminf(fmaxf(r, -65000.0f), 65000.0f);
    }
  }
  __syncthreads();
  if (a.pro != PRO_PLAIN) {
    if ((a.pro == PRO_EMBED_NORM || a.pro == PRO_RES_NORM) && blockIdx.x == 0) {
      for (int i = tid; i < K; i += kWg) a.res_out[i] = xs[i];
    }
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += xs[i] * xs[i];
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), a.w_norm[i]);
    __syncthreads();
  }
  for (int j = tid; j < K / 16; j += kWg) {
    const float4* p = (const float4*)(xs + 16 * j);
    const float4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
    xs16[j] = ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
              ((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w));
  }
  __syncthreads();
}

// Rows [t0, t0 + nt) of segment g (2*nt interleaved gate/up rows when glu);
// row results into res[] (virtual row order).
template <int T>
__device__ void mv_core(const MvSeg& g, bool glu, int t0, int nt, const float* xs, const float* xs16, float* res) {
  const int U = g.w.k >> 5;
  const int lpr = g.lpr;
  const int shift = __builtin_ctz((unsigned)lpr);
  const int ng = kWg >> shift;
  const int lg = threadIdx.x >> shift, li = threadIdx.x & (lpr - 1);
  const int nv = glu ? 2 * nt : nt;
  for (int v0 = lg; v0 < nv; v0 += 2 * ng) {
    const int v1 = v0 + ng;
    const bool has1 = v1 < nv;
    const QMat& m0 = (glu && (v0 & 1)) ? g.w2 : g.w;
    const QMat& m1 = (glu && (v1 & 1)) ? g.w2 : g.w;
    const int r0 = t0 + (glu ? (v0 >> 1) : v0);
    const int r1 = t0 + (glu ? (v1 >> 1) : v1);
    float a0 = 0.f, a1 = 0.f;
    for (int u = li; u < U; u += lpr) {
      const Frag<T> f0 = load_unit<T>(m0, r0, u);
      Frag<T> f1;
      if (has1) f1 = load_unit<T>(m1, r1, u);
      a0 += dot_unit<T>(f0, u, xs, xs16);
      if (has1) a1 += dot_unit<T>(f1, u, xs, xs16);
    }
    for (int off = lpr >> 1; off > 0; off >>= 1) {
      a0 += __shfl_xor(a0, off, 64);
      a1 += __shfl_xor(a1, off, 64);
    }
    if (li == 0) {
      res[v0] = a0;
      if (has1) res[v1] = a1;
    }
  }
}

__global__ __launch_bounds__(kWg) void k_matvec(const MvArgs a) {
  extern __shared__ __align__(16) float smem[];
  if (a.st->stopped) return;
  const int K = a.k;
  float* xs = smem;
  float* xs16 = xs + K;
  float* red = xs16 + K / 16;      // 4 floats (padded to 8)
  float* res = red + 8;            // up to max(2*tile, 256) floats
  int s = 0;
  if (a.nseg > 1 && (int)blockIdx.x >= a.seg[1].wg_begin) s = 1;
  if (a.nseg > 2 && (int)blockIdx.x >= a.seg[2].wg_begin) s = 2;
  const MvSeg& g = s == 0 ? a.seg[0] : (s == 1 ? a.seg[1] : a.seg[2]);

  mv_prologue(a, xs, xs16, red);

  const int t0 = ((int)blockIdx.x - g.wg_begin) * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  const bool glu = a.epi == EPI_GLU_SILU || a.epi == EPI_GLU_GELU;
  if (nt > 0) {
    with_type(g.w.type, [&]<int T>() { mv_core<T>(g, glu, t0, nt, xs, xs16, res); });
  }
  __syncthreads();

  const int tid = threadIdx.x;
  switch (a.epi) {
    case EPI_STORE:
      for (int t = tid; t < nt; t += kWg) g.out[t0 + t] = res[t];
      break;
    case EPI_ADD:
      for (int t = tid; t < nt; t += kWg) g.out[t0 + t] = __fadd_rn(g.add[t0 + t], res[t]);
      break;
    case EPI_GLU_SILU:
      for (int t = tid; t < nt; t += kWg) g.out[t0 + t] = silu_mul(res[2 * t], res[2 * t + 1]);
      break;
    case EPI_GLU_GELU:
      for (int t = tid; t < nt; t += kWg) g.out[t0 + t] = __fmul_rn(gelu_tanh(res[2 * t]), res[2 * t + 1]);
      break;
    case EPI_LOGITS: {
      // tile == 256: one ARGMAX_STAGE1 group per workgroup
      float* vals = res + 256;
      uint32_t* idx = (uint32_t*)(vals + 256);
      float v = kNegBig;
      uint32_t id = 0xffffffffu;
      const int row = t0 + tid;
      if (tid < nt && row < a.vocab) {
        v = res[tid];
        g.out[row] = v;
        if (a.samp->stage1_penalty && bit_test(a.pen_bits, (uint32_t)row)) {
          const float p = a.samp->stage1_pen;
          v = v > 0.0f ? __fdiv_rn(v, p) : __fmul_rn(v, p);
        }
        id = (uint32_t)row;
      }
      vals[tid] = v;
      idx[tid] = id;
      __syncthreads();
      for (int stride = 128; stride >= 1; stride >>= 1) {
        if (tid < stride) {
          const float ov = vals[tid + stride];
          const uint32_t oi = idx[tid + stride];
          if (better(ov, oi, vals[tid], idx[tid])) {
            vals[tid] = ov;
            idx[tid] = oi;
          }
        }
        __syncthreads();
      }
      if (tid == 0) {
        Candidate c;
        c.value = vals[0];
        c.index = idx[0];
        a.cand[(int)blockIdx.x - g.wg_begin] = c;
      }
      break;
    }
  }
  if (a.advance_pos && blockIdx.x == 0 && tid == 0) a.st->pos = a.st->pos + 1;
}

// ---------------------------------------------------------------------------
// GQA decode attention over a chunk of positions, one workgroup per
// (kv head, chunk). Requires hd in {32, 64, 128, 256}, G <= 8.
constexpr int kMaxG = 8;

__device__ __forceinline__ void load8(const void* cache, int kv_f16, size_t off, float out[8]) {
  if (kv_f16) {
    const uint4 raw = *(const uint4*)((const __half*)cache + off);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = h2f(w[i]);
      out[2 * i + 1] = h2f(w[i] >> 16);
    }
  } else {
    const float4* p = (const float4*)((const float*)cache + off);
    const float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

template <int G>
__global__ __launch_bounds__(kWg) void k_attention(const AttnArgs a) {
  extern __shared__ __align__(16) float sm[];
  DevState* st = a.st;
  if (st->stopped) return;
  const int pos = st->pos;
  if (pos >= a.ctx) {
    if (threadIdx.x == 0) st->error = 1;
    return;
  }
  const int kv = blockIdx.x, c = blockIdx.y;
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_lo = start / a.chunk, c_hi = pos / a.chunk;
  if (c < c_lo || c > c_hi) return;

  const int hd = a.hd, half = hd / 2, CH = a.chunk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* q_s = sm;                 // [G][hd]
  float* k_new = q_s + G * hd;     // [hd]
  float* v_new = k_new + hd;       // [hd]
  float* sc_s = v_new + hd;        // [G][CH]
  float* ml_s = sc_s + G * CH;     // [G][2]
  float* red = ml_s + 2 * kMaxG;   // [(256 / (hd/8))][G][hd]
  __shared__ uint32_t s_last;

  const bool own_new = (c == c_hi);
  const float* qraw = a.qkv;
  const float* kraw = a.qkv + a.heads * hd;
  const float* vraw = kraw + a.kv_heads * hd;

  // A: per-head RMSNorm (or copy) of the group's q heads and, in the chunk
  // holding `pos`, of the new k.
  const int nh = G + (own_new ? 1 : 0);
  for (int hh = wave; hh < nh; hh += 4) {
    const bool is_k = hh == G;
    const float* src = is_k ? kraw + kv * hd : qraw + (kv * G + hh) * hd;
    float* dst = is_k ? k_new : q_s + hh * hd;
    const float* w = is_k ? a.kn_w : a.qn_w;
    if (w) {
      float ss = 0.f;
      for (int d = lane; d < hd; d += 64) ss += src[d] * src[d];
      ss = wave_sum(ss);
      const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
      for (int d = lane; d < hd; d += 64) dst[d] = __fmul_rn(__fmul_rn(src[d], inv), w[d]);
    } else {
      for (int d = lane; d < hd; d += 64) dst[d] = src[d];
    }
  }
  if (own_new)
    for (int d = tid; d < hd; d += kWg) v_new[d] = vraw[kv * hd + d];
  __syncthreads();

  // B: rotary embedding in place.
  const int npairs = nh * half;
  for (int i = tid; i < npairs; i += kWg) {
    const int hh = i / half, d = i - hh * half;
    float* base = hh < G ? q_s + hh * hd : k_new;
    const int ia = a.interleaved ? 2 * d : d;
    const int ib = a.interleaved ? 2 * d + 1 : d + half;
    const float e = __fdiv_rn(-2.0f * (float)d, (float)hd);
    const float ang = __fmul_rn((float)pos, powf((float)a.theta, e));
    const float co = cosf(ang), si = sinf(ang);
    const float x0 = base[ia], x1 = base[ib];
    base[ia] = __fsub_rn(__fmul_rn(x0, co), __fmul_rn(x1, si));
    base[ib] = __fadd_rn(__fmul_rn(x0, si), __fmul_rn(x1, co));
  }
  __syncthreads();
  if (own_new) {
    const size_t row = ((size_t)kv * a.ctx + pos) * hd;
    for (int d = tid; d < hd; d += kWg) {
      if (a.kv_f16) {
        const __half kh = __float2half_rn(k_new[d]), vh = __float2half_rn(v_new[d]);
        ((__half*)a.kc)[row + d] = kh;
        ((__half*)a.vc)[row + d] = vh;
        k_new[d] = __half2float(kh);
        v_new[d] = __half2float(vh);
      } else {
        ((float*)a.kc)[row + d] = k_new[d];
        ((float*)a.vc)[row + d] = v_new[d];
      }
    }
  }
  __syncthreads();

  // C: scores of the chunk's positions.
  const int t_begin = max(c * CH, start);
  const int t_end = min(c * CH + CH, pos + 1);
  const int n = t_end - t_begin;
  const int slices = hd >> 3;
  const int ppp = kWg / slices;
  const int sl = tid % slices, pi = tid / slices;
  for (int p0 = 0; p0 < n; p0 += ppp) {
    const int p = p0 + pi;
    float dots[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) dots[gg] = 0.f;
    if (p < n) {
      const int t = t_begin + p;
      float kf[8];
      if (t == pos) {
#pragma unroll
        for (int j = 0; j < 8; ++j) kf[j] = k_new[sl * 8 + j];
      } else {
        load8(a.kc, a.kv_f16, ((size_t)kv * a.ctx + t) * hd + sl * 8, kf);
      }
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        const float* qq = q_s + gg * hd + sl * 8;
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s += qq[j] * kf[j];
        dots[gg] = s;
      }
    }
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
      for (int off = slices >> 1; off > 0; off >>= 1) dots[gg] += __shfl_xor(dots[gg], off, 64);
    if (sl == 0 && p < n) {
      for (int gg = 0; gg < G; ++gg) sc_s[gg * CH + p] = dots[gg] * a.scale;
    }
  }
  __syncthreads();

  // D: chunk-local softmax statistics; sc_s becomes exp(s - m).
  for (int gg = wave; gg < G; gg += 4) {
    float m = -INFINITY;
    for (int p = lane; p < n; p += 64) m = fmaxf(m, sc_s[gg * CH + p]);
    m = wave_max(m);
    float l = 0.f;
    for (int p = lane; p < n; p += 64) {
      const float e = expf(sc_s[gg * CH + p] - m);
      sc_s[gg * CH + p] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml_s[2 * gg] = m;
      ml_s[2 * gg + 1] = l;
    }
  }
  __syncthreads();

  // E: probability-weighted V sum.
  const int pgroups = ppp;
  float acc[G][8];
#pragma unroll
  for (int gg = 0; gg < G; ++gg)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[gg][j] = 0.f;
  for (int p = pi; p < n; p += pgroups) {
    const int t = t_begin + p;
    float vf[8];
    if (t == pos) {
#pragma unroll
      for (int j = 0; j < 8; ++j) vf[j] = v_new[sl * 8 + j];
    } else {
      load8(a.vc, a.kv_f16, ((size_t)kv * a.ctx + t) * hd + sl * 8, vf);
    }
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      const float w = sc_s[gg * CH + p];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[gg][j] += w * vf[j];
    }
  }
#pragma unroll
  for (int gg = 0; gg < G; ++gg)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[((size_t)pi * G + gg) * hd + sl * 8 + j] = acc[gg][j];
  __syncthreads();

  // F: publish the chunk partial (m, l, acc[hd]) per head with write-through
  // stores, then count arrivals; the last chunk to arrive merges all chunks.
  float* part = a.part + ((size_t)(kv * a.nchunk + c) * G) * (hd + 2);
  for (int i = tid; i < G * hd; i += kWg) {
    float s = 0.f;
    for (int q = 0; q < pgroups; ++q) s += red[(size_t)q * G * hd + i];
    const int gg = i / hd, d = i - gg * hd;
    st_relaxed(part + gg * (hd + 2) + 2 + d, s);
  }
  if (tid < G) {
    st_relaxed(part + tid * (hd + 2), ml_s[2 * tid]);
    st_relaxed(part + tid * (hd + 2) + 1, ml_s[2 * tid + 1]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(&a.cnt[kv], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (old == (uint32_t)(c_hi - c_lo)) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  for (int i = tid; i < G * hd; i += kWg) {
    const int gg = i / hd, d = i - gg * hd;
    float M = -INFINITY;
    for (int cc = c_lo; cc <= c_hi; ++cc) {
      const float* pp = a.part + ((size_t)(kv * a.nchunk + cc) * G + gg) * (hd + 2);
      M = fmaxf(M, ld_relaxed(pp));
    }
    float L = 0.f, o = 0.f;
    for (int cc = c_lo; cc <= c_hi; ++cc) {
      const float* pp = a.part + ((size_t)(kv * a.nchunk + cc) * G + gg) * (hd + 2);
      const float f = expf(ld_relaxed(pp) - M);
      L += ld_relaxed(pp + 1) * f;
      o += ld_relaxed(pp + 2 + d) * f;
    }
    a.out[(kv * G + gg) * hd + d] = o / L;
  }
  if (tid == 0) __hip_atomic_store(&a.cnt[kv], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
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

__global__ __launch_bounds__(kWg) void k_select(const SelArgs a) {
  DevState* st = a.st;
  if (st->stopped) return;
  const DevSampling& s = *a.samp;
  const int tid = threadIdx.x;
  __shared__ float vals[kWg];
  __shared__ uint32_t idx[kWg];
  __shared__ double sv[kMaxGroups];
  __shared__ uint32_t sg[kMaxGroups];
  __shared__ int s_int[4];
  int token = 0;
  const int groups = a.groups;

  if (s.sample_mode == 0) {
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

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kWg) void k_dequant(const QMat w, float* out) {
  const int U = w.k >> 5;
  const long long unit = (long long)blockIdx.x * kWg + threadIdx.x;
  if (unit >= (long long)w.n * U) return;
  const int row = (int)(unit / U), u = (int)(unit % U);
  with_type(w.type, [&]<int T>() {
    const Frag<T> f = load_unit<T>(w, row, u);
    float v[32];
    dequant_unit<T>(f, u, v);
#pragma unroll
    for (int e = 0; e < 32; ++e) out[(size_t)row * w.k + unit_col<T>(u, e)] = v[e];
  });
}

__global__ __launch_bounds__(kWg) void k_fill_kv(void* kc, void* vc, int kv_heads, int ctx, int hd, int pos,
                                                 int kv_f16, uint64_t seed) {
  const size_t total = (size_t)kv_heads * pos * hd;
  for (size_t i = (size_t)blockIdx.x * kWg + threadIdx.x; i < total; i += (size_t)gridDim.x * kWg) {
    const size_t h = i / ((size_t)pos * hd), rem = i % ((size_t)pos * hd);
    const size_t dst = h * (size_t)ctx * hd + rem;
    const uint64_t z = mix64(seed + i * 0x9e3779b97f4a7c15ull);
    const float v = (float)((z >> 40) & 0xffff) / 65536.0f - 0.5f;
    if (kv_f16) {
      ((__half*)kc)[dst] = __float2half_rn(v);
      ((__half*)vc)[dst] = __float2half_rn(-v);
    } else {
      ((float*)kc)[dst] = v;
      ((float*)vc)[dst] = -v;
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
int pick_lpr(int units) {
  if (units <= 64) {
    int l = 1;
    while (l < units) l <<= 1;
    return l < 4 ? 4 : l;
  }
  const int slots64 = (units + 63) / 64 * 64, slots32 = (units + 31) / 32 * 32;
  return slots32 < slots64 ? 32 : 64;
}

size_t mv_shared_bytes(int k, int max_tile_rows) {
  const int res = max_tile_rows * 2 > 768 ? max_tile_rows * 2 : 768;  // GLU rows or logits scratch
  return sizeof(float) * ((size_t)k + (size_t)k / 16 + 8 + (size_t)res);
}

size_t attn_shared_bytes(int group, int hd, int chunk) {
  const int pgroups = kWg / (hd / 8);
  return sizeof(float) * ((size_t)group * hd + 2 * (size_t)hd + (size_t)group * chunk + 2 * kMaxG +
                          (size_t)pgroups * group * hd);
}

namespace {
size_t g_lds_limit = 64 * 1024;
}

size_t lds_limit() { return g_lds_limit; }

hipError_t init_kernel_attributes() {
  // Raise the dynamic LDS limit to what the device grants per block; keep the
  // 64 KiB default when the runtime refuses.
  int dev = 0, max_optin = 0, max_block = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  (void)hipDeviceGetAttribute(&max_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  (void)hipDeviceGetAttribute(&max_optin, hipDeviceAttributeSharedMemPerBlockOptin, dev);
  const int want = max_optin > max_block ? max_optin : max_block;
  const void* fns[9] = {(const void*)k_matvec,       (const void*)k_attention<1>, (const void*)k_attention<2>,
                        (const void*)k_attention<3>, (const void*)k_attention<4>, (const void*)k_attention<5>,
                        (const void*)k_attention<6>, (const void*)k_attention<7>, (const void*)k_attention<8>};
  bool raised = want > 64 * 1024;
  for (const void* f : fns) {
    if (!raised) break;
    // the attention kernels hold a few bytes of static LDS
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, want - 256) != hipSuccess) raised = false;
  }
  (void)hipGetLastError();
  g_lds_limit = raised ? (size_t)want - 256 : 64 * 1024;
  return hipSuccess;
}

hipError_t launch_matvec(const MvArgs& a, int grid, size_t shmem, hipStream_t s) {
  hipLaunchKernelGGL(k_matvec, dim3(grid), dim3(kWg), shmem, s, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, size_t shmem, hipStream_t s) {
  const int group = a.heads / a.kv_heads;
  const dim3 grid(a.kv_heads, a.nchunk);
  switch (group) {
    case 1: hipLaunchKernelGGL(k_attention<1>, grid, dim3(kWg), shmem, s, a); break;
    case 2: hipLaunchKernelGGL(k_attention<2>, grid, dim3(kWg), shmem, s, a); break;
    case 3: hipLaunchKernelGGL(k_attention<3>, grid, dim3(kWg), shmem, s, a); break;
    case 4: hipLaunchKernelGGL(k_attention<4>, grid, dim3(kWg), shmem, s, a); break;
    case 5: hipLaunchKernelGGL(k_attention<5>, grid, dim3(kWg), shmem, s, a); break;
    case 6: hipLaunchKernelGGL(k_attention<6>, grid, dim3(kWg), shmem, s, a); break;
    case 7: hipLaunchKernelGGL(k_attention<7>, grid, dim3(kWg), shmem, s, a); break;
    case 8: hipLaunchKernelGGL(k_attention<8>, grid, dim3(kWg), shmem, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_select(const SelArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_select, dim3(1), dim3(kWg), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dequant(const QMat& w, float* out, hipStream_t s) {
  const long long units = (long long)w.n * (w.k / 32);
  const int grid = (int)((units + kWg - 1) / kWg);
  hipLaunchKernelGGL(k_dequant, dim3(grid), dim3(kWg), 0, s, w, out);
  return hipGetLastError();
}

hipError_t launch_fill_kv(void* kc, void* vc, int kv_heads, int ctx, int hd, int pos, int kv_f16, uint64_t seed,
                          hipStream_t s) {
  if (pos <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_kv, dim3(1024), dim3(kWg), 0, s, kc, vc, kv_heads, ctx, hd, pos, kv_f16, seed);
  return hipGetLastError();
}

}  // namespace chonk
