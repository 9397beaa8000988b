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

#include <algorithm>
#include <cmath>

#include "attn_dec_body.h"
#include "kernel_common.h"
#include "kernels.h"
#include "qdot.h"

namespace chonk {

namespace {

// This workgroup's segment, picked field by field (forming a reference into
// the argument block would make the compiler copy the whole block to scratch).

// ONE: a single-segment launch (the host checks nseg == 1): the fields come
// straight from seg[0], so the kernel's argument loads are one round of scalar
// loads instead of two (the segment index, then that segment's fields).
template <bool ONE = false>
__device__ __forceinline__ SegView seg_view(const MvArgs& a, int b) {
  const bool s1 = !ONE && a.nseg > 1 && b >= a.seg[1].wg_begin;
  const bool s2 = !ONE && a.nseg > 2 && b >= a.seg[2].wg_begin;
#define CHONK_PICK(f) (s2 ? a.seg[2].f : (s1 ? a.seg[1].f : a.seg[0].f))
  SegView v;
  v.w.s0 = CHONK_PICK(w.s0);
  v.w.s1 = CHONK_PICK(w.s1);
  v.w.s2 = CHONK_PICK(w.s2);
  v.w.s3 = CHONK_PICK(w.s3);
  v.w.type = CHONK_PICK(w.type);
  v.w.n = CHONK_PICK(w.n);
  v.w.k = CHONK_PICK(w.k);
  v.w.pad = 0;
  v.u0 = CHONK_PICK(w2.s0);
  v.u1 = CHONK_PICK(w2.s1);
  v.u2 = CHONK_PICK(w2.s2);
  v.u3 = CHONK_PICK(w2.s3);
  v.out = CHONK_PICK(out);
  v.add = CHONK_PICK(add);
  v.bias = CHONK_PICK(bias);
  v.n_out = CHONK_PICK(n_out);
  v.tile = CHONK_PICK(tile);
  v.lpr = CHONK_PICK(lpr);
  v.wg_begin = CHONK_PICK(wg_begin);
  v.tag_div = CHONK_PICK(tag_div);
#undef CHONK_PICK
  return v;
}

// LDS layout of the matvec kernels (floats):
//   xs[K] | wn[K] | dl[K] | wd[K] | xs16[K/16] | red[8] | res[...]
struct MvLds {
  float *xs, *wn, *dl, *wd, *xs16, *red, *res;
};

__device__ __forceinline__ MvLds mv_lds(float* smem, int K) {
  MvLds l;
  l.xs = smem;
  l.wn = smem + K;
  l.dl = smem + 2 * K;
  l.wd = smem + 3 * K;
  l.xs16 = smem + 4 * K;
  l.red = l.xs16 + K / 16;
  l.res = l.red + 8;
  return l;
}

// The prologue's inputs, copied out of the kernel arguments once: every typed
// variant of the matvec inlines the prologue, and reading the argument block
// from all of them makes the compiler stage the whole block in scratch.
struct MvPro {
  const float *in, *delta, *w_delta, *w_norm, *norm_b, *pos_embd;
  float* res_out;
  QMat embed;
  const int32_t* hist;
  DevState* st;
  float embed_scale, eps;
  int32_t pro, k, vocab;
};

__device__ __forceinline__ MvPro mv_pro(const MvArgs& a) {
  MvPro p;
  p.in = a.in;
  p.delta = a.delta;
  p.w_delta = a.w_delta;
  p.w_norm = a.w_norm;
  p.norm_b = a.norm_b;
  p.pos_embd = a.pos_embd;
  p.res_out = a.res_out;
  p.embed = a.embed;
  p.hist = a.hist;
  p.st = a.st;
  p.embed_scale = a.embed_scale;
  p.eps = a.eps;
  p.pro = a.pro;
  p.k = a.k;
  p.vocab = a.vocab;
  return p;
}

// Issues the activation loads of the prologue (no waiting).
__device__ __forceinline__ void mv_stage(const MvPro& a, const MvLds& l) {
  const int K = a.k;
  switch (a.pro) {
    case PRO_PLAIN: lds_dma(a.in, l.xs, K); break;
    case PRO_NORM:
      lds_dma(a.in, l.xs, K);
      lds_dma(a.w_norm, l.wn, K);
      break;
    case PRO_RES_NORM:
      lds_dma(a.in, l.xs, K);
      lds_dma(a.delta, l.dl, K);
      lds_dma(a.w_delta, l.wd, K);
      lds_dma(a.w_norm, l.wn, K);
      break;
    case PRO_LN:
      lds_dma(a.in, l.xs, K);
      lds_dma(a.w_norm, l.wn, K);
      lds_dma(a.norm_b, l.wd, K);
      break;
    case PRO_EMBED_LN:  // the row depends on the token
      lds_dma(a.w_norm, l.wn, K);
      lds_dma(a.norm_b, l.wd, K);
      break;
    default:  // PRO_EMBED_NORM: the row depends on the token; only the norm weight is staged
      lds_dma(a.w_norm, l.wn, K);
      break;
  }
}

// Completes the prologue once the staged data has landed: xs becomes the
// matvec input, normalised as the mode requires (ends with a barrier after
// the last write of xs, or with none when xs is the staged input itself).
__device__ __forceinline__ void mv_norm(const MvPro& a, const MvLds& l) {
  const int K = a.k, tid = threadIdx.x;
  float* xs = l.xs;
  if (a.pro == PRO_EMBED_NORM || a.pro == PRO_EMBED_LN) {
    const int pos = a.st->pos;
    int tok = a.hist[pos];
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
    __syncthreads();
    if (a.pro == PRO_EMBED_LN) {
      // ADD_POSITION (gpt-wgsl-runtime.ts:1639-1656)
      for (int i = tid; i < K; i += kWg) xs[i] = __fadd_rn(xs[i], a.pos_embd[(size_t)pos * K + i]);
      __syncthreads();
    }
  } else if (a.pro == PRO_RES_NORM) {
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += l.dl[i] * l.dl[i];
    ss = block_sum(ss, l.red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) {
      const float nd = __fmul_rn(__fmul_rn(l.dl[i], inv), l.wd[i]);
      xs[i] = fminf(fmaxf(__fadd_rn(xs[i], nd), -65000.0f), 65000.0f);
    }
    __syncthreads();
  }
  if (a.pro == PRO_LN || a.pro == PRO_EMBED_LN) {
    // LAYER_NORM_WGSL (gpt-wgsl-runtime.ts:1658-1706): mean and E[x^2] in one
    // pass, variance max(E[x^2] - mean^2, 0), ((x - mean) * inv_std) * w + b
    if (a.pro == PRO_EMBED_LN && blockIdx.x == 0) {
      for (int i = tid; i < K; i += kWg) a.res_out[i] = xs[i];
    }
    float sm = 0.f, sq = 0.f;
    for (int i = tid; i < K; i += kWg) {
      sm += xs[i];
      sq += xs[i] * xs[i];
    }
    sm = block_sum(sm, l.red);
    sq = block_sum(sq, l.red);
    const float mean = sm / (float)K;
    const float var = fmaxf(__fsub_rn(sq / (float)K, __fmul_rn(mean, mean)), 0.0f);
    const float inv = 1.0f / sqrtf(var + a.eps);
    __syncthreads();  // every thread has read xs for the sums
    for (int i = tid; i < K; i += kWg)
      xs[i] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(xs[i], mean), inv), l.wn[i]), l.wd[i]);
    __syncthreads();
  } else if (a.pro != PRO_PLAIN) {
    if ((a.pro == PRO_EMBED_NORM || a.pro == PRO_RES_NORM) && blockIdx.x == 0) {
      for (int i = tid; i < K; i += kWg) a.res_out[i] = xs[i];
    }
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += xs[i] * xs[i];
    ss = block_sum(ss, l.red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), l.wn[i]);
    __syncthreads();
  }
}

// mv_norm, then the integer-digit form of xs (dl) and its 16-element sums.
__device__ __forceinline__ void mv_finish(const MvPro& a, const MvLds& l) {
  mv_norm(a, l);
  quantize_x(l.xs, a.k, l.dl, l.xs16);  // dl / wd are free from here on
  __syncthreads();
}

// Rows [t0, t0 + nt) of the segment (2*nt interleaved gate/up rows when GLU).
// The first weight batch is issued right after the activation staging
// (weights do not depend on it); mv_stream walks the rest.
template <int T, int UC, bool GLU, int AHEAD>
__device__ __forceinline__ bool mv_work(const MvPro& a, const SegView& g, int t0, int nt, const MvLds& l,
                                        uint64_t (&tr)[8]) {
  const MvLane m = mv_lane(g, t0, nt, GLU);
  Frag<T> cur[MvShape<T, UC>::N];
  mv_fetch<T, UC>(g, m, 0, cur);
  const int stopped = __hip_atomic_load(&a.st->stopped, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  CHONK_MV_T(tr, 1);
  if (stopped) return false;
  mv_finish(a, l);
  CHONK_MV_T(tr, 2);
  mv_stream<T, UC, AHEAD>(g, m, xq_view(l.dl, l.xs16, a.k), l.res, cur);
  CHONK_MV_T(tr, 3);
  return true;
}

// TT >= 0: the weight type is known at compile time (the lm_head kernels, one
// per type, so that each allocates only the registers its type needs); AH > 0
// overrides the number of weight batches in flight.
template <int EPI, int TT = -1, int AH = 0>
__device__ __forceinline__ void matvec_body(const MvArgs& a) {
  extern __shared__ __align__(16) float smem[];
  const MvLds l = mv_lds(smem, a.k);
  const SegView g = seg_view(a, (int)blockIdx.x);
  const int t0 = ((int)blockIdx.x - g.wg_begin) * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  constexpr bool glu = EPI == EPI_GLU_SILU || EPI == EPI_GLU_GELU;
  constexpr int ahead = AH > 0 ? AH : (EPI == EPI_LOGITS ? 2 : 1);  // the lm_head's long row streams
  // the type is uniform per workgroup, so every thread takes the same branch
  // (the staging and prologue inside hold barriers)
  bool live = false;
  uint64_t tr[8];
  CHONK_MV_T(tr, 0);
  const MvPro p = mv_pro(a);
  mv_stage(p, l);
  const int uc = mv_uc(g);
  auto work = [&]<int T>() {
    if (uc == 1) {
      live = mv_work<T, 1, glu, ahead>(p, g, t0, nt, l, tr);
    } else {
      live = mv_work<T, 2, glu, ahead>(p, g, t0, nt, l, tr);
    }
  };
  if constexpr (TT >= 0)
    work.template operator()<TT>();
  else
    with_type(g.w.type, work);
  if (!live) return;
  __syncthreads();

  float* res = l.res;
  const int tid = threadIdx.x;
  switch (EPI) {
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
      // tile == 256 (class-major: up to 512): one ARGMAX_STAGE1 group per workgroup
      float* vals = res + 256;
      uint32_t* idx = (uint32_t*)(vals + 256);
      float v = kNegBig;
      uint32_t id = (a.gpt_argmax || a.lfm_classes) ? 0u : 0xffffffffu;
      // lfm2 / granitehybrid: the rows are stored class-major, so workgroup c
      // holds ids c, c + 256, ... in order and its candidate is TOPK256_WGSL's
      // slot c; a class of more than 256 ids (granitehybrid's 100352-entry
      // vocab) gives a thread two rows, tid and tid + 256, scanned in id order
      const int cls = (int)blockIdx.x - g.wg_begin;
      for (int part = 0; part < (a.lfm_classes ? 2 : 1); ++part) {
        const int j = tid + 256 * part;
        const int row = a.lfm_classes ? j * 256 + cls : t0 + j;
        if (j < nt && row < a.vocab) {
          float rv = res[j];
          if (a.logit_scale != 0.f) rv = __fmul_rn(rv, a.logit_scale);  // SCALE_LOGITS_WGSL (granite :1740-1751)
          g.out[row] = rv;
          if (a.samp->stage1_penalty && bit_test(a.pen_bits, (uint32_t)row)) {
            const float p = a.samp->stage1_pen;
            rv = rv > 0.0f ? __fdiv_rn(rv, p) : __fmul_rn(rv, p);
          }
          if (part == 0) {
            v = rv;
            id = (uint32_t)row;
            // (the slot's scan starts from (-3.402823e38, 0) and only a strictly
            // greater logit replaces it: NaN and values at or below it never do)
            if (a.lfm_classes && !(v > kNegBig)) {
              v = kNegBig;
              id = 0u;
            }
          } else if (rv > v) {
            v = rv;
            id = (uint32_t)row;
          }
        }
      }
      // (each thread read only res[tid] and res[tid + 256], the slots written here)
      vals[tid] = v;
      idx[tid] = id;
      __syncthreads();
      // (the GPT-2 runtime's ARGMAX_STAGE1, gpt-wgsl-runtime.ts:1896-1959,
      // keeps the left slot unless the right one is strictly greater)
      for (int stride = 128; stride >= 1; stride >>= 1) {
        if (tid < stride) {
          const float ov = vals[tid + stride];
          const uint32_t oi = idx[tid + stride];
          if (a.gpt_argmax ? ov > vals[tid] : better(ov, oi, vals[tid], idx[tid])) {
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
  CHONK_MV_T(tr, 4);
  CHONK_MV_TRACE_END(tr, EPI * 65536 + a.k);
}

// CONV_BLOCK_WGSL (lfm-wgsl-runtime.ts:1641-1672) for channels 4*i4 .. 4*i4+3:
// cur = B * x, conv = (s1 * w0 + s2 * w1) + cur * w2, out = C * conv, every
// product and sum rounded once as written. proj holds B | C | x (n channels
// each); the taps are [n][3], so four channels' twelve taps are three float4.
__device__ __forceinline__ float4 conv_block4(const float* proj, const float* s1, const float* s2, const float* w,
                                              int n, int i4) {
  const float4 B = ldg4f(proj + 4 * i4), C = ldg4f(proj + n + 4 * i4), X = ldg4f(proj + 2 * n + 4 * i4);
  const float4 p1 = ldg4f(s1 + 4 * i4), p2 = ldg4f(s2 + 4 * i4);
  const float4 wa = ldg4f(w + 12 * i4), wb = ldg4f(w + 12 * i4 + 4), wc = ldg4f(w + 12 * i4 + 8);
  auto ch = [](float b, float c, float x, float q1, float q2, float w0, float w1, float w2) {
    const float cur = __fmul_rn(b, x);
    const float conv = __fadd_rn(__fadd_rn(__fmul_rn(q1, w0), __fmul_rn(q2, w1)), __fmul_rn(cur, w2));
    return __fmul_rn(c, conv);
  };
  return make_float4(ch(B.x, C.x, X.x, p1.x, p2.x, wa.x, wa.y, wa.z), ch(B.y, C.y, X.y, p1.y, p2.y, wa.w, wb.x, wb.y),
                     ch(B.z, C.z, X.z, p1.z, p2.z, wb.z, wb.w, wc.x), ch(B.w, C.w, X.w, p1.w, p2.w, wc.y, wc.z, wc.w));
}

// The state shift of CONV_BLOCK_WGSL (state[s] = p1, state[s+1] = p2,
// state[s+2] = cur: only the last two are ever read back), run by one
// workgroup of a launch that follows every reader of the old state.
__device__ __forceinline__ void conv_commit(const float* proj, float* s1, float* s2, int n) {
  for (int i = (int)threadIdx.x; i < n; i += kWg) {
    const float cur = __fmul_rn(proj[i], proj[2 * n + i]);
    const float prev = s2[i];
    s1[i] = prev;
    s2[i] = cur;
  }
}

// One output row per lane group: lane group lg of lpr lanes owns row t0 + lg
// (GLU: both the gate and the up row), lane li owns units li, li + lpr, ...
// (at most kRowUnits). Every address is computed once, the weight loads are
// issued unconditionally (ragged lanes load a valid unit and drop its
// product), the prologue mode is fixed at compile time and the owning lane
// stores the row's result directly: a short straight path for the decode
// step, whose matvecs are bound by instruction latency rather than bytes.
// GB: 0 llama family; 1 GPT-2 epilogue terms (a per-row bias and the residual sanitize)
// compiled in; 2 as 1 with the input staged through LDS (rows wider than the 4096 that the
// register-resident prologue holds)
// wg: the workgroup's index in the launch's matvec grid (blockIdx.x, or its
// index among the q|k|v workgroups of the fused attention launch).
template <int EPI, int PRO, int GB>
__device__ __forceinline__ void mv_row_body(const MvArgs& a, int wg) {
  // (the q|k|v launches pick one of three segments: their argument lines are
  // warmed first; the fused attention launch, EPI_TAG, warms all of its
  // arguments at entry)
  if constexpr (EPI == EPI_STORE && GB == 0 && (PRO == PRO_NORM || PRO == PRO_EMBED_NORM))
    warm_kernarg<(int)sizeof(MvArgs)>();
  extern __shared__ __align__(16) float smem[];
  constexpr bool glu = EPI == EPI_GLU_SILU || EPI == EPI_GLU_GELU;
  const MvLds l = mv_lds(smem, a.k);
  // (the add and GLU epilogues run single-segment launches)
  constexpr bool one = EPI == EPI_ADD || EPI == EPI_GLU_SILU || EPI == EPI_GLU_GELU || EPI == EPI_GELU;
  // (the q|k|v launches pick one of three segments: their argument lines are warmed first)
  const SegView g = seg_view<one>(a, wg);
  const int t0 = (wg - g.wg_begin) * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  const int lpr = g.lpr;
  const int lg = (int)threadIdx.x >> __builtin_ctz((unsigned)lpr);
  const int li = (int)threadIdx.x & (lpr - 1);
  const bool owner = li == 0 && lg < nt;
  const int row = t0 + min(lg, nt - 1);
  const int U = a.k >> 5;
  // x in the fp32 unit layout (qdot.h): X in dl, the run sums in wd
  float4* xfx = reinterpret_cast<float4*>(l.dl);
  uint64_t tr[8];
  CHONK_MV_T(tr, 0);
  MvPro p = mv_pro(a);
  p.pro = PRO;
  if constexpr (one && (PRO == PRO_PLAIN || PRO == PRO_NORM)) {
    // every kernel argument the loads below need, in one round of scalar loads
    // (left to the scheduler they come in two, the second after the first is
    // awaited): the asm takes them as operands, the barrier keeps the vector
    // loads after it
    asm volatile("" ::"s"(g.w.s0), "s"(g.w.s1), "s"(g.w.s2), "s"(g.w.s3), "s"(g.w.type), "s"(g.w.k), "s"(g.u0),
                 "s"(g.u1), "s"(g.out), "s"(g.add), "s"(t0), "s"(nt), "s"(lpr), "s"(p.in), "s"(p.w_norm), "s"(p.st),
                 "s"(p.k));
    __builtin_amdgcn_sched_barrier(0);
  }
  // plain, norm and convolution prologues keep x (and the norm weight) in
  // registers: thread t holds elements 4 * (t + 256 r) .. + 3 for r < 4 (K <= 4096)
  constexpr bool reg_pro = (PRO == PRO_PLAIN || PRO == PRO_NORM || PRO == PRO_CONV || PRO == PRO_GATE) && GB != 2;
  constexpr bool norm_pro = PRO == PRO_NORM || PRO == PRO_GATE;
  const int n4 = a.k >> 2;
  float4 xv[4], wv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) xv[r] = wv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (reg_pro) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i4 = (int)threadIdx.x + kWg * r;
      if (i4 < n4) {
        if constexpr (PRO == PRO_CONV) {
          xv[r] = conv_block4(a.conv_proj, a.conv_s1, a.conv_s2, a.conv_w, a.k, i4);
        } else if constexpr (PRO == PRO_GATE) {
          // MAMBA_GATE_NORM_WGSL's v = ssm_y * silu(z) (granite-wgsl-runtime.ts:1590-1606)
          const float4 y4 = ldg4f(p.in + 4 * i4), z4 = ldg4f(a.gate_z + 4 * i4);
          auto gz = [](float y, float z) { return __fmul_rn(y, __fdiv_rn(z, __fadd_rn(1.0f, expf(-z)))); };
          xv[r] = make_float4(gz(y4.x, z4.x), gz(y4.y, z4.y), gz(y4.z, z4.z), gz(y4.w, z4.w));
          wv[r] = ldg4f(p.w_norm + 4 * i4);
        } else {
          xv[r] = ldg4f(p.in + 4 * i4);
          if constexpr (PRO == PRO_NORM) wv[r] = ldg4f(p.w_norm + 4 * i4);
        }
      }
    }
  } else {
    mv_stage(p, l);
  }
  float addv = 0.f, biasv = 0.f;
  if constexpr (EPI == EPI_ADD) addv = g.add[row];
  uint32_t tagv = 0;
  if constexpr (EPI == EPI_TAG) tagv = a.tag_epoch[row / g.tag_div];
  if constexpr (GB) {
    if (g.bias) biasv = g.bias[row];
  }
  float rg = 0.f, ru = 0.f;
  bool live = false;
  with_type(g.w.type, [&]<int T>() {
    QMat wu = g.w;
    wu.s0 = g.u0;
    wu.s1 = g.u1;
    wu.s2 = g.u2;
    wu.s3 = g.u3;
    Frag<T> fg[kRowUnits], fu[glu ? kRowUnits : 1];
#pragma unroll
    for (int j = 0; j < kRowUnits; ++j) {
      if (j * lpr < U) {  // uniform
        const int u = min(li + j * lpr, U - 1);
        fg[j] = load_unit<T>(g.w, row, u);
        if constexpr (glu) fu[j] = load_unit<T>(wu, row, u);
      }
    }
    const int stopped = __hip_atomic_load(&p.st->stopped, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (!reg_pro) __syncthreads();
    CHONK_MV_T(tr, 1);
    if (stopped) return;
    if constexpr (reg_pro) {
      if constexpr (norm_pro) {
        float ss = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((int)threadIdx.x + kWg * r < n4)
            ss += (xv[r].x * xv[r].x + xv[r].y * xv[r].y) + (xv[r].z * xv[r].z + xv[r].w * xv[r].w);
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) l.red[threadIdx.x >> 6] = ss;
        __syncthreads();
        CHONK_MV_T(tr, 5);
        ss = (l.red[0] + l.red[1]) + (l.red[2] + l.red[3]);
        const float inv = 1.0f / sqrtf(ss / (float)a.k + p.eps);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          xv[r].x = __fmul_rn(__fmul_rn(xv[r].x, inv), wv[r].x);
          xv[r].y = __fmul_rn(__fmul_rn(xv[r].y, inv), wv[r].y);
          xv[r].z = __fmul_rn(__fmul_rn(xv[r].z, inv), wv[r].z);
          xv[r].w = __fmul_rn(__fmul_rn(xv[r].w, inv), wv[r].w);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i4 = (int)threadIdx.x + kWg * r;
        if (i4 < n4) xf_put<T>(xv[r], i4, U, xfx, l.wd);
      }
      __syncthreads();
    } else {
      mv_norm(p, l);
      xf_build<T>(l.xs, a.k, xfx, l.wd);
      __syncthreads();
    }
    CHONK_MV_T(tr, 2);
    float ag = 0.f, au = 0.f;
#pragma unroll
    for (int j = 0; j < kRowUnits; ++j) {
      const int u = li + j * lpr;
      if (j * lpr < U && u < U) {
        XF xr;
        load_xf(xfx, (const float4*)l.wd, U, u, xr);
        if (j == 0) CHONK_MV_T(tr, 6);
        ag += dot_f<T>(fg[j], u, xr);
        if constexpr (glu) au += dot_f<T>(fu[j], u, xr);
      }
    }
    rg = group_sum_n(ag, lpr);
    if constexpr (glu) ru = group_sum_n(au, lpr);
    CHONK_MV_T(tr, 3);
    live = true;
  });
  if (!live) return;
  if (a.conv_commit && wg == 0) conv_commit(a.conv_proj, a.conv_s1, a.conv_s2, a.conv_n);
  if (owner) {
    if constexpr (GB) {
      if (g.bias) rg = __fadd_rn(rg, biasv);
    }
    if constexpr (EPI == EPI_STORE) g.out[row] = rg;
    if constexpr (EPI == EPI_ADD) {
      // (granitehybrid: ADD_SCALED_WGSL's residual + add * 0.246, granite-wgsl-runtime.ts:1458-1474)
      float y = a.add_scale != 0.f ? __fadd_rn(addv, __fmul_rn(rg, a.add_scale)) : __fadd_rn(addv, rg);
      if (GB && a.sanitize) y = y != y ? 0.0f : fminf(fmaxf(y, -10000.0f), 10000.0f);  // SANITIZE (gpt-wgsl-runtime.ts:1726-1746)
      g.out[row] = y;
    }
    if constexpr (EPI == EPI_GLU_SILU) g.out[row] = silu_mul(rg, ru);
    if constexpr (EPI == EPI_GLU_GELU) g.out[row] = __fmul_rn(gelu_tanh(rg), ru);
    if constexpr (EPI == EPI_GELU) g.out[row] = gelu_tanh(rg);
    if constexpr (EPI == EPI_TAG) tag_put((tagged_t*)g.out + row, rg, tagv);
  }
  if (a.advance_pos && wg == 0 && threadIdx.x == 0) a.st->pos = a.st->pos + 1;
  CHONK_MV_T(tr, 4);
  CHONK_MV_TRACE_END(tr, EPI * 65536 + a.k);
}

#define CHONK_MVR(NAME, EPI, PRO, GB) \
  __global__ __launch_bounds__(kWg) void NAME(const MvArgs a) { mv_row_body<EPI, PRO, GB>(a, (int)blockIdx.x); }
CHONK_MVR(k_mvr_store_plain, EPI_STORE, PRO_PLAIN, 0)
CHONK_MVR(k_mvr_store_norm, EPI_STORE, PRO_NORM, 0)
CHONK_MVR(k_mvr_store_embed, EPI_STORE, PRO_EMBED_NORM, 0)
CHONK_MVR(k_mvr_store_resnorm, EPI_STORE, PRO_RES_NORM, 0)
CHONK_MVR(k_mvr_add_plain, EPI_ADD, PRO_PLAIN, 0)
CHONK_MVR(k_mvr_add_conv, EPI_ADD, PRO_CONV, 0)
CHONK_MVR(k_mvr_add_gate, EPI_ADD, PRO_GATE, 0)
CHONK_MVR(k_mvr_swiglu_norm, EPI_GLU_SILU, PRO_NORM, 0)
CHONK_MVR(k_mvr_swiglu_resnorm, EPI_GLU_SILU, PRO_RES_NORM, 0)
CHONK_MVR(k_mvr_geglu_norm, EPI_GLU_GELU, PRO_NORM, 0)
CHONK_MVR(k_mvr_geglu_resnorm, EPI_GLU_GELU, PRO_RES_NORM, 0)
// gpt2: LayerNorm prologues, biases, GELU-tanh, the sanitized residual add
CHONK_MVR(k_mvr_store_ln, EPI_STORE, PRO_LN, 1)
CHONK_MVR(k_mvr_store_embed_ln, EPI_STORE, PRO_EMBED_LN, 1)
CHONK_MVR(k_mvr_gelu_ln, EPI_GELU, PRO_LN, 1)
CHONK_MVR(k_mvr_add_bias, EPI_ADD, PRO_PLAIN, 1)
CHONK_MVR(k_mvr_add_bias_wide, EPI_ADD, PRO_PLAIN, 2)
#undef CHONK_MVR

// One attention layer's q|k|v matvec and decode attention in one launch.
// Workgroups [0, nq) are the matvec (RMSNorm prologue; each row stored as a
// word tagged with its kv head's epoch, the tag the attention of that head
// polls for); workgroup nq + w is the attention of kv head w % kv_heads, chunk
// w / kv_heads, which requests its K/V rows at entry and polls its group's q,
// k and v words while they are in flight. The matvec workgroups wait for
// nothing, and the engine uses this kernel only when the whole grid fits on
// the device at once (the attention's chunks wait for each other's rows).
template <int G, int HD>
__global__ __launch_bounds__(kWg, 4) void k_qkv_attn(const MvArgs m, const AttnArgs a, int nq) {
  warm_kernarg<(int)(sizeof(MvArgs) + sizeof(AttnArgs) + sizeof(int))>();
  const int b = (int)blockIdx.x;
  if (b < nq) {
    mv_row_body<EPI_TAG, PRO_NORM, 0>(m, b);
    return;
  }
  const int w = b - nq;
  attn_dec_body<G, HD, false, true>(a, w % a.kv_heads, w / a.kv_heads);
}

template <int G, int HD>
const void* qkv_attn_fn() {
  return (const void*)k_qkv_attn<G, HD>;
}
// the instances built: groups 1-4 at head sizes 64 and 128
const void* qkv_attn_kernel(int group, int hd) {
  if (hd != 64 && hd != 128) return nullptr;
  switch (group) {
    case 1: return hd == 64 ? qkv_attn_fn<1, 64>() : qkv_attn_fn<1, 128>();
    case 2: return hd == 64 ? qkv_attn_fn<2, 64>() : qkv_attn_fn<2, 128>();
    case 3: return hd == 64 ? qkv_attn_fn<3, 64>() : qkv_attn_fn<3, 128>();
    case 4: return hd == 64 ? qkv_attn_fn<4, 64>() : qkv_attn_fn<4, 128>();
    default: return nullptr;
  }
}

__global__ __launch_bounds__(kWg) void k_mv_store(const MvArgs a) { matvec_body<EPI_STORE>(a); }
__global__ __launch_bounds__(kWg) void k_mv_add(const MvArgs a) { matvec_body<EPI_ADD>(a); }
__global__ __launch_bounds__(kWg) void k_mv_swiglu(const MvArgs a) { matvec_body<EPI_GLU_SILU>(a); }
__global__ __launch_bounds__(kWg) void k_mv_geglu(const MvArgs a) { matvec_body<EPI_GLU_GELU>(a); }
__global__ __launch_bounds__(kWg) void k_mv_logits(const MvArgs a) { matvec_body<EPI_LOGITS>(a); }
// (Q6_K keeps one batch of rows ahead: with two its fragments take 228
// registers and the 151936-row lm_head ran 4% slower). Three workgroups per
// CU (at most 168 registers, a few spilled): the 594 workgroups of a
// 151936-row lm_head are then all resident at once instead of 512 and a tail
// of 82, and the step ran 0.7% faster.
template <int T>
__global__ __launch_bounds__(kWg, 3) void k_mv_logits_t(const MvArgs a) {
  matvec_body<EPI_LOGITS, T, T == QT_Q6_K ? 1 : 2>(a);
}

// lm_head over the lane-interleaved copy (qdot.h): every lane owns one vocab
// row and walks all of its units, so no cross-lane reduction is needed; the
// wave's 64 rows of one unit are one contiguous run, and every lane reads the
// same x unit from LDS (a broadcast). D units of every lane (and, for the
// K-quants, the next super-block's scales) are in flight while one unit is
// reduced. Workgroup b covers ids [256 b, 256 b + 256) (thread t owns id
// 256 b + t) and ends with ARGMAX_STAGE1 over them, as k_mv_logits.
template <int T, int D>
__device__ __forceinline__ void lm_lanes_body(const MvArgs& a) {
  extern __shared__ __align__(16) float smem[];
  constexpr bool kq = T != QT_Q8_0;  // K-quants: 8 units per super-block of scales
  const MvLds l = mv_lds(smem, a.k);
  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int blk = (int)blockIdx.x * 4 + (tid >> 6);
  const int U = a.k >> 5;
  const QMat w = a.seg[0].w;
  const int SB = U >> 3;  // (K-quants)
  LaneFrag<T> f[D];
  LaneHead<T> ha{}, hb{};
#pragma unroll
  for (int j = 0; j < D; ++j) f[j] = load_lane_frag<T>(w, blk, j, lane);
  if constexpr (kq) {
    ha = load_lane_head<T>(w, blk, 0, lane);
    hb = load_lane_head<T>(w, blk, min(1, SB - 1), lane);
  }
  const MvPro p = mv_pro(a);
  mv_stage(p, l);
  const int stopped = __hip_atomic_load(&p.st->stopped, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (stopped) return;
  mv_norm(p, l);
  float4* XU = reinterpret_cast<float4*>(l.dl);  // 1.125 K floats: dl and the start of wd
  xu_build<T>(l.xs, a.k, XU);
  __syncthreads();
  float acc = 0.f;
  // (each unit register is reloaded right after its unit is reduced, so the
  // D - 1 other units stay in flight; past the last unit the loads repeat
  // unit U - 1 and are dropped, so that every load is unconditional and the
  // loop bodies are straight-line code)
  auto run = [&](int u0, int n, const LaneHead<T>& h) {
    const float4* xg = XU + 9 * u0;
#pragma unroll
    for (int c = 0; c < n; ++c) {
      acc = acc_lane<T>(f[c % D], h, c, xg + 9 * c, acc);
      f[c % D] = load_lane_frag<T>(w, blk, min(u0 + c + D, U - 1), lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (kq) {
    // super-blocks in pairs, their scales in two alternating register sets
    // (ha: even super-blocks, hb: odd), each reloaded two super-blocks ahead
    int sb = 0;
    for (; sb + 1 < SB; sb += 2) {
      run(8 * sb, 8, ha);
      ha = load_lane_head<T>(w, blk, min(sb + 2, SB - 1), lane);
      run(8 * sb + 8, 8, hb);
      hb = load_lane_head<T>(w, blk, min(sb + 3, SB - 1), lane);
    }
    if (sb < SB) run(8 * sb, 8, ha);
  } else {
    for (int u0 = 0; u0 < U; u0 += D) run(u0, D, ha);  // (U is a multiple of D)
  }
  // epilogue: logits, stage-1 penalty and the group argmax (as matvec_body's EPI_LOGITS)
  float* vals = l.res + 256;
  uint32_t* idx = (uint32_t*)(vals + 256);
  const int row = (int)blockIdx.x * 256 + tid;
  float v = kNegBig;
  uint32_t id = a.gpt_argmax ? 0u : 0xffffffffu;
  if (row < a.vocab) {
    float rv = acc;
    if (a.logit_scale != 0.f) rv = __fmul_rn(rv, a.logit_scale);
    a.seg[0].out[row] = rv;
    if (a.samp->stage1_penalty && bit_test(a.pen_bits, (uint32_t)row)) {
      const float pen = a.samp->stage1_pen;
      rv = rv > 0.0f ? __fdiv_rn(rv, pen) : __fmul_rn(rv, pen);
    }
    v = rv;
    id = (uint32_t)row;
  }
  vals[tid] = v;
  idx[tid] = id;
  __syncthreads();
  for (int stride = 128; stride >= 1; stride >>= 1) {
    if (tid < stride) {
      const float ov = vals[tid + stride];
      const uint32_t oi = idx[tid + stride];
      if (a.gpt_argmax ? ov > vals[tid] : better(ov, oi, vals[tid], idx[tid])) {
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
    a.cand[blockIdx.x] = c;
  }
  if (a.advance_pos && blockIdx.x == 0 && tid == 0) a.st->pos = a.st->pos + 1;
}

// D units in flight per lane; the row length in units must be a multiple of D
template <int T, int D>
__global__ __launch_bounds__(kWg, 3) void k_lm_lanes(const MvArgs a) {
  lm_lanes_body<T, D>(a);
}

// ---------------------------------------------------------------------------
// GQA decode attention, one workgroup per (kv head, chunk of positions).
//
//   A  every load that does not depend on the position (the group's q heads,
//      the new k/v, norm weights, rotary table and, for short full-context
//      caches, the chunk's K rows into registers and V rows into LDS) is
//      issued before the position is read.
//   B  one wave per head: q/k RMSNorm + rotary in one pass; the wave holding
//      the new k also stores k/v to the cache.
//   C  each wave owns P = 64/tpp positions (tpp threads per position, each
//      dotting hd/tpp dims), keeps its own softmax max/sum, then walks its
//      positions over V with the weights broadcast by readlane.
//   D  the four wave partials combine into the chunk partial (m, l, acc[hd])
//      in uncached memory; the last chunk of a kv head to arrive merges.
template <int G, bool KV16>
__global__ __launch_bounds__(kWg) void k_attention(const AttnArgs a) {
  extern __shared__ __align__(16) float sm[];
  DevState* st = a.st;
  const int kv = blockIdx.x, c = blockIdx.y;
  const int hd = a.hd, half = hd / 2, CH = a.chunk;
  const int tid = threadIdx.x;
  const int tpp = a.tpp;
  const int my_p = tid / tpp, my_j = tid & (tpp - 1);
  const int dpt = hd / tpp;
  const int t_lo = c * CH;  // positions of this chunk: t_lo + p, p < CH
  constexpr int kElem = KV16 ? 2 : 4;
  constexpr int kVec = KV16 ? 8 : 16;  // 16-byte K vectors per thread, dpt <= 64
  const int nvec = dpt * kElem / 16;
  const int ncp = (a.nchunk + 3) & ~3;

  float* q_s = sm;                 // [G][hd]  raw q, then normalised + rotated
  float* k_new = q_s + G * hd;     // [hd]
  float* v_new = k_new + hd;       // [hd]
  float* qn = v_new + hd;          // [hd] q-norm weight
  float* kn = qn + hd;             // [hd] k-norm weight
  float* inv = kn + hd;            // [hd/2] rotary inverse frequencies (area of hd)
  float* wpart = inv + hd;         // [4][G][hd] wave partials
  float* wml = wpart + 4 * G * hd; // [4][kMaxG][2] wave (max, sum)
  float* wts = wml + 8 * kMaxG;    // [G][ncp] merge weights
  // wts + G * ncp: [rowf] this chunk's partial
  float* tile = wts + G * ncp + attn_rowf(G, hd);  // V rows [CH][hd] (kElem bytes each), later merge staging
  __shared__ uint32_t s_last;

  const float* kraw = a.qkv + a.heads * hd;
  const float* vraw = kraw + a.kv_heads * hd;
  lds_dma(a.qkv + (size_t)kv * G * hd, q_s, G * hd);
  lds_dma(kraw + (size_t)kv * hd, k_new, hd);
  lds_dma(vraw + (size_t)kv * hd, v_new, hd);
  lds_dma(a.rope_inv, inv, half);
  if (a.qn_w) {
    lds_dma(a.qn_w, qn, hd);
    lds_dma(a.kn_w, kn, hd);
  }
  uint4 kreg[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) kreg[v] = make_uint4(0u, 0u, 0u, 0u);
  const size_t head_base = (size_t)kv * a.ctx * hd;
  auto load_chunk = [&](int p_begin, int p_end) {
    // K: this thread's dims of its position, into registers
    const int t = t_lo + my_p;
    if (my_p < CH && my_p >= p_begin && my_p < p_end && t < a.ctx) {
      const uint4* src = (const uint4*)((const uint8_t*)a.kc + (head_base + (size_t)t * hd + my_j * dpt) * kElem);
#pragma unroll
      for (int v = 0; v < kVec; ++v)
        if (v < nvec) kreg[v] = src[v];
    }
    // V: rows [p_begin, p_end) of the chunk, direct to LDS
    const int rows = min(p_end, a.ctx - t_lo) - p_begin;
    if (rows > 0)
      lds_dma((const float*)((const uint8_t*)a.vc + (head_base + (size_t)(t_lo + p_begin) * hd) * kElem),
              (float*)((uint8_t*)tile + (size_t)p_begin * hd * kElem), rows * hd * kElem / 4);
  };
  if (a.spec_kv) load_chunk(0, CH);
  const int stopped = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&st->stopped, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const int pos = __builtin_amdgcn_readfirstlane(
      __hip_atomic_load(&st->pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (stopped) return;
  if (pos >= a.ctx) {
    if (tid == 0) st->error = 1;
    return;
  }
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_lo = start / CH, c_hi = pos / CH;
  if (c < c_lo || c > c_hi) return;
  const int p_begin = max(start - t_lo, 0);  // valid positions: [p_begin, p_end)
  const int p_end = min(pos + 1 - t_lo, CH);
  if (!a.spec_kv) {
    load_chunk(p_begin, p_end);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  attn_compute<G, KV16>(a, sm, kv, c, pos, kreg, &s_last,
                        [&](int i, float v) { a.out[(size_t)kv * G * hd + i] = v; });
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// Mamba2 step of a granitehybrid layer: MAMBA_CONV_WGSL + MAMBA_SSM_WGSL
// (granite-wgsl-runtime.ts:1476-1562) in one launch. Workgroup (n, y) owns the
// 8 channels 8y .. 8y+7 of SSM head n (32 lanes per channel, 4 of the 128
// states per lane). The convolution window of each xBC channel is read from
// the position's parity buffer and shifted into the other one (no reader of
// the old window is ever raced): the workgroup owning an x channel writes its
// window, workgroup (0, 0) those of the shared B and C channels.
constexpr int kSsmHd = 32, kSsmState = 128, kSsmCh = 8;

__global__ __launch_bounds__(kWg) void k_mamba_ssm(const SsmArgs a) {
  __shared__ float sB[kSsmState], sC[kSsmState], sx[kSsmCh], sdt[2];
  const int n = (int)blockIdx.x, c0 = (int)blockIdx.y * kSsmCh, tid = (int)threadIdx.x;
  const int h = tid >> 5, l = tid & 31;
  const int nh = n * kSsmHd + c0 + h;
  // the state rows first: nothing else in this launch writes or depends on them
  float* sp = a.ssm_state + (size_t)nh * kSsmState + l;
  float sv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sv[j] = sp[32 * j];
  const int stopped = __hip_atomic_load(&a.st->stopped, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (stopped) return;
  const int par = a.st->pos & 1;
  const float* cs_old = a.conv_state + (size_t)par * a.conv * 3;
  float* cs_new = a.conv_state + (size_t)(par ^ 1) * a.conv * 3;
  // channel c of xBC: ((((p1 w0 + p2 w1) + p3 w2) + x w3) + bias), then silu
  auto conv_ch = [&](int c, bool write) {
    const float nv = a.proj[a.inner + c];
    const float p1 = cs_old[3 * c], p2 = cs_old[3 * c + 1], p3 = cs_old[3 * c + 2];
    const float4 w = reinterpret_cast<const float4*>(a.conv_w)[c];
    const float y = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(__fmul_rn(p1, w.x), __fmul_rn(p2, w.y)), __fmul_rn(p3, w.z)),
                                        __fmul_rn(nv, w.w)),
                              a.conv_b[c]);
    if (write) {
      cs_new[3 * c] = p2;
      cs_new[3 * c + 1] = p3;
      cs_new[3 * c + 2] = nv;
    }
    return __fdiv_rn(y, __fadd_rn(1.0f, expf(-y)));
  };
  if (tid < 2 * kSsmState) {
    const float v = conv_ch(a.inner + tid, n == 0 && c0 == 0);
    if (tid < kSsmState)
      sB[tid] = v;
    else
      sC[tid - kSsmState] = v;
  }
  // (kWg == 2 * kSsmState: a second pass covers the x channels and dt)
  if (tid < kSsmCh) sx[tid] = conv_ch(n * kSsmHd + c0 + tid, true);
  if (tid == kSsmCh) {
    // softplus as MAMBA_SSM_WGSL selects it, then the decay
    const float x = __fadd_rn(a.proj[a.inner + a.conv + n], a.dt_bias[n]);
    const float dt = x > 20.0f ? __fadd_rn(x, logf(__fadd_rn(1.0f, expf(-x)))) : logf(__fadd_rn(1.0f, expf(x)));
    sdt[0] = dt;
    sdt[1] = expf(__fmul_rn(dt, a.a_neg[n]));
  }
  __syncthreads();
  const float dt = sdt[0], decay = sdt[1], hs = sx[h];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s = l + 32 * j;
    const float next = __fadd_rn(__fmul_rn(sv[j], decay), __fmul_rn(__fmul_rn(dt, sB[s]), hs));
    sp[32 * j] = next;
    acc += next * sC[s];
  }
  acc = group_sum<32>(acc);
  if (l == 0) a.y[nh] = __fadd_rn(acc, __fmul_rn(a.d[n], hs));
}

__global__ __launch_bounds__(kWg) void k_select(const SelArgs a) {
  __shared__ __align__(16) uint8_t ws[kSelectWorkspaceBytes];
  if (a.st->stopped) return;
  select_token(a, ws);
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
  return sizeof(float) * (4 * (size_t)k + (size_t)k / 16 + 8 + (size_t)res);
}

int attn_merge_floats(int group, int hd, int nchunk) {
  // stage up to 32 KiB of chunk partials per batch; the V tile area is reused
  const int rowf = attn_rowf(group, hd);
  return std::min(nchunk * rowf, std::max(8192, rowf));
}

size_t attn_shared_bytes(int group, int hd, int chunk, int nchunk, int kv_elem) {
  const size_t tile = std::max((size_t)chunk * hd * kv_elem / 4, (size_t)attn_merge_floats(group, hd, nchunk));
  const size_t ncp = ((size_t)nchunk + 3) & ~(size_t)3;
  return sizeof(float) * ((size_t)(5 * group + 5) * hd + 8 * kMaxG + (size_t)group * ncp + attn_rowf(group, hd) + tile);
}

int attn_max_chunk(int hd) { return kWg / attn_tpp(hd); }

int attn_threads_per_position(int hd, int chunk, int kv_elem) {
  // enough threads per position to occupy the workgroup, each loading at
  // least one 16-byte K vector
  int t = attn_tpp(hd);
  while (t * chunk < kWg && t * 2 <= hd * kv_elem / 16) t *= 2;
  return t;
}

size_t g_lds_limit = 64 * 1024;

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
  const void* fns[47] = {
      (const void*)k_lm_lanes<QT_Q4_K, 8>,   (const void*)k_lm_lanes<QT_Q6_K, 8>,   (const void*)k_lm_lanes<QT_Q8_0, 4>,
      (const void*)k_lm_lanes<QT_Q8_0, 2>,
      (const void*)k_mvr_add_conv,           (const void*)k_mvr_add_gate,
      (const void*)k_mvr_add_bias,           (const void*)k_mvr_add_bias_wide,
      (const void*)k_mvr_store_ln,           (const void*)k_mvr_store_embed_ln,     (const void*)k_mvr_gelu_ln,
      (const void*)k_mv_logits_t<QT_Q4_K>,   (const void*)k_mv_logits_t<QT_Q5_K>,   (const void*)k_mv_logits_t<QT_Q6_K>,
      (const void*)k_mv_logits_t<QT_Q8_0>,   (const void*)k_mv_logits_t<QT_Q5_0>,   (const void*)k_mv_logits_t<QT_Q5_1>,
      (const void*)k_mvr_store_plain,        (const void*)k_mvr_store_norm,         (const void*)k_mvr_store_embed,
      (const void*)k_mvr_store_resnorm,      (const void*)k_mvr_add_plain,          (const void*)k_mvr_swiglu_norm,
      (const void*)k_mvr_swiglu_resnorm,     (const void*)k_mvr_geglu_norm,         (const void*)k_mvr_geglu_resnorm,
      (const void*)k_mv_store,               (const void*)k_mv_add,                 (const void*)k_mv_swiglu,
      (const void*)k_mv_geglu,               (const void*)k_mv_logits,              (const void*)k_attention<1, true>,
      (const void*)k_attention<2, true>,     (const void*)k_attention<3, true>,     (const void*)k_attention<4, true>,
      (const void*)k_attention<5, true>,     (const void*)k_attention<6, true>,     (const void*)k_attention<7, true>,
      (const void*)k_attention<8, true>,     (const void*)k_attention<1, false>,    (const void*)k_attention<2, false>,
      (const void*)k_attention<3, false>,    (const void*)k_attention<4, false>,    (const void*)k_attention<5, false>,
      (const void*)k_attention<6, false>,    (const void*)k_attention<7, false>,    (const void*)k_attention<8, false>};
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
  if (a.row_kernel) {
    void (*k)(const MvArgs) = nullptr;
    // (the add, GLU and GELU row kernels read segment 0 only)
    if (a.epi != EPI_STORE && a.nseg != 1) return hipErrorInvalidValue;
    bool gb = a.sanitize != 0;
    for (int i = 0; i < a.nseg; ++i) gb = gb || a.seg[i].bias != nullptr;
    const bool ln = a.pro == PRO_LN || a.pro == PRO_EMBED_LN;
    // bias / sanitize need a GB kernel: the GPT-2 set below
    if (gb && !ln && !(a.epi == EPI_ADD && a.pro == PRO_PLAIN)) return hipErrorInvalidValue;
    switch (a.epi * 8 + a.pro) {
      case EPI_STORE * 8 + PRO_PLAIN: k = k_mvr_store_plain; break;
      case EPI_STORE * 8 + PRO_NORM: k = k_mvr_store_norm; break;
      case EPI_STORE * 8 + PRO_EMBED_NORM: k = k_mvr_store_embed; break;
      case EPI_STORE * 8 + PRO_RES_NORM: k = k_mvr_store_resnorm; break;
      case EPI_ADD * 8 + PRO_PLAIN:
        // (rows wider than the register-resident prologue's 4096 stage the input through LDS)
        k = a.k > 4 * 4 * kWg ? k_mvr_add_bias_wide : !gb ? k_mvr_add_plain : k_mvr_add_bias;
        break;
      case EPI_ADD * 8 + PRO_CONV:
        if (gb || a.k > 4 * 4 * kWg) return hipErrorInvalidValue;
        k = k_mvr_add_conv;
        break;
      case EPI_ADD * 8 + PRO_GATE:
        if (gb || a.k > 4 * 4 * kWg) return hipErrorInvalidValue;
        k = k_mvr_add_gate;
        break;
      case EPI_GLU_SILU * 8 + PRO_NORM: k = k_mvr_swiglu_norm; break;
      case EPI_GLU_SILU * 8 + PRO_RES_NORM: k = k_mvr_swiglu_resnorm; break;
      case EPI_GLU_GELU * 8 + PRO_NORM: k = k_mvr_geglu_norm; break;
      case EPI_GLU_GELU * 8 + PRO_RES_NORM: k = k_mvr_geglu_resnorm; break;
      case EPI_STORE * 8 + PRO_LN: k = k_mvr_store_ln; break;
      case EPI_STORE * 8 + PRO_EMBED_LN: k = k_mvr_store_embed_ln; break;
      case EPI_GELU * 8 + PRO_LN: k = k_mvr_gelu_ln; break;
      default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(kWg), shmem, s, a);
    return hipGetLastError();
  }
  switch (a.epi) {
    case EPI_STORE: hipLaunchKernelGGL(k_mv_store, dim3(grid), dim3(kWg), shmem, s, a); break;
    case EPI_ADD: hipLaunchKernelGGL(k_mv_add, dim3(grid), dim3(kWg), shmem, s, a); break;
    case EPI_GLU_SILU: hipLaunchKernelGGL(k_mv_swiglu, dim3(grid), dim3(kWg), shmem, s, a); break;
    case EPI_GLU_GELU: hipLaunchKernelGGL(k_mv_geglu, dim3(grid), dim3(kWg), shmem, s, a); break;
    case EPI_LOGITS:
      if (a.lm_lanes) {
        // the lane-interleaved copy: 256 ids per workgroup
        if (a.nseg != 1 || a.lfm_classes || grid * 256 < a.vocab || a.seg[0].w.n < grid * 256 ||
            (a.seg[0].w.k & (a.seg[0].w.type == QT_Q8_0 ? 31 : 255)) != 0)
          return hipErrorInvalidValue;
        const int U = a.seg[0].w.k >> 5;
        switch (a.seg[0].w.type * 8 + (U % 4 == 0 ? 4 : U % 2 == 0 ? 2 : 0)) {
          case QT_Q4_K * 8 + 4: hipLaunchKernelGGL((k_lm_lanes<QT_Q4_K, 8>), dim3(grid), dim3(kWg), shmem, s, a); break;
          case QT_Q6_K * 8 + 4: hipLaunchKernelGGL((k_lm_lanes<QT_Q6_K, 8>), dim3(grid), dim3(kWg), shmem, s, a); break;
          case QT_Q8_0 * 8 + 4: hipLaunchKernelGGL((k_lm_lanes<QT_Q8_0, 4>), dim3(grid), dim3(kWg), shmem, s, a); break;
          case QT_Q8_0 * 8 + 2: hipLaunchKernelGGL((k_lm_lanes<QT_Q8_0, 2>), dim3(grid), dim3(kWg), shmem, s, a); break;
          default: return hipErrorInvalidValue;
        }
        break;
      }
      // one segment, a type known here: the per-type lm_head kernel
      switch (a.nseg == 1 ? a.seg[0].w.type : -1) {
        case QT_Q4_K: hipLaunchKernelGGL(k_mv_logits_t<QT_Q4_K>, dim3(grid), dim3(kWg), shmem, s, a); break;
        case QT_Q5_K: hipLaunchKernelGGL(k_mv_logits_t<QT_Q5_K>, dim3(grid), dim3(kWg), shmem, s, a); break;
        case QT_Q6_K: hipLaunchKernelGGL(k_mv_logits_t<QT_Q6_K>, dim3(grid), dim3(kWg), shmem, s, a); break;
        case QT_Q8_0: hipLaunchKernelGGL(k_mv_logits_t<QT_Q8_0>, dim3(grid), dim3(kWg), shmem, s, a); break;
        case QT_Q5_0: hipLaunchKernelGGL(k_mv_logits_t<QT_Q5_0>, dim3(grid), dim3(kWg), shmem, s, a); break;
        case QT_Q5_1: hipLaunchKernelGGL(k_mv_logits_t<QT_Q5_1>, dim3(grid), dim3(kWg), shmem, s, a); break;
        default: hipLaunchKernelGGL(k_mv_logits, dim3(grid), dim3(kWg), shmem, s, a); break;
      }
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ssm(const SsmArgs& a, hipStream_t s) {
  // the kernel's fixed geometry: 32-wide heads of 128 states, one x channel
  // per lane group of 32, B | C over the 256 threads
  if (a.inner != a.heads * kSsmHd || a.conv != a.inner + 2 * kSsmState || kWg != 2 * kSsmState)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_mamba_ssm, dim3(a.heads, kSsmHd / kSsmCh), dim3(kWg), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, size_t shmem, hipStream_t s) {
  if (a.variant == 1) return launch_attn_dec(a, shmem, s);
  const int group = a.heads / a.kv_heads;
  const dim3 grid(a.kv_heads, a.nchunk);
#define CHONK_ATTN_CASE(GG)                                                                  \
  case GG:                                                                                   \
    if (a.kv_f16)                                                                            \
      hipLaunchKernelGGL((k_attention<GG, true>), grid, dim3(kWg), shmem, s, a);             \
    else                                                                                     \
      hipLaunchKernelGGL((k_attention<GG, false>), grid, dim3(kWg), shmem, s, a);            \
    break;
  switch (group) {
    CHONK_ATTN_CASE(1)
    CHONK_ATTN_CASE(2)
    CHONK_ATTN_CASE(3)
    CHONK_ATTN_CASE(4)
    CHONK_ATTN_CASE(5)
    CHONK_ATTN_CASE(6)
    CHONK_ATTN_CASE(7)
    CHONK_ATTN_CASE(8)
    default: return hipErrorInvalidValue;
  }
#undef CHONK_ATTN_CASE
  return hipGetLastError();
}

int qkv_attn_resident(int device, int group, int hd, size_t shmem) {
  const void* f = qkv_attn_kernel(group, hd);
  if (!f) return 0;
  // an instance that spills to scratch is not used (0: cannot run)
  hipFuncAttributes at{};
  if (hipFuncGetAttributes(&at, f) != hipSuccess || at.localSizeBytes != 0) return 0;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, kWg, shmem) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return per_cu * cus;
}

hipError_t launch_qkv_attn(const MvArgs& m, int nq, const AttnArgs& a, size_t shmem, hipStream_t s) {
  const int group = a.heads / a.kv_heads;
  const void* f = qkv_attn_kernel(group, a.hd);
  if (!f || a.variant != 1 || a.sub != 1 || !a.qkv_tag || m.epi != EPI_TAG || m.pro != PRO_NORM || !m.row_kernel ||
      nq <= 0)
    return hipErrorInvalidValue;
  void* args[] = {(void*)&m, (void*)&a, (void*)&nq};
  return hipLaunchKernel(f, dim3((unsigned)(nq + a.kv_heads * a.nchunk)), dim3(kWg), args, shmem, s);
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
