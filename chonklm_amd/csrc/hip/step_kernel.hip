// Persistent decode step for gfx950: every phase of one token (q|k|v,
// attention, o_proj, gate|up, down for each layer, then lm_head and token
// selection) in one launch of one workgroup per CU.
//
// The arithmetic of each phase is that of the per-phase kernels in
// kernels.hip (same prologues, dequant-dot units, epilogues, attention
// phases); what changes is the hand-off between phases. A kernel boundary
// costs a launch gap and a cold start; here a workgroup that finishes its
// task of one phase immediately requests the weights (or K/V rows) of its
// next task, which do not depend on the previous phase, and only then waits
// for its input vector. Inputs crossing workgroups are tagged words
// {f32 value, u32 epoch} stored and loaded with agent-scope atomics: the
// consumer polls the words themselves, so a hand-off is one memory round
// trip, with no counter and no cache maintenance.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "kernel_common.h"
#include "kernels.h"
#include "qdot.h"

namespace chonk {
namespace {

// A wait for an input is bounded in time (wall clock, 100 MHz): past the
// bound the step is aborted (DevState.error = 3, details in StepDebug) rather
// than left spinning; every other waiting workgroup then leaves within a few
// polls.
constexpr uint64_t kPollTicks = 20ull * 100000ull;  // 20 ms

__device__ __forceinline__ void tag_store(tagged_t* p, float v, uint32_t tag) {
  __hip_atomic_store(gblw(p), ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Phase and task of the current wait, for the abort record.
struct WaitSite {
  int phase, task;
};

// Up to three tagged ranges copied into LDS by one poll.
struct PollSeg {
  const tagged_t* src;
  float* dst;
  int n;
};

// Copies every segment's src[0, n) into its dst (LDS) once every word carries
// `tag`. All threads of the workgroup call it. Returns false when the step is
// aborted (this wait exceeded its bound, or another workgroup's did). A pass
// over a window of B words per thread issues all of its loads before it
// waits, so it costs one memory round trip; B is small where registers are
// scarce. Every lane issues every load and store (past the end it reads and
// stores the last word again), which keeps the code branch-free and the
// compiler's wait counts exact.
template <int NS, int B>
__device__ __forceinline__ bool poll_segs(const PollSeg (&sg)[NS], uint32_t tag, DevState* st, StepDebug* dbg,
                                          const WaitSite& site, int pos) {
  int total = 0;
#pragma unroll
  for (int q = 0; q < NS; ++q) total += sg[q].n;
  // element e of the concatenation: the last segment that starts at or before
  // e (selects, not an indexed array, so everything stays in registers)
  auto locate = [&](int e, const tagged_t*& src, float*& dst) {
    src = sg[0].src + e;
    dst = sg[0].dst + e;
    int off = e;
#pragma unroll
    for (int r = 1; r < NS; ++r) {
      off -= sg[r - 1].n;
      if (off >= 0) {
        src = sg[r].src + off;
        dst = sg[r].dst + off;
      }
    }
  };
  const uint64_t t0 = wall_clock64();
  for (int base = 0; base < total; base += B * kWg) {
    for (uint32_t it = 0;; ++it) {
      int stale = 0;
      uint64_t w[B];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const tagged_t* src;
        float* dst;
        locate(min(base + (int)threadIdx.x + j * kWg, total - 1), src, dst);
        w[j] = __hip_atomic_load(gbl(src), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const tagged_t* src;
        float* dst;
        locate(min(base + (int)threadIdx.x + j * kWg, total - 1), src, dst);
        stale |= (uint32_t)(w[j] >> 32) != tag;
        *dst = __uint_as_float((uint32_t)w[j]);
      }
      if (!__syncthreads_or(stale)) break;
      if ((it & 3) == 3) {
        int flag = 0;
        bool timeout = false;
        if (threadIdx.x == 0) {
          timeout = wall_clock64() - t0 > kPollTicks;
          flag = timeout || __hip_atomic_load(gbl(&st->error), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
        }
        if (__syncthreads_or(flag)) {
          if (threadIdx.x == 0 && timeout) {
            uint32_t expect = 0;
            if (__hip_atomic_compare_exchange_strong(&dbg->claimed, &expect, 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)) {
              int idx = -1;
              uint32_t seen = 0;
              for (int e = 0; e < total && idx < 0; ++e) {
                const tagged_t* src;
                float* dst;
                locate(e, src, dst);
                const uint64_t v = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((uint32_t)(v >> 32) != tag) {
                  idx = e;
                  seen = (uint32_t)(v >> 32);
                }
              }
              __hip_atomic_store(&dbg->wg, (int32_t)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->phase, site.phase, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->task, site.task, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->index, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->seen, seen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->want, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->pos, pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              __hip_atomic_store(&dbg->abort_time, (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(&st->error, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          return false;
        }
      }
    }
  }
  return true;
}

// The task's segment of a matvec phase, picked field by field.
struct TaskSeg {
  SegView g;
  tagged_t* tout;
  int task;  // task index within the segment
};

__device__ __forceinline__ TaskSeg task_seg(const StepPhase& ph, int t) {
  const bool s1 = ph.nseg > 1 && t >= ph.seg[1].wg_begin;
  const bool s2 = ph.nseg > 2 && t >= ph.seg[2].wg_begin;
#define CHONK_PICK(f) (s2 ? ph.seg[2].f : (s1 ? ph.seg[1].f : ph.seg[0].f))
  TaskSeg r;
  r.g.w.s0 = CHONK_PICK(w.s0);
  r.g.w.s1 = CHONK_PICK(w.s1);
  r.g.w.s2 = CHONK_PICK(w.s2);
  r.g.w.s3 = CHONK_PICK(w.s3);
  r.g.w.type = CHONK_PICK(w.type);
  r.g.w.n = CHONK_PICK(w.n);
  r.g.w.k = CHONK_PICK(w.k);
  r.g.w.pad = 0;
  r.g.u0 = CHONK_PICK(w2.s0);
  r.g.u1 = CHONK_PICK(w2.s1);
  r.g.u2 = CHONK_PICK(w2.s2);
  r.g.u3 = CHONK_PICK(w2.s3);
  r.g.out = nullptr;
  r.g.add = nullptr;
  r.g.n_out = CHONK_PICK(n_out);
  r.g.tile = CHONK_PICK(tile);
  r.g.lpr = CHONK_PICK(lpr);
  r.g.wg_begin = CHONK_PICK(wg_begin);
  r.tout = s2 ? ph.tout[2] : (s1 ? ph.tout[1] : ph.tout[0]);
  r.task = t - r.g.wg_begin;
#undef CHONK_PICK
  return r;
}

// LDS of a matvec task (floats): xs[K] | wn[K] | dl[K] | wd[K] | xs16[K/16] | red[8] | res[R] | addv[tile]
struct StepMvLds {
  float *xs, *wn, *dl, *wd, *xs16, *red, *res, *addv;
};

__device__ __forceinline__ StepMvLds step_mv_lds(float* smem, int K, int res_floats) {
  StepMvLds l;
  l.xs = smem;
  l.wn = smem + K;
  l.dl = smem + 2 * K;
  l.wd = smem + 3 * K;
  l.xs16 = smem + 4 * K;
  l.red = l.xs16 + K / 16;
  l.res = l.red + 8;
  l.addv = l.res + res_floats;
  return l;
}

constexpr int kStepResFloats = 1024;  // matvec row results: >= 2 * tile (GLU) and 768 (logits scratch)

// One matvec task: rows [t0, t0 + nt) of the task's segment. Order: norm
// weights staged and the first weight fragments requested, then the input
// polled, then the prologue, the streaming dot products and the epilogue.
template <int T, int UC>
__device__ __forceinline__ bool mv_task(const StepArgs& a, const StepPhase& ph, const TaskSeg& ts, bool glu, int gtask,
                                        int pos, uint32_t tag, const StepMvLds& l, const WaitSite& ws) {
  const SegView& g = ts.g;
  const int tid = threadIdx.x;
  const int K = ph.k;
  const int t0 = ts.task * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  const MvLane m = mv_lane(g, t0, nt, glu);

  // 1. inputs that do not depend on the previous phase
  if (ph.pro != PRO_PLAIN) lds_dma(ph.w_norm, l.wn, K);
  if (ph.pro == PRO_RES_NORM) lds_dma(ph.w_delta, l.wd, K);
  Frag<T> cur[MvShape<T, UC>::N];
  mv_fetch<T, UC>(g, m, 0, cur);

  // 2. inputs of the previous phases
  {
    const PollSeg sg[3] = {{ph.in, l.xs, ph.pro != PRO_EMBED_NORM ? K : 0},
                           {ph.delta, l.dl, ph.pro == PRO_RES_NORM ? K : 0},
                           {ph.epi == EPI_ADD ? ph.add + t0 : ph.add, l.addv, ph.epi == EPI_ADD ? max(nt, 0) : 0}};
    if (!poll_segs<3, UC == 1 ? 4 : 12>(sg, tag, a.st, a.dbg, ws, pos)) return false;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // 3. prologue (mv_finish of the per-phase kernels)
  float* xs = l.xs;
  if (ph.pro == PRO_EMBED_NORM) {
    // xs holds the embedding row (staged by the caller)
  } else if (ph.pro == PRO_RES_NORM) {
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
  if (ph.pro != PRO_PLAIN) {
    if (ph.pro == PRO_EMBED_NORM || ph.pro == PRO_RES_NORM) {
      // this task's slice of the residual, for the later phases that add to it
      const int S = (K + ph.n_tasks - 1) / ph.n_tasks;
      const int lo = gtask * S, hi = min(K, lo + S);
      for (int i = lo + tid; i < hi; i += kWg) tag_store(ph.res_out + i, xs[i], tag);
    }
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += xs[i] * xs[i];
    ss = block_sum(ss, l.red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), l.wn[i]);
    __syncthreads();
  }
  quantize_x(xs, K, l.dl, l.xs16);  // dl / wd are free from here on
  __syncthreads();

  // 4. dot products (the lm_head's long row streams keep two batches in flight)
  if (ph.epi == EPI_LOGITS)
    mv_stream<T, UC, 2>(g, m, xq_view(l.dl, l.xs16, K), l.res, cur);
  else
    mv_stream<T, UC, 1>(g, m, xq_view(l.dl, l.xs16, K), l.res, cur);
  __syncthreads();

  // 5. epilogue
  const float* res = l.res;
  switch (ph.epi) {
    case EPI_STORE:
      for (int t = tid; t < nt; t += kWg) tag_store(ts.tout + t0 + t, res[t], tag);
      break;
    case EPI_ADD:
      for (int t = tid; t < nt; t += kWg) tag_store(ts.tout + t0 + t, __fadd_rn(l.addv[t], res[t]), tag);
      break;
    case EPI_GLU_SILU:
      for (int t = tid; t < nt; t += kWg) tag_store(ts.tout + t0 + t, silu_mul(res[2 * t], res[2 * t + 1]), tag);
      break;
    case EPI_GLU_GELU:
      for (int t = tid; t < nt; t += kWg)
        tag_store(ts.tout + t0 + t, __fmul_rn(gelu_tanh(res[2 * t]), res[2 * t + 1]), tag);
      break;
    default: {  // EPI_LOGITS, 256 rows per task: one ARGMAX_STAGE1 group
      float* vals = l.res + 256;
      uint32_t* idx = (uint32_t*)(vals + 256);
      float v = kNegBig;
      uint32_t id = 0xffffffffu;
      const int row = t0 + tid;
      if (tid < nt && row < a.vocab) {
        v = res[tid];
        *gblw(ph.logits + row) = v;
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
      if (tid == 0)
        __hip_atomic_store(gblw((uint64_t*)&a.cand[ts.task]), ((uint64_t)idx[0] << 32) | (uint64_t)__float_as_uint(vals[0]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
  }
  return true;
}

// Embedding row of the token at `pos` times the embedding scale, into xs (the
// layer-0 prologue; ggufEmbedding, llama-wgsl-runtime.ts:1326-1342).
__device__ __forceinline__ void embed_into(const StepArgs& a, int pos, int K, float* xs) {
  const int tid = threadIdx.x;
  int tok = a.hist[pos];
  if (tok < 0 || tok >= a.vocab) {
    if (tid == 0) a.st->error = 2;
    tok = 0;
  }
  with_type(a.embed.type, [&]<int TE>() {
    for (int u = tid; u < K / 32; u += kWg) {
      const Frag<TE> f = load_unit<TE>(a.embed, tok, u);
      float v[32];
      dequant_unit<TE>(f, u, v);
#pragma unroll
      for (int e = 0; e < 32; ++e) xs[unit_col<TE>(u, e)] = __fmul_rn(v[e], a.embed_scale);
    }
  });
}

__device__ __forceinline__ bool mv_dispatch(const StepArgs& a, const StepPhase& ph, int t, int pos, uint32_t tag,
                                            float* smem, const WaitSite& ws) {
  const TaskSeg ts = task_seg(ph, t);
  const StepMvLds l = step_mv_lds(smem, ph.k, kStepResFloats);
  if (ph.pro == PRO_EMBED_NORM) embed_into(a, pos, ph.k, l.xs);  // made visible by the task's first barrier
  const bool glu = ph.epi == EPI_GLU_SILU || ph.epi == EPI_GLU_GELU;
  bool ok = true;
  const int uc = mv_uc(ts.g);
  with_type(ts.g.w.type, [&]<int T>() {
    if (uc == 1) {
      ok = mv_task<T, 1>(a, ph, ts, glu, t, pos, tag, l, ws);
    } else {
      ok = mv_task<T, 2>(a, ph, ts, glu, t, pos, tag, l, ws);
    }
  });
  return ok;
}

// One attention task: (kv head, chunk) = (t / nchunk, t % nchunk). Every
// chunk but the newest stores its partial (tagged); the newest chunk's task
// merges the head's partials as they arrive and stores the head's output.
template <int G, bool KV16>
__device__ __forceinline__ bool attn_task(const StepArgs& a, const StepPhase& ph, int t, int pos, uint32_t tag, float* sm,
                                          const WaitSite& ws) {
  const AttnArgs& at = ph.at;
  const int kv = t / at.nchunk, c = t - kv * at.nchunk;
  const int hd = at.hd, CH = at.chunk;
  const int start = (at.window != 0 && pos + 1 > at.window) ? pos + 1 - at.window : 0;
  const int c_lo = start / CH, c_hi = pos / CH;
  if (c < c_lo || c > c_hi) return true;  // chunk outside [start, pos]
  const int tid = threadIdx.x;
  const int tpp = at.tpp;
  const int my_p = tid / tpp, my_j = tid & (tpp - 1);
  const int dpt = hd / tpp;
  const int t_lo = c * CH;
  constexpr int kElem = KV16 ? 2 : 4;
  constexpr int kVec = KV16 ? 8 : 16;
  const int nvec = dpt * kElem / 16;
  const int ncp = (at.nchunk + 3) & ~3;
  const int rowf = attn_rowf(G, hd);
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
  float* tile = cpart + rowf;
  const int p_begin = max(start - t_lo, 0);
  const int p_end = min(pos + 1 - t_lo, CH);

  // K/V rows of the cache (positions before this step): registers and LDS
  lds_dma(at.rope_inv, inv, hd / 2);
  if (at.qn_w) {
    lds_dma(at.qn_w, qn, hd);
    lds_dma(at.kn_w, kn, hd);
  }
  uint4 kreg[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) kreg[v] = make_uint4(0u, 0u, 0u, 0u);
  const size_t head_base = (size_t)kv * at.ctx * hd;
  if (my_p < CH && my_p >= p_begin && my_p < p_end) {
    const uint8_t* src = (const uint8_t*)at.kc + (head_base + (size_t)(t_lo + my_p) * hd + my_j * dpt) * kElem;
#pragma unroll
    for (int v = 0; v < kVec; ++v)
      if (v < nvec) kreg[v] = ldg4(src + 16 * v);
  }
  if (p_end > p_begin)
    lds_dma((const float*)((const uint8_t*)at.vc + (head_base + (size_t)(t_lo + p_begin) * hd) * kElem),
            (float*)((uint8_t*)tile + (size_t)p_begin * hd * kElem), (p_end - p_begin) * hd * kElem / 4);

  // this step's q (group heads), k and v of the head, in one polling pass
  const int qdim = at.heads * hd, kvdim = at.kv_heads * hd;
  {
    const PollSeg sg[3] = {{ph.qkv_in + (size_t)kv * G * hd, q_s, G * hd},
                           {ph.qkv_in + qdim + (size_t)kv * hd, k_new, hd},
                           {ph.qkv_in + qdim + kvdim + (size_t)kv * hd, v_new, hd}};
    if (!poll_segs<3, 2>(sg, tag, a.st, a.dbg, ws, pos)) return false;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  attn_chunk<G, KV16>(at, sm, kv, c, pos, kreg);

  // partial rows [kv][nchunk], rowf words each (padding words carry the tag too)
  tagged_t* rows = ph.tpart + (size_t)kv * at.nchunk * rowf;
  if (c != c_hi) {
    for (int i = tid; i < rowf; i += kWg) tag_store(rows + (size_t)c * rowf + i, i < G * (hd + 2) ? cpart[i] : 0.0f, tag);
    return true;
  }

  // merge of chunks c_lo..c_hi (this one last), in batches of LDS rows with a
  // running maximum: per head [M, rescale of the earlier batches, L] in wml
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nact = c_hi - c_lo + 1;
  const int cap = max(1, min(at.merge_floats / rowf, ncp));
  float* stage = tile;
  float o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = 0.f;
  if (tid < G) {
    wml[3 * tid] = -INFINITY;
    wml[3 * tid + 2] = 0.0f;
  }
  for (int b0 = 0; b0 < nact; b0 += cap) {
    const int nb = min(cap, nact - b0);
    const int n_mem = min(nb, nact - 1 - b0);  // rows of other chunks in this batch
    __syncthreads();  // the previous batch (or the V tile) is consumed
    if (n_mem > 0) {
      const PollSeg sg[1] = {{rows + (size_t)(c_lo + b0) * rowf, stage, n_mem * rowf}};
      if (!poll_segs<1, 17>(sg, tag, a.st, a.dbg, ws, pos)) return false;
    }
    if (n_mem < nb)
      for (int i = tid; i < G * (hd + 2); i += kWg) stage[(size_t)(nb - 1) * rowf + i] = cpart[i];
    __syncthreads();
    for (int gg = wave; gg < G; gg += 4) {
      float mb = -INFINITY;
      for (int cc = lane; cc < nb; cc += 64) mb = fmaxf(mb, stage[cc * rowf + gg * (hd + 2)]);
      mb = wave_max(mb);
      const float M0 = wml[3 * gg];
      const float M = fmaxf(M0, mb);
      float L = 0.f;
      for (int cc = lane; cc < nb; cc += 64) {
        const float* pp = stage + cc * rowf + gg * (hd + 2);
        const float f = expf(pp[0] - M);
        wts[gg * ncp + cc] = f;
        L += pp[1] * f;
      }
      L = wave_sum(L);
      if (lane == 0) {
        const float r = M0 == -INFINITY ? 0.0f : expf(M0 - M);
        wml[3 * gg] = M;
        wml[3 * gg + 1] = r;
        wml[3 * gg + 2] = wml[3 * gg + 2] * r + L;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = tid + q * kWg;
      if (i < G * hd) {
        const int gg = i / hd, d = i - gg * hd;
        const float* src = stage + gg * (hd + 2) + 2 + d;
        const float* wv = wts + gg * ncp;
        float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
        int cc = 0;
        for (; cc + 4 <= nb; cc += 4) {
          acc0 += src[cc * rowf] * wv[cc];
          acc1 += src[(cc + 1) * rowf] * wv[cc + 1];
          acc2 += src[(cc + 2) * rowf] * wv[cc + 2];
          acc3 += src[(cc + 3) * rowf] * wv[cc + 3];
        }
        for (; cc < nb; ++cc) acc0 += src[cc * rowf] * wv[cc];
        o[q] = o[q] * wml[3 * gg + 1] + ((acc0 + acc1) + (acc2 + acc3));
      }
    }
  }
  tagged_t* out = ph.attn_out + (size_t)kv * G * hd;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = tid + q * kWg;
    if (i < G * hd) {
      const int gg = i / hd, d = i - gg * hd;
      tag_store(out + gg * hd + d, o[q] * (1.0f / wml[3 * gg + 2]), tag);
    }
  }
  return true;
}

template <int G, bool KV16>
__global__ __launch_bounds__(kWg, 1) void k_step(const StepArgs* __restrict__ ap, const StepPhase* __restrict__ phases) {
  // both tables live in device memory and are never written by the kernel:
  // their fields are read with scalar loads
  const StepArgs& a = *ap;
  extern __shared__ __align__(16) float smem[];
  __shared__ uint32_t s_flag;
  DevState* st = a.st;
  if (st->stopped) return;
  const int pos = st->pos;
  const uint32_t tag = *a.epoch;
  const int nwg = (int)gridDim.x;
  if (threadIdx.x == 0 && blockIdx.x < 1024)
    __hip_atomic_store(&a.dbg->start[blockIdx.x], (uint64_t)wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (a.trace && threadIdx.x == 0)
    __hip_atomic_store(&a.trace[(size_t)a.n_phases * nwg + blockIdx.x], (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  bool ok = pos < a.sel.ctx;
  if (!ok && threadIdx.x == 0) st->error = 1;
  for (int p = 0; p < a.n_phases && ok; ++p) {
    const StepPhase& ph = phases[p];
    int t = (int)blockIdx.x - ph.rot;
    if (t < 0) t += nwg;
    for (; t < ph.n_tasks && ok; t += nwg) {
      const WaitSite ws{p, t};
      if (ph.kind == PH_ATTN) {
        ok = attn_task<G, KV16>(a, ph, t, pos, tag, smem, ws);
      } else {
        ok = mv_dispatch(a, ph, t, pos, tag, smem, ws);
      }
      __syncthreads();  // LDS is reused by the next task
    }
    if (a.trace && threadIdx.x == 0)
      __hip_atomic_store(&a.trace[(size_t)p * nwg + blockIdx.x], (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }

  // the last workgroup to finish selects the token and advances the step
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_flag = old == (uint32_t)(nwg - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_flag) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const int err = __hip_atomic_load(&st->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!err) {
    if (a.logits) {
      select_token(a.sel, (uint8_t*)smem);
    } else if (threadIdx.x == 0) {
      st->pos = pos + 1;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    *a.epoch = tag + 1;
    __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// (group, fp16 K/V) pairs compiled into the persistent step
#define CHONK_STEP_CASES(X) X(1, true) X(2, true) X(3, true) X(4, true) X(1, false) X(2, false) X(3, false) X(4, false)

const void* step_fn(int group, bool kv_f16) {
#define CHONK_STEP_FN(GG, KK) \
  if (group == GG && kv_f16 == KK) return (const void*)k_step<GG, KK>;
  CHONK_STEP_CASES(CHONK_STEP_FN)
#undef CHONK_STEP_FN
  return nullptr;
}

}  // namespace

size_t step_shared_bytes(int max_k, int max_tile_rows, int group, int hd, int chunk, int nchunk, int kv_elem) {
  (void)max_tile_rows;
  const size_t mv = sizeof(float) * (4 * (size_t)max_k + (size_t)max_k / 16 + 8 + kStepResFloats + 1024);
  const size_t at = attn_shared_bytes(group, hd, chunk, nchunk, kv_elem);
  return std::max(std::max(mv, at), (size_t)kSelectWorkspaceBytes);
}

bool step_supported(int group, bool kv_f16) { return step_fn(group, kv_f16) != nullptr; }

int step_occupancy(int group, bool kv_f16, size_t shmem) {
  const void* f = step_fn(group, kv_f16);
  if (!f) return 0;
  if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shmem) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, kWg, shmem) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

hipError_t launch_step(const StepArgs* a, const StepPhase* phases, int group, bool kv_f16, int grid, size_t shmem, hipStream_t s) {
#define CHONK_STEP_LAUNCH(GG, KK)                                                     \
  if (group == GG && kv_f16 == KK) {                                                  \
    hipLaunchKernelGGL((k_step<GG, KK>), dim3(grid), dim3(kWg), shmem, s, a, phases); \
    return hipGetLastError();                                                         \
  }
  CHONK_STEP_CASES(CHONK_STEP_LAUNCH)
#undef CHONK_STEP_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace chonk
