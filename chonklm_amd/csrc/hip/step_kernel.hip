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

// Copies src[0, n) into dst (LDS) once every word carries `tag`. All threads
// of the workgroup call it. Returns false when the step is aborted (this wait
// exceeded its bound, or another workgroup's did).
__device__ __forceinline__ bool poll_in(const tagged_t* src, int n, float* dst, uint32_t tag, DevState* st, StepDebug* dbg,
                        const WaitSite& site, int pos) {
  const uint64_t t0 = wall_clock64();
  for (uint32_t it = 0;; ++it) {
    int stale = 0;
    for (int i = threadIdx.x; i < n; i += kWg) {
      const uint64_t w = __hip_atomic_load(gbl(src + i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      stale |= (uint32_t)(w >> 32) != tag;
      dst[i] = __uint_as_float((uint32_t)w);
    }
    if (!__syncthreads_or(stale)) return true;
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
            for (int i = 0; i < n && idx < 0; ++i) {
              const uint64_t w = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              if ((uint32_t)(w >> 32) != tag) {
                idx = i;
                seen = (uint32_t)(w >> 32);
              }
            }
            __hip_atomic_store(&dbg->wg, (int32_t)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->phase, site.phase, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->task, site.task, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->index, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->seen, seen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->want, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->pos, pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&dbg->abort_time, (uint64_t)wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          __hip_atomic_store(&st->error, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return false;
      }
    }
  }
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
template <int T>
__device__ __forceinline__ bool mv_task(const StepArgs& a, const StepPhase& ph, const TaskSeg& ts, bool glu, int gtask,
                                        int pos, uint32_t tag, const StepMvLds& l, const WaitSite& ws) {
  constexpr int kPf = sizeof(Frag<T>) > 40 ? 2 : 4;
  const SegView& g = ts.g;
  const int tid = threadIdx.x;
  const int K = ph.k;
  const int U = g.w.k >> 5;
  const int lpr = g.lpr;
  const int shift = __builtin_ctz((unsigned)lpr);
  const int ng = kWg >> shift;
  const int lg = tid >> shift, li = tid & (lpr - 1);
  const int t0 = ts.task * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  const int nv = nt > 0 ? (glu ? 2 * nt : nt) : 0;
  const int rows_lane = lg < nv ? (nv - lg + ng - 1) / ng : 0;
  const int ucount = (U + lpr - 1) / lpr;
  const int items = rows_lane * ucount;

  auto load_item = [&](int ii, Frag<T>& f) {
    const int r = ii / ucount, j = ii - r * ucount;
    const int v = lg + r * ng, u = li + j * lpr;
    if (ii < items && u < U) {
      QMat m = g.w;
      if (glu && (v & 1)) {
        m.s0 = g.u0;
        m.s1 = g.u1;
        m.s2 = g.u2;
        m.s3 = g.u3;
      }
      f = load_unit<T>(m, t0 + (glu ? (v >> 1) : v), u);
    }
  };

  // 1. inputs that do not depend on the previous phase
  if (ph.pro != PRO_PLAIN) lds_dma(ph.w_norm, l.wn, K);
  if (ph.pro == PRO_RES_NORM) lds_dma(ph.w_delta, l.wd, K);
  Frag<T> cur[kPf];
#pragma unroll
  for (int q = 0; q < kPf; ++q) load_item(q, cur[q]);

  // 2. inputs of the previous phases
  if (ph.pro != PRO_EMBED_NORM && !poll_in(ph.in, K, l.xs, tag, a.st, a.dbg, ws, pos)) return false;
  if (ph.pro == PRO_RES_NORM && !poll_in(ph.delta, K, l.dl, tag, a.st, a.dbg, ws, pos)) return false;
  if (ph.epi == EPI_ADD && nt > 0 && !poll_in(ph.add + t0, nt, l.addv, tag, a.st, a.dbg, ws, pos)) return false;
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
  for (int j = tid; j < K / 16; j += kWg) {
    const float4* p = (const float4*)(xs + 16 * j);
    const float4 a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3];
    l.xs16[j] = ((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w)) +
                ((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w));
  }
  __syncthreads();

  // 4. dot products (mv_work)
  {
    const float* xs16 = l.xs16;
    float acc = 0.f;
    for (int base = 0; base < items; base += kPf) {
      Frag<T> nxt[kPf];
#pragma unroll
      for (int q = 0; q < kPf; ++q) load_item(base + kPf + q, nxt[q]);
#pragma unroll
      for (int q = 0; q < kPf; ++q) {
        const int ii = base + q;
        if (ii < items) {
          const int r = ii / ucount, j = ii - r * ucount;
          const int u = li + j * lpr;
          if (u < U) acc += dot_unit<T>(cur[q], u, xs, xs16);
          if (j == ucount - 1) {
            acc = group_sum_n(acc, lpr);
            if (li == 0) l.res[lg + r * ng] = acc;
            acc = 0.f;
          }
        }
      }
#pragma unroll
      for (int q = 0; q < kPf; ++q) cur[q] = nxt[q];
    }
  }
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
  with_type(ts.g.w.type, [&]<int T>() { ok = mv_task<T>(a, ph, ts, glu, t, pos, tag, l, ws); });
  return ok;
}

// One attention task: (kv head, chunk) = (t / nchunk, t % nchunk).
template <int G, bool KV16>
__device__ __forceinline__ bool attn_task(const StepArgs& a, const StepPhase& ph, int t, int pos, uint32_t tag, float* sm,
                          uint32_t* s_last, const WaitSite& ws) {
  const AttnArgs& at = ph.at;
  const int kv = t / at.nchunk, c = t - kv * at.nchunk;
  const int hd = at.hd, CH = at.chunk;
  const int start = (at.window != 0 && pos + 1 > at.window) ? pos + 1 - at.window : 0;
  if (c < start / CH || c > pos / CH) return true;  // chunk outside [start, pos]
  const int tid = threadIdx.x;
  const int tpp = at.tpp;
  const int my_p = tid / tpp, my_j = tid & (tpp - 1);
  const int dpt = hd / tpp;
  const int t_lo = c * CH;
  constexpr int kElem = KV16 ? 2 : 4;
  constexpr int kVec = KV16 ? 8 : 16;
  const int nvec = dpt * kElem / 16;
  const int ncp = (at.nchunk + 3) & ~3;
  float* q_s = sm;
  float* k_new = q_s + G * hd;
  float* v_new = k_new + hd;
  float* qn = v_new + hd;
  float* kn = qn + hd;
  float* inv = kn + hd;
  float* wpart = inv + hd;
  float* wml = wpart + 4 * G * hd;
  float* wts = wml + 8 * kMaxG;
  float* tile = wts + G * ncp;
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

  // this step's q (group heads), k and v of the head
  const int qdim = at.heads * hd, kvdim = at.kv_heads * hd;
  if (!poll_in(ph.qkv_in + (size_t)kv * G * hd, G * hd, q_s, tag, a.st, a.dbg, ws, pos)) return false;
  if (!poll_in(ph.qkv_in + qdim + (size_t)kv * hd, hd, k_new, tag, a.st, a.dbg, ws, pos)) return false;
  if (!poll_in(ph.qkv_in + qdim + kvdim + (size_t)kv * hd, hd, v_new, tag, a.st, a.dbg, ws, pos)) return false;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  tagged_t* out = ph.attn_out + (size_t)kv * G * hd;
  attn_compute<G, KV16>(at, sm, kv, c, pos, kreg, s_last, [&](int i, float v) { tag_store(out + i, v, tag); });
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
        ok = attn_task<G, KV16>(a, ph, t, pos, tag, smem, &s_flag, ws);
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
