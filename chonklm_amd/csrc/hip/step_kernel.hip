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
//
// Each workgroup walks a list of task records built on the host (StepTask:
// rows, slot layout, the slot's direct-to-LDS copies, input and output
// addresses), kept a few records ahead in LDS, so a task starts from one
// record instead of chains of dependent reads of the phase table. One wave
// per SIMD runs the whole step (the kernel needs all 512 registers of a
// lane), so every dependent instruction's latency is exposed: the code
// between hand-offs is kept short and free of per-type copies except the
// dot products.
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

// Records the first wait that exceeded its time bound and aborts the step
// (DevState.error = 3). `locate` maps an element of the concatenated segments
// to its source word.
template <class Locate>
__device__ __forceinline__ void poll_abort(Locate locate, int total, uint32_t tag, DevState* st, StepDebug* dbg,
                                        const WaitSite& site, int pos) {
  uint32_t expect = 0;
  if (__hip_atomic_compare_exchange_strong(gblw(&dbg->claimed), &expect, 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)) {
    int idx = -1;
    uint32_t seen = 0;
    for (int e = 0; e < total && idx < 0; ++e) {
      const uint64_t v = __hip_atomic_load(gbl(locate(e)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)(v >> 32) != tag) {
        idx = e;
        seen = (uint32_t)(v >> 32);
      }
    }
    __hip_atomic_store(gblw(&dbg->wg), (int32_t)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->phase), site.phase, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->task), site.task, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->index), idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->seen), seen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->want), tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->pos), pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gblw(&dbg->abort_time), (uint64_t)wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __hip_atomic_store(gblw(&st->error), 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Copies every segment's src[0, n) into its dst (LDS) once every word carries
// `tag`. All threads of the workgroup call it; it ends with one barrier.
// Returns false when the step is aborted (this wait exceeded its bound, or
// another workgroup's did). Each wave polls its own quarter of the words on
// its own (no barrier per poll): a pass issues the lane's B loads before it
// waits, so it costs one memory round trip, and a wave moves on as soon as
// its words are current. Every lane issues every load (past the end it reads
// the last word again), which keeps the code branch-free and the compiler's
// wait counts exact.
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int per = (total + 3) / 4;  // this wave's words: [w0, w1)
  const int w0 = min(total, wave * per), w1 = min(total, w0 + per);
  const uint64_t t0 = wall_clock64();
  bool aborted = false;
  for (int base = w0; base < w1 && !aborted; base += B * 64) {
    for (uint32_t it = 0;; ++it) {
      uint64_t w[B];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        const tagged_t* src;
        float* dst;
        locate(min(base + lane + j * 64, w1 - 1), src, dst);
        w[j] = __hip_atomic_load(gbl(src), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      int stale = 0;
#pragma unroll
      for (int j = 0; j < B; ++j) stale |= (uint32_t)(w[j] >> 32) != tag;
      if (__builtin_amdgcn_ballot_w64(stale) == 0) {
#pragma unroll
        for (int j = 0; j < B; ++j) {
          const tagged_t* src;
          float* dst;
          locate(min(base + lane + j * 64, w1 - 1), src, dst);
          *dst = __uint_as_float((uint32_t)w[j]);
        }
        break;
      }
      if ((it & 3) == 3) {
        const bool timeout = wall_clock64() - t0 > kPollTicks;
        const bool err = __hip_atomic_load(gbl(&st->error), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
        if (timeout || err) {
          if (timeout && lane == 0)
            poll_abort([&](int e) {
              const tagged_t* src;
              float* dst;
              locate(e, src, dst);
              return src;
            }, total, tag, st, dbg, site, pos);
          aborted = true;
          break;
        }
      }
    }
  }
  return !__syncthreads_or(aborted ? 1 : 0);
}

// ---- prefetch slots ------------------------------------------------------------
//
// A task's inputs that do not depend on earlier phases (norm weights, its rows
// of every weight stream, its K/V chunk) are copied into one of two LDS slots
// by direct-to-LDS loads that the workgroup issues during its previous task,
// right after that task's last read of its own slot. The copy then overlaps
// the previous task's epilogue and the hand-off wait, and the task's compute
// reads LDS instead of waiting on memory after its input arrives. (A load
// into a slot makes the compiler wait for every outstanding load before the
// next read of either slot, hence the issue point after the last read.)
__shared__ __align__(16) uint8_t s_slots[2][kStepSlotBytes];

typedef const __attribute__((address_space(3))) uint8_t* lds_cptr;
typedef uint32_t u32x4l_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2l_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 lds16(const uint8_t* p) {
  const u32x4l_t v = *(const __attribute__((address_space(3))) u32x4l_t*)(lds_cptr)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 lds8(const uint8_t* p) {
  const u32x2l_t v = *(const __attribute__((address_space(3))) u32x2l_t*)(lds_cptr)p;
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t lds4(const uint8_t* p) {
  return *(const __attribute__((address_space(3))) uint32_t*)(lds_cptr)p;
}
__device__ __forceinline__ uint32_t lds2(const uint8_t* p) {
  return *(const __attribute__((address_space(3))) unsigned short*)(lds_cptr)p;
}

// Workgroup barrier that waits for this wave's LDS operations only, not for
// its outstanding global loads and stores or direct-to-LDS loads (a
// __syncthreads() waits for all of them, which would put the next task's slot
// copy on the critical path). The memory clobber keeps the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Direct-to-LDS copy of n16 16-byte units (each wave a 1 KiB stripe per instruction).
__device__ __forceinline__ void dma16(const uint8_t* src, uint8_t* dst, int n16) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int base = wave * 64; base < n16; base += 256) {
    const int c = base + lane;
    if (c < n16)
      __builtin_amdgcn_global_load_lds((gmem_void*)(src + 16 * (size_t)c), (lds_void*)(dst + 16 * (size_t)base), 16, 0, 0);
  }
}

// The unit's fragment from a slot copy of rows [t0, t0 + nt): sp[s] is row
// t0 of stream s in the slot, `row` is relative to t0. Same element placement
// as load_unit.
template <int T>
__device__ __forceinline__ Frag<T> slot_unit(const uint8_t* const (&sp)[4], int row, int u, int K);

template <>
__device__ __forceinline__ Frag<QT_Q4_K> slot_unit<QT_Q4_K>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  Frag<QT_Q4_K> f;
  f.qs = lds16(sp[0] + row * (K / 2) + 16 * u);
  f.hdr = lds16(sp[1] + row * (K / 16) + 16 * (u >> 3));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_K> slot_unit<QT_Q5_K>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  Frag<QT_Q5_K> f;
  f.qs = lds16(sp[0] + row * (K / 2) + 16 * u);
  f.hdr = lds16(sp[1] + row * (K / 16) + 16 * (u >> 3));
  f.qh = lds16(sp[2] + row * (K / 8) + 32 * (u >> 3) + 16 * (u & 1));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q6_K> slot_unit<QT_Q6_K>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  const int sb = u >> 3, c = u & 7, h = c >> 2, b = c & 3;
  Frag<QT_Q6_K> f;
  const uint8_t* ql = sp[0] + row * (K / 2) + 128 * sb + 64 * h + 8 * b;
  f.qa = lds8(ql);
  f.qb = lds8(ql + 32);
  f.qh = lds8(sp[1] + row * (K / 4) + 64 * sb + 32 * h + 8 * b);
  f.sc = lds8(sp[2] + row * (K / 16) + 16 * sb + 8 * h);
  f.d = lds2(sp[3] + 2 * (row * (K / 256) + sb));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q8_0> slot_unit<QT_Q8_0>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  Frag<QT_Q8_0> f;
  const uint8_t* q = sp[0] + row * K + 32 * u;
  f.q0 = lds16(q);
  f.q1 = lds16(q + 16);
  f.d = lds2(sp[1] + 2 * (row * (K / 32) + u));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_0> slot_unit<QT_Q5_0>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  Frag<QT_Q5_0> f;
  f.qs = lds16(sp[0] + row * (K / 2) + 16 * u);
  f.qh = lds4(sp[1] + 4 * (row * (K / 32) + u));
  f.d = lds2(sp[2] + 2 * (row * (K / 32) + u));
  return f;
}
template <>
__device__ __forceinline__ Frag<QT_Q5_1> slot_unit<QT_Q5_1>(const uint8_t* const (&sp)[4], int row, int u, int K) {
  Frag<QT_Q5_1> f;
  f.qs = lds16(sp[0] + row * (K / 2) + 16 * u);
  f.qh = lds4(sp[1] + 4 * (row * (K / 32) + u));
  f.d = lds2(sp[2] + 2 * (row * (K / 32) + u));
  f.m = lds2(sp[3] + 2 * (row * (K / 32) + u));
  return f;
}

// Dot products of the lane's rows against the digit planes, fragments read
// from the slot; same row / unit walk and accumulation order as mv_stream.
template <int T, int UC>
__device__ __forceinline__ void mv_stream_slot(const uint8_t* slot, const int (&data)[2][4], const MvLane& m,
                                               const XqView& x, float* res, int K) {
  const int nj = m.rows > 0 ? (m.ucount + UC - 1) / UC : 0;
  XU xr[UC];
  for (int jb = 0; jb < nj; ++jb) {
#pragma unroll
    for (int j = 0; j < UC; ++j) {
      const int u = m.li + (jb * UC + j) * m.lpr;
      if (u < m.U) load_xu<T>(x, u, xr[j]);
    }
    for (int r = 0; r < m.rows; ++r) {  // uniform in the lane group
      const int v = m.lg + r * m.ng;
      const bool up = m.glu && (v & 1);
      const int row = m.glu ? (v >> 1) : v;
      const uint8_t* sp[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) sp[q] = slot + (up ? data[1][q] : data[0][q]);
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < UC; ++j) {
        const int u = m.li + (jb * UC + j) * m.lpr;
        if (u < m.U) acc += dot_q<T>(slot_unit<T>(sp, row, u, K), u, xr[j]);
      }
      acc = group_sum_n(acc, m.lpr);
      if (m.li == 0) {
        float* d = res + m.lg + r * m.ng;
        *d = jb == 0 ? acc : *d + acc;
      }
    }
  }
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

// Uniform values read from a task record in LDS, as scalars.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <class P>
__device__ __forceinline__ P* unip(P* v) {
  const uint64_t u = (uint64_t)v;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (P*)(((uint64_t)hi << 32) | lo);
}

// Each workgroup keeps the records of its next tasks in LDS: record i + 7 is
// copied (direct-to-LDS) during task i, into the entry of task i - 1.
__shared__ __align__(16) StepTask s_desc[kStepDescRing];

// Fills `slot` with an attention task's inputs that do not depend on earlier
// phases: the rotary table, q/k norm weights and the K/V rows of its chunk
// that precede this step's position.
__device__ __forceinline__ void attn_fill(const StepPhase& ph, int t, int pos, uint8_t* slot) {
  const AttnArgs& at = ph.at;
  const int kv = t / at.nchunk, c = t - kv * at.nchunk;
  const int hd = at.hd, CH = at.chunk;
  const int start = (at.window != 0 && pos + 1 > at.window) ? pos + 1 - at.window : 0;
  if (c < start / CH || c > pos / CH) return;
  const int elem = at.kv_f16 ? 2 : 4;
  AttnSlot L;
  attn_slot_layout(hd, CH, elem, &L);
  dma16((const uint8_t*)at.rope_inv, slot + L.inv, (hd / 2 * 4 + 15) / 16);
  if (at.qn_w) {
    dma16((const uint8_t*)at.qn_w, slot + L.qn, hd / 4);
    dma16((const uint8_t*)at.kn_w, slot + L.kn, hd / 4);
  }
  const int t_lo = c * CH;
  const int p_begin = max(start - t_lo, 0), p_end = min(pos + 1 - t_lo, CH);
  if (p_end > p_begin) {
    const size_t off = ((size_t)kv * at.ctx * hd + (size_t)(t_lo + p_begin) * hd) * elem;
    const int n16 = (p_end - p_begin) * hd * elem / 16;
    dma16((const uint8_t*)at.kc + off, slot + L.k + p_begin * hd * elem, n16);
    dma16((const uint8_t*)at.vc + off, slot + L.v + p_begin * hd * elem, n16);
  }
}

// Fills `slot` for the task of record `nd`: a matvec task's norm weights and
// rows of every weight stream (the copies listed in its record), an attention
// task's chunk; an lm_head task streams its rows from memory.
__device__ __forceinline__ void fill_task(const StepArgs& a, const StepTask& nd, int pos, uint8_t* slot) {
  const int ph = uni(nd.phase);
  if (ph >= a.n_phases) return;
  const int kind = uni(nd.kind);
  if (kind == STASK_MV) {
    const int n = uni(nd.n_dma);
    for (int j = 0; j < n; ++j) dma16(unip(nd.dma[j].src), slot + uni(nd.dma[j].dst), uni(nd.dma[j].n16));
  } else if (kind == STASK_ATTN) {
    attn_fill(a.phases[ph], uni(nd.t), pos, slot);
  }
}

// Profiling stamps of the current task (thread 0 writes them; see NextFill::mark).
__shared__ uint64_t s_stamp[kStepStamps];

// What a task requests once it has read its own slot for the last time: the
// next task's slot and a task record kStepDescRing - 1 tasks ahead.
struct NextFill {
  const StepArgs* a;
  const StepTask* nd;     // next task's record (LDS)
  int pos;
  uint8_t* slot;
  const StepTask* rec;    // record to prefetch (device memory) and its LDS entry
  StepTask* rec_dst;
  uint64_t* stamp;        // profiling: this task's kStepStamps wall-clock stamps (null: off)
  __device__ __forceinline__ void fill() const {
    fill_task(*a, *nd, pos, slot);
    dma16((const uint8_t*)rec, (uint8_t*)rec_dst, (int)(sizeof(StepTask) / 16));
  }
  // stamps go to LDS and are copied out once the task has ended, so that no
  // barrier inside the task waits for the store of a stamp
  __device__ __forceinline__ void mark(int k) const {
    if (stamp && threadIdx.x == 0) s_stamp[k] = wall_clock64();
  }
};

// The matvec fields of a task record, as scalars.
struct MvTask {
  int phase, t, type, uc, k, lpr, t0, nt, glu, pro, epi, res_lo, res_hi, wn, wd;
  int data[2][4];
  const tagged_t *in, *delta, *add;
  tagged_t *out, *res_out;
};

__device__ __forceinline__ MvTask load_mv_task(const StepTask& d) {
  MvTask m;
  m.phase = uni(d.phase);
  m.t = uni(d.t);
  m.type = uni(d.type);
  m.uc = uni(d.uc);
  m.k = uni(d.k);
  m.lpr = uni(d.lpr);
  m.t0 = uni(d.t0);
  m.nt = uni(d.nt);
  m.glu = uni(d.glu);
  m.pro = uni(d.pro);
  m.epi = uni(d.epi);
  m.res_lo = uni(d.res_lo);
  m.res_hi = uni(d.res_hi);
  m.wn = uni(d.wn);
  m.wd = uni(d.wd);
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) m.data[j][q] = uni(d.data[j][q]);
  m.in = unip(d.in);
  m.delta = unip(d.delta);
  m.add = unip(d.add);
  m.out = unip(d.out);
  m.res_out = unip(d.res_out);
  return m;
}

__device__ __forceinline__ MvLane mv_lane_k(int K, int lpr, int nt, bool glu) {
  MvLane m;
  m.U = K >> 5;
  m.lpr = lpr;
  const int shift = __builtin_ctz((unsigned)lpr);
  m.ng = kWg >> shift;
  m.lg = threadIdx.x >> shift;
  m.li = threadIdx.x & (lpr - 1);
  const int nv = nt > 0 ? (glu ? 2 * nt : nt) : 0;
  m.rows = m.lg < nv ? (nv - m.lg + m.ng - 1) / m.ng : 0;
  m.ucount = (m.U + lpr - 1) / lpr;
  m.t0 = 0;
  m.glu = glu;
  return m;
}

// The residual add and RMSNorm prologues (mv_finish of the per-phase
// kernels) and the quantization of the normalised input, over xs in LDS.
__device__ __forceinline__ void mv_prologue(const StepArgs& a, const MvTask& d, const StepMvLds& l, const float* wn,
                                            const float* wd, uint32_t tag) {
  const int tid = threadIdx.x;
  const int K = d.k;
  float* xs = l.xs;
  if (d.pro == PRO_RES_NORM) {
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += l.dl[i] * l.dl[i];
    ss = block_sum(ss, l.red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) {
      const float nd = __fmul_rn(__fmul_rn(l.dl[i], inv), wd[i]);
      xs[i] = fminf(fmaxf(__fadd_rn(xs[i], nd), -65000.0f), 65000.0f);
    }
    __syncthreads();
  }
  if (d.pro != PRO_PLAIN) {
    // this task's slice of the residual, for the later phases that add to it
    for (int i = d.res_lo + tid; i < d.res_hi; i += kWg) tag_store(d.res_out + i, xs[i], tag);
    float ss = 0.f;
    for (int i = tid; i < K; i += kWg) ss += xs[i] * xs[i];
    ss = block_sum(ss, l.red);
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    for (int i = tid; i < K; i += kWg) xs[i] = __fmul_rn(__fmul_rn(xs[i], inv), wn[i]);
    __syncthreads();
  }
}

// Stores a matvec task's rows (EPI_STORE / EPI_ADD / EPI_GLU_*) as tagged words.
__device__ __forceinline__ void mv_epilogue(const MvTask& d, const StepMvLds& l, uint32_t tag) {
  const int tid = threadIdx.x;
  const float* res = l.res;
  switch (d.epi) {
    case EPI_STORE:
      for (int t = tid; t < d.nt; t += kWg) tag_store(d.out + t, res[t], tag);
      break;
    case EPI_ADD:
      for (int t = tid; t < d.nt; t += kWg) tag_store(d.out + t, __fadd_rn(l.addv[t], res[t]), tag);
      break;
    case EPI_GLU_SILU:
      for (int t = tid; t < d.nt; t += kWg) tag_store(d.out + t, silu_mul(res[2 * t], res[2 * t + 1]), tag);
      break;
    default:  // EPI_GLU_GELU
      for (int t = tid; t < d.nt; t += kWg) tag_store(d.out + t, __fmul_rn(gelu_tanh(res[2 * t]), res[2 * t + 1]), tag);
      break;
  }
}

// Embedding row of the token at `pos` times the embedding scale, into xs (the
// layer-0 prologue; ggufEmbedding, llama-wgsl-runtime.ts:1326-1342).
__device__ __forceinline__ void embed_into(const StepArgs& a, int pos, int K, float* xs) {
  const int tid = threadIdx.x;
  int tok = *gbl(a.hist + pos);
  if (tok < 0 || tok >= a.vocab) {
    if (tid == 0) *gblw(&a.st->error) = 2;
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

// One matvec task whose norm weights and weight rows are in `slot`: the
// input is polled, the prologue and dot products read LDS only, and the next
// task's slot is requested before the epilogue. Only the dot products depend
// on the weight type, so the rest of the task is one body of code for every
// phase.
__device__ __forceinline__ bool mv_slot_task(const StepArgs& a, const MvTask& d, int pos, uint32_t tag, float* smem,
                                             const WaitSite& ws, const uint8_t* slot, const NextFill& nf) {
  const int K = d.k;
  const StepMvLds l = step_mv_lds(smem, K, kStepResFloats);
  if (d.pro == PRO_EMBED_NORM) embed_into(a, pos, K, l.xs);  // made visible by the poll's barrier
  {
    const PollSeg sg[3] = {{d.in, l.xs, d.pro != PRO_EMBED_NORM ? K : 0},
                           {d.delta, l.dl, d.pro == PRO_RES_NORM ? K : 0},
                           {d.add, l.addv, d.epi == EPI_ADD ? max(d.nt, 0) : 0}};
    if (!poll_segs<3, 8>(sg, tag, a.st, a.dbg, ws, pos)) return false;
  }
  nf.mark(1);
  mv_prologue(a, d, l, (const float*)(slot + max(d.wn, 0)), (const float*)(slot + max(d.wd, 0)), tag);
  nf.mark(2);
  quantize_x(l.xs, K, l.dl, l.xs16);  // dl is free from here on
  __syncthreads();
  nf.mark(3);
  const MvLane m = mv_lane_k(K, d.lpr, d.nt, d.glu != 0);
  const XqView x = xq_view(l.dl, l.xs16, K);
  with_type(d.type, [&]<int T>() {
    if (d.uc == 1)
      mv_stream_slot<T, 1>(slot, d.data, m, x, l.res, K);
    else
      mv_stream_slot<T, 2>(slot, d.data, m, x, l.res, K);
  });
  __syncthreads();
  nf.mark(4);
  nf.fill();  // the slot is read for the last time above
  nf.mark(5);
  mv_epilogue(d, l, tag);
  nf.mark(6);
  return true;
}

// The phase's segment holding task t (lm_head phases have one segment).
__device__ __forceinline__ SegView lm_seg(const StepPhase& ph) {
  SegView g;
  g.w = ph.seg[0].w;
  g.u0 = g.u1 = g.u2 = g.u3 = nullptr;
  g.out = nullptr;
  g.add = nullptr;
  g.bias = nullptr;
  g.n_out = ph.seg[0].n_out;
  g.tile = ph.seg[0].tile;
  g.lpr = ph.seg[0].lpr;
  g.wg_begin = 0;
  return g;
}

// One lm_head task: 256 rows streamed from memory (the first fragments are
// requested before the poll), then the group argmax of its rows with the
// first-stage repetition penalty.
template <int T, int UC>
__device__ __forceinline__ bool lm_task_t(const StepArgs& a, const StepPhase& ph, const SegView& g, int task, int pos,
                                          uint32_t tag, const StepMvLds& l, const WaitSite& ws, const NextFill& nf) {
  const int tid = threadIdx.x;
  const int K = ph.k;
  const int t0 = task * g.tile;
  const int nt = min(g.tile, g.n_out - t0);
  const MvLane m = mv_lane(g, t0, nt, false);
  Frag<T> cur[MvShape<T, UC>::N];
  if (ph.pro != PRO_PLAIN) lds_dma(ph.w_norm, l.wn, K);
  if (ph.pro == PRO_RES_NORM) lds_dma(ph.w_delta, l.wd, K);
  mv_fetch<T, UC>(g, m, 0, cur);
  {
    const PollSeg sg[2] = {{ph.in, l.xs, K}, {ph.delta, l.dl, ph.pro == PRO_RES_NORM ? K : 0}};
    if (!poll_segs<2, 8>(sg, tag, a.st, a.dbg, ws, pos)) return false;
  }
  nf.mark(1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  MvTask d{};
  d.k = K;
  d.pro = ph.pro;
  d.res_out = ph.res_out;
  if (ph.pro == PRO_RES_NORM) {
    const int S = (K + ph.n_tasks - 1) / ph.n_tasks;
    d.res_lo = min(K, task * S);
    d.res_hi = min(K, d.res_lo + S);
  }
  mv_prologue(a, d, l, l.wn, l.wd, tag);
  nf.mark(2);
  quantize_x(l.xs, K, l.dl, l.xs16);
  __syncthreads();
  nf.mark(3);
  mv_stream<T, UC, 2>(g, m, xq_view(l.dl, l.xs16, K), l.res, cur);
  __syncthreads();
  nf.mark(4);
  nf.fill();
  nf.mark(5);
  // group argmax over the task's 256 rows (ARGMAX_STAGE1)
  const float* res = l.res;
  float* vals = l.res + 256;
  uint32_t* idx = (uint32_t*)(vals + 256);
  float v = kNegBig;
  uint32_t id = 0xffffffffu;
  const int row = t0 + tid;
  if (tid < nt && row < a.vocab) {
    v = res[tid];
    *gblw(ph.logits + row) = v;
    if (*gbl(&a.samp->stage1_penalty) && bit_test(a.pen_bits, (uint32_t)row)) {
      const float p = *gbl(&a.samp->stage1_pen);
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
    __hip_atomic_store(gblw((uint64_t*)&a.cand[task]), ((uint64_t)idx[0] << 32) | (uint64_t)__float_as_uint(vals[0]),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  nf.mark(6);
  return true;
}

__device__ __forceinline__ bool lm_task(const StepArgs& a, const StepPhase& ph, int t, int pos, uint32_t tag, float* smem,
                                        const WaitSite& ws, const NextFill& nf) {
  const SegView g = lm_seg(ph);
  const StepMvLds l = step_mv_lds(smem, ph.k, kStepResFloats);
  bool ok = true;
  const int uc = mv_uc(g);
  with_type(g.w.type, [&]<int T>() {
    ok = uc == 1 ? lm_task_t<T, 1>(a, ph, g, t, pos, tag, l, ws, nf) : lm_task_t<T, 2>(a, ph, g, t, pos, tag, l, ws, nf);
  });
  return ok;
}

// One attention task: (kv head, chunk) = (t / nchunk, t % nchunk). The
// chunk's K/V rows, the rotary table and the q/k norm weights are in `slot`
// (filled during the previous task). Every chunk but the newest stores its
// partial (tagged); the newest chunk's task merges the head's partials as they
// arrive and stores the head's output.
template <int G, bool KV16>
__device__ __forceinline__ bool attn_task(const StepArgs& a, const StepPhase& ph, int t, int pos, uint32_t tag, float* sm,
                                          const WaitSite& ws, uint8_t* slot, const NextFill& nf) {
  const AttnArgs& at = ph.at;
  const int kv = t / at.nchunk, c = t - kv * at.nchunk;
  const int hd = at.hd, CH = at.chunk;
  const int start = (at.window != 0 && pos + 1 > at.window) ? pos + 1 - at.window : 0;
  const int c_lo = start / CH, c_hi = pos / CH;
  if (c < c_lo || c > c_hi) {  // chunk outside [start, pos]
    nf.fill();
    return true;
  }
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
  (void)qn;
  const int p_begin = max(start - t_lo, 0);
  const int p_end = min(pos + 1 - t_lo, CH);
  AttnSlot L;
  attn_slot_layout(hd, CH, kElem, &L);

  // this step's q (group heads), k and v of the head, in one polling pass
  const int qdim = at.heads * hd, kvdim = at.kv_heads * hd;
  {
    const PollSeg sg[3] = {{ph.qkv_in + (size_t)kv * G * hd, q_s, G * hd},
                           {ph.qkv_in + qdim + (size_t)kv * hd, k_new, hd},
                           {ph.qkv_in + qdim + kvdim + (size_t)kv * hd, v_new, hd}};
    if (!poll_segs<3, 2>(sg, tag, a.st, a.dbg, ws, pos)) return false;
  }
  nf.mark(1);

  // K rows of the chunk (positions before this step) from the slot into registers
  uint4 kreg[kVec];
#pragma unroll
  for (int v = 0; v < kVec; ++v) kreg[v] = make_uint4(0u, 0u, 0u, 0u);
  if (my_p < CH && my_p >= p_begin && my_p < p_end) {
    const uint8_t* src = slot + L.k + ((size_t)my_p * hd + my_j * dpt) * kElem;
#pragma unroll
    for (int v = 0; v < kVec; ++v)
      if (v < nvec) kreg[v] = lds16(src + 16 * v);
  }
  nf.mark(2);

  attn_chunk<G, KV16>(at, sm, kv, c, pos, kreg, (const float*)(slot + L.inv),
                      at.qn_w ? (const float*)(slot + L.qn) : nullptr, at.qn_w ? (const float*)(slot + L.kn) : nullptr,
                      slot + L.v);
  // the slot is read for the last time above (attn_chunk ends with a
  // barrier); the merging chunk requests the next slot after its merge, whose
  // polls would otherwise wait for the copy
  nf.mark(3);
  if (c != c_hi) {
    nf.fill();
    nf.mark(4);
  }

  // partial rows [kv][nchunk], rowf words each (padding words carry the tag too)
  tagged_t* rows = ph.tpart + (size_t)kv * at.nchunk * rowf;
  if (c != c_hi) {
    for (int i = tid; i < rowf; i += kWg) tag_store(rows + (size_t)c * rowf + i, i < G * (hd + 2) ? cpart[i] : 0.0f, tag);
    nf.mark(5);
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
  nf.mark(5);
  nf.fill();
  nf.mark(6);
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
  if (*gbl(&st->stopped)) return;
  const int pos = *gbl(&st->pos);
  const uint32_t tag = *gbl(a.epoch);
  const int nwg = (int)gridDim.x;
  if (threadIdx.x == 0 && blockIdx.x < 1024)
    __hip_atomic_store(gblw(&a.dbg->start[blockIdx.x]), (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  if (a.trace && threadIdx.x == 0)
    __hip_atomic_store(gblw(&a.trace[(size_t)a.n_phases * nwg + blockIdx.x]), (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  bool ok = pos < a.sel.ctx;
  if (!ok && threadIdx.x == 0) *gblw(&st->error) = 1;
  // this workgroup's tasks in order (task t of a phase runs on workgroup
  // t mod grid), as records resolved on the host; each task's slot is filled
  // during the task before it
  const StepTask* my = a.tasks + (size_t)blockIdx.x * a.task_stride;
  for (int j = 0; j < kStepDescRing - 1; ++j)
    dma16((const uint8_t*)(my + j), (uint8_t*)&s_desc[j], (int)(sizeof(StepTask) / 16));
  __syncthreads();  // waits for the copies
  if (ok) fill_task(a, s_desc[0], pos, s_slots[0]);
  int stamped = 0;
  for (int i = 0; ok; ++i) {
    const StepTask& d = s_desc[i % kStepDescRing];
    const int p = uni(d.phase);
    if (p >= a.n_phases) break;
    const int t = uni(d.t);
    const int kind = uni(d.kind);
    const StepTask& nd = s_desc[(i + 1) % kStepDescRing];
    const int np = min(uni(nd.phase), a.n_phases);
    uint64_t* stamp =
        a.trace ? a.trace + (size_t)(a.n_phases + 1) * nwg + ((size_t)p * nwg + blockIdx.x) * kStepStamps : nullptr;
    const NextFill nf{&a, &nd, pos, s_slots[(i + 1) & 1], my + i + kStepDescRing - 1,
                      &s_desc[(i + kStepDescRing - 1) % kStepDescRing], stamp};
    const WaitSite ws{p, t};
    uint8_t* slot = s_slots[i & 1];
    if (stamp && threadIdx.x < kStepStamps) s_stamp[threadIdx.x] = 0;
    nf.mark(0);
    if (kind == STASK_MV) {
      ok = mv_slot_task(a, load_mv_task(d), pos, tag, smem, ws, slot, nf);
    } else if (kind == STASK_ATTN) {
      ok = attn_task<G, KV16>(a, phases[p], t, pos, tag, smem, ws, slot, nf);
    } else {
      ok = lm_task(a, phases[p], t, pos, tag, smem, ws, nf);
    }
    lds_barrier();  // LDS (this slot, this record) is reused by the tasks after
    nf.mark(kStepStamps - 1);
    if (stamp && threadIdx.x < kStepStamps) *gblw(stamp + threadIdx.x) = s_stamp[threadIdx.x];
    if (a.trace && threadIdx.x == 0)
      for (; stamped < np; ++stamped)
        __hip_atomic_store(gblw(&a.trace[(size_t)stamped * nwg + blockIdx.x]), (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  if (a.trace && threadIdx.x == 0)
    for (; stamped < a.n_phases; ++stamped)
      __hip_atomic_store(gblw(&a.trace[(size_t)stamped * nwg + blockIdx.x]), (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);

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
  const int err = __hip_atomic_load(gbl(&st->error), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
#ifndef CHONK_STEP_CASES
#define CHONK_STEP_CASES(X) X(1, true) X(2, true) X(3, true) X(4, true) X(1, false) X(2, false) X(3, false) X(4, false)
#endif

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
