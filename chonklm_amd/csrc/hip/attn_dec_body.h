// Decode attention over the fp16 K/V cache for one new token: the body of
// k_attn_dec (attn_decode.hip, which describes its phases) and of the fused
// q|k|v + attention launch (kernels.hip), where the group's q, k and v rows
// arrive as tagged words from the q|k|v workgroups of the same launch instead
// of being read from the q|k|v vector.
#pragma once

#include <hip/hip_runtime.h>

#include "kernel_common.h"
#include "kernels.h"

namespace chonk {
namespace {

constexpr int kDecChunk = 64;  // positions per workgroup
constexpr int kDecWave = 16;   // positions per wave
constexpr int kDecSubMax = 16; // sub-chunks per workgroup (128 workgroups per kv head merge)

__device__ __forceinline__ float2 ldg2f(const float2* p) {
  const uint2 v = ldg2(p);
  return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
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
// qn[G][HD] (normalised, rotated q, shared by the waves) | wmx[4][G] (each
// wave's score maximum) | ew[G][64] (the chunk's weights; position p at
// (p % PG) * NP + p / PG, so a lane reads its V positions contiguously) |
// hv[G][4] (the new position's score per head) | cs[HD] (the rotary (cos, sin)
// pairs of the position).
//
// Chunk rows (a.tpart, [kv][nchunk][rowf] tagged words): per head [max, sum,
// acc[HD]], each word {f32, u32 tag}; the tag of a launch is the kv head's
// epoch a.cnt[kv], which the newest chunk advances when it is done.
// WALK: the workgroup walks a.sub sub-chunks (long contexts); otherwise its
// chunk is one sub-chunk and the code is that of a single chunk.
template <int G, int HD, bool WALK, bool FUSED>
__device__ __forceinline__ void attn_dec_body(const AttnArgs& a, int kv, int c) {
  extern __shared__ __align__(16) float sm[];
  constexpr int HALF = HD / 2;
  constexpr int DPT = HD / 4;            // K dims per lane (four lanes per position)
  constexpr int NKV = DPT / 8;           // 16-byte K vectors per lane
  constexpr int NPR = (HALF + 63) / 64;  // rotary pairs per lane
  // V: wave w owns dims [w * HD / 4, (w + 1) * HD / 4) of all 64 positions;
  // a lane holds VD consecutive dims (VW dwords) of NP positions
  constexpr int VD = HD >= 256 ? 4 : 2;
  constexpr int VW = VD / 2;
  constexpr int DW = HD / 4 / VD;        // lanes per position row: 8 or 16
  constexpr int LDW = DW == 8 ? 3 : 4;
  constexpr int PG = 64 / DW;            // position groups
  constexpr int NP = kDecChunk / PG;     // positions per lane
  static_assert(DW == 8 || DW == 16, "head size");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* q_s = sm;
  float* kx = q_s + G * HD;
  float* vx = kx + HD;
  float* nq = vx + HD;
  float* nk = nq + HD;
  float* qn = nk + HD;
  float* wmx = qn + G * HD;
  float* ew = wmx + 4 * G;
  float* hv = ew + kDecChunk * G;
  float* cs_s = hv + 4 * G;  // (cos, sin) of the rotary pairs at the position
  uint64_t tr[8];
  CHONK_MV_T(tr, 0);

  // A: the position, stop flag and epoch by scalar loads (their own counter,
  // so nothing below waits on them early), then the vector loads: the rotary
  // frequencies, the K/V rows, the LDS copies — with the rotary cos/sin
  // computed while they are in flight
  DevState* st = a.st;
  const int pos = ld_scalar(&st->pos);
  const int stopped = ld_scalar(&st->stopped);
  const uint32_t tag = ld_scalar(&a.cnt[kv]);
  const int span = WALK ? kDecChunk * a.sub : kDecChunk;  // positions of this workgroup's chunk
  const int t_lo = c * span;
  const int kp = kDecWave * wave + (lane >> 2);  // this lane's K position in the chunk
  const int kd0 = (lane & 3) * DPT;
  const int pg = lane >> LDW;                    // this lane's V positions: pg + PG * j
  const int vd = wave * (HD / 4) + VD * (lane & (DW - 1));
  const __half* kc = (const __half*)a.kc + (size_t)kv * a.ctx * HD;
  const __half* vc = (const __half*)a.vc + (size_t)kv * a.ctx * HD;
  uint4 kr[NKV];
  uint32_t vr[NP][VW];
  // K / V rows of the 64 positions from t0
  auto load_k = [&](int t0) {
    const int tk = min(t0 + kp, a.ctx - 1);
#pragma unroll
    for (int v = 0; v < NKV; ++v) kr[v] = ldg4(kc + (size_t)tk * HD + kd0 + 8 * v);
  };
  auto load_v = [&](int t0) {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const __half* p = vc + (size_t)min(t0 + pg + PG * j, a.ctx - 1) * HD + vd;
      if constexpr (VW == 1) {
        vr[j][0] = ldg1(p);
      } else {
        const uint2 w = ldg2(p);
        vr[j][0] = w.x;
        vr[j][VW - 1] = w.y;
      }
    }
  };
  auto load_kv = [&](int t0) {
    load_k(t0);
    load_v(t0);
  };
  // (the q/k/v copies and the rotary table first: the K/V loads are the last
  // NKV + NP of the wave, so phase B only waits for what was issued before
  // them and runs while they are in flight)
  if constexpr (!FUSED) {
    lds_dma(a.qkv + (size_t)kv * G * HD, q_s, G * HD);
    lds_dma(a.qkv + (size_t)a.heads * HD + (size_t)kv * HD, kx, HD);
    lds_dma(a.qkv + (size_t)(a.heads + a.kv_heads) * HD + (size_t)kv * HD, vx, HD);
  }
  if (a.qn_w) {
    lds_dma(a.qn_w, nq, HD);
    lds_dma(a.kn_w, nk, HD);
  }
  // the rotary (cos, sin) row of the position, through LDS as well (a value
  // loaded into registers before the K/V loads would be awaited with them)
  lds_dma((const float*)(a.rope_cs + (size_t)min(pos, a.ctx - 1) * HALF), cs_s, HD);
  __builtin_amdgcn_sched_barrier(0);  // (kept in this order)
  if constexpr (FUSED) {
    // (the q|k|v rows come no sooner than the matvec's own loads land: the
    // K/V requests wait a.kv_delay ticks of 10 ns so as not to queue ahead of them)
    if (a.kv_delay > 0) {
      const uint64_t d0 = wall_clock64();
      while (wall_clock64() - d0 < (uint64_t)a.kv_delay) __builtin_amdgcn_s_sleep(2);
    }
  }
  if (a.spec_kv) load_kv(t_lo);
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int c_lo = start / span, c_hi = pos / span;
  const bool active = !stopped && pos < a.ctx && c >= c_lo && c <= c_hi;
  if (active && !a.spec_kv) load_kv(t_lo);
  // everything but the K/V loads has landed (an inactive workgroup, which may
  // not have issued them, leaves below without reading LDS)
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(NKV + NP));
  lds_barrier();
  CHONK_MV_T(tr, 1);
  if (stopped) return;
  if (pos >= a.ctx) {
    if (tid == 0) st->error = 1;
    return;
  }
  if (!active) return;
  if constexpr (FUSED) {
    // the group's q rows, k row and v row come from the q|k|v workgroups of
    // the same launch as words tagged with this kv head's epoch: poll them
    // (the first pass is awaited together with the K/V rows, issued before)
    // and copy them to q_s | kx | vx, which are contiguous
    constexpr int NW = (G + 2) * HD;
    constexpr int PER = (NW + kWg - 1) / kWg;
    const tagged_t* src[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int w = min(tid + kWg * i, NW - 1);
      src[i] = a.qkv_tag + (w < G * HD       ? (size_t)kv * G * HD + w
                            : w < (G + 1) * HD ? (size_t)a.heads * HD + (size_t)kv * HD + (w - G * HD)
                                               : (size_t)(a.heads + a.kv_heads) * HD + (size_t)kv * HD +
                                                     (w - (G + 1) * HD));
    }
    uint64_t wv[PER];
    const uint64_t t0 = wall_clock64();
    for (uint32_t it = 0;; ++it) {
      bool stale = false;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        wv[i] = tag_get(src[i]);
        stale |= !tag_is(wv[i], tag);
      }
      if (__builtin_amdgcn_ballot_w64(stale) == 0) break;
      if ((it & 3) == 3 && __builtin_amdgcn_readfirstlane(wall_clock64() - t0 > kDecPollTicks ? 1 : 0)) {
        if (lane == 0) st->error = 5;  // (5: the q|k|v rows did not arrive in time)
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (tid + kWg * i < NW) q_s[tid + kWg * i] = tag_val(wv[i]);
    lds_barrier();
  }

  // B: the group's q heads, the new k and the new v are G + 2 items spread
  // over the waves: RMSNorm (if any) and rotary of q into qn; of k, rounded to
  // fp16 like the cache, into kx; v rounded into vx. The newest chunk also
  // stores k and v to the cache.
  int ia[NPR], ib[NPR];
  float co[NPR], si[NPR];
#pragma unroll
  for (int j = 0; j < NPR; ++j) {
    const int d = min(lane + 64 * j, HALF - 1);
    ia[j] = a.interleaved ? 2 * d : d;
    ib[j] = a.interleaved ? 2 * d + 1 : d + HALF;
    co[j] = cs_s[2 * d];
    si[j] = cs_s[2 * d + 1];
  }
  const size_t kv_row = ((size_t)kv * a.ctx + pos) * HD;
  for (int it = wave; it < G + 2; it += 4) {
    if (it <= G) {
      const float* src = it < G ? q_s + it * HD : kx;
      const float* nw = it < G ? nq : nk;
      float x0[NPR], x1[NPR];
#pragma unroll
      for (int j = 0; j < NPR; ++j) {
        x0[j] = src[ia[j]];
        x1[j] = src[ib[j]];
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
          x0[j] = __fmul_rn(__fmul_rn(x0[j], r), nw[ia[j]]);
          x1[j] = __fmul_rn(__fmul_rn(x1[j], r), nw[ib[j]]);
        }
      }
      float y0[NPR], y1[NPR];
#pragma unroll
      for (int j = 0; j < NPR; ++j) {
        y0[j] = __fsub_rn(__fmul_rn(x0[j], co[j]), __fmul_rn(x1[j], si[j]));
        y1[j] = __fadd_rn(__fmul_rn(x0[j], si[j]), __fmul_rn(x1[j], co[j]));
      }
      if (it < G) {
#pragma unroll
        for (int j = 0; j < NPR; ++j)
          if (lane + 64 * j < HALF) {
            qn[it * HD + ia[j]] = y0[j];
            qn[it * HD + ib[j]] = y1[j];
          }
      } else {
        // (every lane read its kx elements above; a lane writes only its own)
#pragma unroll
        for (int j = 0; j < NPR; ++j)
          if (lane + 64 * j < HALF) {
            const __half h0 = __float2half_rn(y0[j]), h1 = __float2half_rn(y1[j]);
            if (c == c_hi) {
              *gblw((unsigned short*)a.kc + kv_row + ia[j]) = __half_as_ushort(h0);
              *gblw((unsigned short*)a.kc + kv_row + ib[j]) = __half_as_ushort(h1);
            }
            kx[ia[j]] = __half2float(h0);
            kx[ib[j]] = __half2float(h1);
          }
      }
    } else {
#pragma unroll
      for (int d = lane; d < HD; d += 64) {
        const __half vh = __float2half_rn(vx[d]);
        if (c == c_hi) *gblw((unsigned short*)a.vc + kv_row + d) = __half_as_ushort(vh);
        vx[d] = __half2float(vh);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the chunk's K/V rows
  __syncthreads();

  // C: over the workgroup's sub-chunks of 64 positions that hold cached
  // positions of [start, pos) (the new position is not in the registers: the
  // merge adds it): scores, the sub-chunk maximum per head, the weights
  // exp(s - max) into ew, weighted V; the softmax runs online over the
  // sub-chunks (running maximum and sum, accumulators rescaled when the
  // maximum grows). The next sub-chunk's K rows are requested once the scores
  // are formed, its V rows once the weighted sum is done.
  const int s_first = max(0, (start - t_lo) / kDecChunk);
  // (-1 when no cached position of [start, pos) lies in this chunk)
  const int s_last = pos > t_lo && start < pos ? min(WALK ? a.sub - 1 : 0, (pos - 1 - t_lo) / kDecChunk) : -1;
  const int ei = (kp % PG) * NP + kp / PG;
  float mx[G], lsum[G], o[G][VD];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mx[g] = -INFINITY;
    lsum[g] = 0.f;  // wave g % 4's running sum of head g
#pragma unroll
    for (int k = 0; k < VD; ++k) o[g][k] = 0.f;
  }
  if (WALK && s_first > 0 && s_first <= s_last) load_kv(t_lo + kDecChunk * s_first);  // (a window start)
  for (int sc = s_first; sc <= s_last; ++sc) {
    const int t0 = t_lo + kDecChunk * sc;
    const int tk = t0 + kp;
    const bool kvalid = tk >= start && tk < pos;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.f;
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const uint32_t w[4] = {kr[v].x, kr[v].y, kr[v].z, kr[v].w};
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 q0 = *(const float4*)(qn + g * HD + kd0 + 8 * v);
        const float4 q1 = *(const float4*)(qn + g * HD + kd0 + 8 * v + 4);
        s[g] = fmaf(q0.x, h2f(w[0]), s[g]);
        s[g] = fmaf(q0.y, h2f(w[0] >> 16), s[g]);
        s[g] = fmaf(q0.z, h2f(w[1]), s[g]);
        s[g] = fmaf(q0.w, h2f(w[1] >> 16), s[g]);
        s[g] = fmaf(q1.x, h2f(w[2]), s[g]);
        s[g] = fmaf(q1.y, h2f(w[2] >> 16), s[g]);
        s[g] = fmaf(q1.z, h2f(w[3]), s[g]);
        s[g] = fmaf(q1.w, h2f(w[3] >> 16), s[g]);
      }
    }
    if (WALK && sc < s_last) load_k(t0 + kDecChunk);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sc4 = group_sum<4>(s[g]);  // (all lanes take part in the DPP steps)
      s[g] = kvalid ? sc4 * a.scale : -INFINITY;
      const float mw = wave_max(s[g]);
      if (lane == 0) wmx[wave * G + g] = mw;
    }
    __syncthreads();  // the maxima (and the previous sub-chunk's weights are consumed)
    float alpha[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      // finite: the sub-chunk holds a cached position
      const float mp = fmaxf(fmaxf(wmx[g], wmx[G + g]), fmaxf(wmx[2 * G + g], wmx[3 * G + g]));
      const float mn = WALK ? fmaxf(mx[g], mp) : mp;
      if constexpr (WALK) alpha[g] = exp_fast(mx[g] - mn);  // 0 on the first sub-chunk
      mx[g] = mn;
      const float e = kvalid ? exp_fast(s[g] - mn) : 0.f;
      if ((lane & 3) == 0) ew[g * kDecChunk + ei] = e;
    }
    __syncthreads();
    // rows outside [start, pos) carry weight 0, and their registers are
    // cleared so that no unwritten value reaches the sum
    if (t0 < start || t0 + kDecChunk > pos) {
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        const int p = t0 + pg + PG * j;
        if (p < start || p >= pos)
#pragma unroll
          for (int t = 0; t < VW; ++t) vr[j][t] = 0u;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if constexpr (WALK) {
        if (g % 4 == wave) lsum[g] = lsum[g] * alpha[g] + wave_sum(ew[g * kDecChunk + lane]);
#pragma unroll
        for (int k = 0; k < VD; ++k) o[g][k] *= alpha[g];
      } else {
        if (g % 4 == wave) lsum[g] = wave_sum(ew[g * kDecChunk + lane]);
      }
    }
#pragma unroll
    for (int j4 = 0; j4 < NP / 4; ++j4) {
      float4 w4[G];
#pragma unroll
      for (int g = 0; g < G; ++g) w4[g] = *(const float4*)(ew + g * kDecChunk + pg * NP + 4 * j4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 4 * j4 + i;
        float vf[VD];
#pragma unroll
        for (int t = 0; t < VW; ++t) {
          vf[2 * t] = h2f(vr[j][t]);
          vf[2 * t + 1] = h2f(vr[j][t] >> 16);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float wt = i == 0 ? w4[g].x : i == 1 ? w4[g].y : i == 2 ? w4[g].z : w4[g].w;
#pragma unroll
          for (int k = 0; k < VD; ++k) o[g][k] = fmaf(wt, vf[k], o[g][k]);
        }
      }
    }
    if (WALK && sc < s_last) load_v(t0 + kDecChunk);
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int k = 0; k < VD; ++k) o[g][k] = pg_sum<DW>(o[g][k]);
  CHONK_MV_T(tr, 2);

  // D: the chunk's row [max, sum, acc[HD]] per head, as tagged words (no
  // wait): in each store instruction lane (pg, dw) writes item pg + PG * it
  // (head item / VD, dim vd + item % VD), so the lanes of one head cover
  // consecutive words and every cache line is written whole
  const int rowf = attn_rowf(G, HD);
  tagged_t* row = a.tpart + (size_t)(kv * a.nchunk + c) * rowf;
#pragma unroll
  for (int it = 0; it < (G * VD + PG - 1) / PG; ++it) {
    const int item = it * PG + pg;
    float val = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < VD; ++k)
        if (g * VD + k == item) val = o[g][k];
    if (item < G * VD) tag_put(row + (item / VD) * (HD + 2) + 2 + vd + item % VD, val, tag);
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
    if (g % 4 == wave) {
      if (lane == 0) {
        tag_put(row + g * (HD + 2), mx[g], tag);  // -inf when no cached position
        tag_put(row + g * (HD + 2) + 1, lsum[g], tag);
      }
    }
  CHONK_MV_T(tr, 3);
  // the new position's score per head, while the rows travel
#pragma unroll
  for (int g = 0; g < G; ++g)
    if (g % 4 == wave) {
      float sn = 0.f;
#pragma unroll
      for (int d = lane; d < HD; d += 64) sn += qn[g * HD + d] * kx[d];
      sn = wave_sum(sn) * a.scale;
      if (lane == 0) hv[4 * g] = sn;
    }
  CHONK_MV_T(tr, 4);

  // merge, shared by the active chunks: chunk c merges dims [s*SD, s*SD+SD)
  // of every head of the group, s = c_hi - c. The newest chunk's slice is
  // never empty, so it has seen every chunk's row carry this launch's tag —
  // every chunk has read the epoch — before it advances the epoch. Each
  // output element (g, d) of the slice has a group of tpi lanes (tpi >=
  // nact / 2, so a lane covers at most two chunks) in one wave; each lane polls its chunks' (max, sum, acc[d]) words until
  // all carry this launch's tag (one pass costs one memory round trip; the
  // wave repeats while any lane still sees an old tag), then the group forms
  // M, the weights exp(m_c - M), the sum L and the weighted acc in registers,
  // the new position joining as one more term.
  const int nact = c_hi - c_lo + 1;
  const int SD = (HD + nact - 1) / nact;
  const int d_lo = min((c_hi - c) * SD, HD), nd = min(SD, HD - d_lo);
  const tagged_t* rows0 = a.tpart + (size_t)(kv * a.nchunk + c_lo) * rowf;
  int ltpi = 0;
  while (ltpi < 6 && (2 << ltpi) < nact) ++ltpi;
  const int tpi = 1 << ltpi;
  const int n_el = G * nd;
  __syncthreads();  // the new-position scores and the rounded v
  const uint64_t t0 = wall_clock64();
  bool late = false;
  for (int base = 0; base < n_el * tpi && !late; base += kWg) {
    const int q = base + tid;
    const int i = q >> ltpi, sub = q & (tpi - 1);
    const bool el = i < n_el;
    const int g = el ? i / nd : 0, d = d_lo + (el ? i - g * nd : 0);
    const bool h0 = el && sub < nact, h1 = el && sub + tpi < nact;
    const tagged_t* r0 = rows0 + (size_t)min(sub, nact - 1) * rowf + g * (HD + 2);
    const tagged_t* r1 = rows0 + (size_t)min(sub + tpi, nact - 1) * rowf + g * (HD + 2);
    uint64_t w[6];
    for (uint32_t it = 0;; ++it) {
      w[0] = tag_get(r0);
      w[1] = tag_get(r0 + 1);
      w[2] = tag_get(r0 + 2 + d);
      w[3] = tag_get(r1);
      w[4] = tag_get(r1 + 1);
      w[5] = tag_get(r1 + 2 + d);
      bool stale = h0 && !(tag_is(w[0], tag) && tag_is(w[1], tag) && tag_is(w[2], tag));
      stale |= h1 && !(tag_is(w[3], tag) && tag_is(w[4], tag) && tag_is(w[5], tag));
      if (__builtin_amdgcn_ballot_w64(stale) == 0) break;
      if ((it & 3) == 3 && __builtin_amdgcn_readfirstlane(wall_clock64() - t0 > kDecPollTicks ? 1 : 0)) {
        late = true;
        break;
      }
    }
    if (late) break;
    const float m0 = h0 ? tag_val(w[0]) : -INFINITY, m1 = h1 ? tag_val(w[3]) : -INFINITY;
    const float sn = hv[4 * g];
    const float M = fmaxf(group_max_n(fmaxf(m0, m1), tpi), sn);
    const float f0 = m0 == -INFINITY ? 0.f : exp_fast(m0 - M);
    const float f1 = m1 == -INFINITY ? 0.f : exp_fast(m1 - M);
    const float l = (h0 ? tag_val(w[1]) * f0 : 0.f) + (h1 ? tag_val(w[4]) * f1 : 0.f);
    const float s = (h0 ? tag_val(w[2]) * f0 : 0.f) + (h1 ? tag_val(w[5]) * f1 : 0.f);
    const float L = group_sum_n(l, tpi), S = group_sum_n(s, tpi);
    const float fn = exp_fast(sn - M);
    if (el && sub == 0) a.out[(size_t)kv * G * HD + g * HD + d] = __fdiv_rn(S + fn * vx[d], L + fn);
  }
  if (late && tid == 0) st->error = 4;
  CHONK_MV_T(tr, 5);
  CHONK_MV_T(tr, 6);
  CHONK_MV_TRACE_END(tr, 7 * 65536);
  // every producer of this launch has read the tag once all rows carry it:
  // the newest chunk advances the epoch for the next launch
  if (c != c_hi) return;
  if (tid == 0) __hip_atomic_store(gblw(&a.cnt[kv]), tag + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace chonk
