// Batched (many-token) kernels for gfx950: the prompt is processed as T rows
// at once instead of T decode steps (the reference prefills token by token,
// llama-wgsl-runtime.ts:276-289; the K/V it leaves in the cache and the last
// prompt token's logits are what must match).
//
// Linear layers are dequant-fused GEMMs on the matrix cores. fp16 MFMA keeps
// fp32-class accuracy by splitting both operands into hi + lo halves:
//   W * 2^ws = Wh + Wl,  x * 2^rs = xh + xl  (per token row),
//   sum W x = 2^-(ws+rs) * (Wh xh + Wh xl + Wl xh)   (Wl xl ~ 2^-22, dropped)
// with the weights dequantized bit-exactly (dequant_unit) into LDS tiles and
// the products accumulated in fp32 by gfx950's v_mfma_f32_16x16x32_f16.
#include <hip/hip_runtime.h>
#include <cstdlib>
#include <cstring>

#include <algorithm>

#include "kernel_common.h"
#include "kernels.h"
#include "prefill.h"

namespace chonk {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kGM = 64;          // weight rows per workgroup tile
// token rows per workgroup tile: 128 for passes over 512 rows (each
// dequantized weight stage serves more products), 64 up to 512 rows (twice the
// tiles, so that short passes need no K split)
__host__ __device__ constexpr int gemm_tokens(int tj) { return 64 * tj; }
inline int gemm_tj(int rows) { return rows > 512 ? 2 : 1; }
constexpr int kGK = 128;         // K per stage (whole units for every type)
constexpr int kGS = kGK + 8;     // LDS row stride in halves (bank spread)

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
// gfx950's double-K shape: lane l holds row (or column) l % 16 and 8 consecutive
// k of the 32 (the same k for both operands, so the product is the dot over k)
__device__ __forceinline__ float4_t mfma32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

constexpr int kMaxDeferSplit = 16;  // K split of a deferred GEMM (loads of a sum issued together)

// Elements j[e] (valid columns) of row t of a deferred result: the partials
// are read four splits at a time, every load of a round issued before any is
// added (split indices past ks are clamped to the last split and their sums
// not taken, so no load sits behind a branch: a conditional load makes the
// compiler wait for every outstanding load where the paths join); the sums
// add the partials in split order. With ks <= 4 a call costs one memory round
// trip for all N elements.
// part_gather in two halves, so that the first round's loads can be issued
// early and summed where the values are needed: part_issue loads splits 0..3
// (clamped to the last split) of elements j[e]; part_finish adds them in split
// order and reads any further splits four at a time.
template <int N>
__device__ __forceinline__ void part_issue(const PartSum& P, int t, const int (&j)[N], float (&w)[N][4]) {
  const float* q = P.p + (int64_t)t * P.ld;
#pragma unroll
  for (int e = 0; e < N; ++e)
#pragma unroll
    for (int z = 0; z < 4; ++z) w[e][z] = q[(int64_t)min(z, P.ks - 1) * P.zs + j[e]];
}
template <int N>
__device__ __forceinline__ void part_finish(const PartSum& P, int t, const int (&j)[N], float (&w)[N][4],
                                            float (&v)[N]) {
  const float* q = P.p + (int64_t)t * P.ld;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    v[e] = w[e][0];
#pragma unroll
    for (int z = 1; z < 4; ++z) v[e] = z < P.ks ? v[e] + w[e][z] : v[e];
  }
  for (int z0 = 4; z0 < P.ks; z0 += 4) {
#pragma unroll
    for (int e = 0; e < N; ++e)
#pragma unroll
      for (int z = 0; z < 4; ++z) w[e][z] = q[(int64_t)min(z0 + z, P.ks - 1) * P.zs + j[e]];
#pragma unroll
    for (int e = 0; e < N; ++e)
#pragma unroll
      for (int z = 0; z < 4; ++z) v[e] = z0 + z < P.ks ? v[e] + w[e][z] : v[e];
  }
}

// Elements j[e] (valid columns) of row t of a deferred result: the partials
// are read four splits at a time, every load of a round issued before any is
// added (split indices past ks are clamped to the last split and their sums
// not taken, so no load sits behind a branch: a conditional load makes the
// compiler wait for every outstanding load where the paths join); the sums
// add the partials in split order. With ks <= 4 a call costs one memory round
// trip for all N elements.
template <int N>
__device__ __forceinline__ void part_gather(const PartSum& P, int t, const int (&j)[N], float (&v)[N]) {
  if (P.ks == 1) {
    const float* q = P.p + (int64_t)t * P.ld;
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = q[j[e]];
    return;
  }
  float w[N][4];
  part_issue<N>(P, t, j, w);
  part_finish<N>(P, t, j, w, v);
}

// Row t of a deferred result, elements j0 + S * e for e < 4 (zero past n).
template <int S = kWg>
__device__ __forceinline__ void part_row4(const PartSum& P, int t, int j0, float (&v)[4]) {
  int j[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) j[e] = min(j0 + S * e, P.n - 1);
  part_gather<4>(P, t, j, v);
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = j0 + S * e < P.n ? v[e] : 0.f;
}

// The per-row glue kernels run one workgroup of kRowT threads per token row
// (a batch of decode rows is a few dozen workgroups; wide ones keep each
// row's deferred partial sums to one or two rounds of loads).
constexpr int kRowT = 1024;
constexpr int kRowW = kRowT / 64;

__device__ __forceinline__ float rowt_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float a = 0.f;
#pragma unroll
  for (int w = 0; w < kRowW; w += 4) a += (red[w] + red[w + 1]) + (red[w + 2] + red[w + 3]);
  return a;
}
__device__ __forceinline__ float rowt_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float a = 0.f;
#pragma unroll
  for (int w = 0; w < kRowW; ++w) a = fmaxf(a, red[w]);
  return a;
}

// ---- operand split ----------------------------------------------------------------

// One workgroup per token row: optional RMSNorm (x * inv) * w with the
// reference's fp32 operation order, then the row scaled by a power of two so
// that |x| < 2^14 and split into fp16 hi + lo planes (zero-padded to kpad).
// mode 0: plain; 1: RMSNorm with w.
__global__ __launch_bounds__(kRowT) void k_pf_split(PfSplitArgs a) {
  warm_kernarg<(int)(sizeof(PfSplitArgs))>();  // (dependent argument rounds hit the scalar cache)
  // the row lives in registers: element tid + kRowT * e of this thread is v[e]
  // (rows of at most 4 * kRowT elements; the launcher checks)
  __shared__ float red[kRowW];
  const int t = blockIdx.x, tid = threadIdx.x;
  float* xw = const_cast<float*>(a.x + (size_t)t * a.ldx);
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = xw[min(tid + kRowT * e, a.k - 1)];  // unconditional (no branch)
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = tid + kRowT * e < a.k ? v[e] : 0.f;
  if (a.add.p) {
    float d[4];
    part_row4<kRowT>(a.add, t, tid, d);
    if (a.add_w) {
      // the branch output goes through RMSNorm first (the Gemma-3 sandwich)
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += d[e] * d[e];
      ss = rowt_sum(ss, red);
      const float inv = 1.0f / sqrtf(ss / (float)a.k + a.eps);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = tid + kRowT * e;
        if (i < a.k) v[e] = fminf(fmaxf(__fadd_rn(v[e], __fmul_rn(__fmul_rn(d[e], inv), a.add_w[i])), -65000.0f), 65000.0f);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(v[e], d[e]);
    }
    // the updated residual row
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = tid + kRowT * e;
      if (i < a.k) xw[i] = v[e];
    }
  }
  if (a.w) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += v[e] * v[e];
    ss = rowt_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)a.k + a.eps);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = tid + kRowT * e;
      if (i < a.k) v[e] = __fmul_rn(__fmul_rn(v[e], inv), a.w[i]);
    }
  }
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(v[e]));
  mx = rowt_max(mx, red);
  int ex = 0;
  (void)frexpf(mx, &ex);  // mx < 2^ex
  const int rs = max(min(14 - ex, 60), -60);
  _Float16* xh = a.xh + (size_t)t * a.kpad;
  _Float16* xl = a.xl + (size_t)t * a.kpad;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = tid + kRowT * e;
    if (i < a.kpad) {
      const float sv = ldexpf(v[e], rs);  // zero past k
      const _Float16 h = (_Float16)sv;
      xh[i] = h;
      xl[i] = (_Float16)(sv - (float)h);
    }
  }
  if (tid == 0) a.xscale[t] = __builtin_isfinite(mx) ? ldexpf(1.0f, -rs) : __int_as_float(0x7fc00000);
}

// ---- dequant-fused GEMM ----------------------------------------------------------

// y[t][n] (=|+=) sum_k x[t][k] W[n][k] for a kGM x 64 TJ tile. The tile's
// weights are dequantized once per stage into LDS (fp16 hi + lo of W * 2^ws)
// and serve 64 TJ token rows; wave w owns token rows 16 TJ w .. 16 TJ (w + 1) - 1
// against all 64 weight rows (4 x TJ MFMA tiles of 16 x 16, three products each) and
// reads its activation operands straight from the planes (each element is
// read by one lane of one wave, so staging them through LDS would only add a
// copy). With only the weights in LDS (35 KB) the registers bound the
// workgroups per CU: at TJ = 2 three for the Q4_K instance, two for Q6_K.
template <int T, int TJ>
__global__ __launch_bounds__(kWg) void k_gemm(GemmArgs a) {
  extern __shared__ __align__(16) _Float16 gsm[];
  _Float16* wh = gsm;
  _Float16* wl = wh + kGM * kGS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * kGM, t0 = blockIdx.y * gemm_tokens(TJ);
  const int N = a.n_all ? a.n_all : a.w.n;
  // the tile's matrix of a fused launch (segments start on tile boundaries)
  const int seg = a.n_all ? (n0 >= a.n2 ? 2 : (n0 >= a.n1 ? 1 : 0)) : 0;
  const int sb = seg == 2 ? a.n2 : (seg == 1 ? a.n1 : 0);
  // picked field by field (a selected struct copy would live in scratch)
  QMat wm = a.w;
#define CHONK_PICK_W(f) wm.f = seg == 2 ? a.w3.f : (seg == 1 ? a.w2.f : a.w.f)
  CHONK_PICK_W(s0);
  CHONK_PICK_W(s1);
  CHONK_PICK_W(s2);
  CHONK_PICK_W(s3);
  CHONK_PICK_W(n);
#undef CHONK_PICK_W
  const int U = a.w.k >> 5;
  const int nst = (a.w.k + kGK - 1) / kGK;
  // this workgroup's stages: part blockIdx.z of ksplit
  const int s_lo = (int)((int64_t)nst * blockIdx.z / a.ksplit);
  const int s_hi = (int)((int64_t)nst * (blockIdx.z + 1) / a.ksplit);
  // staging role: weight unit (row wr, unit j of the stage)
  const int wr = tid >> 2, wj = tid & 3;
  const bool w_ok = n0 + wr < N;
  const float wsc = ldexpf(1.0f, a.ws);
  // operand role: lane l holds row (or token) l % 16 and k 8 (l / 16) .. + 8 of a 32-k step
  const int col = lane & 15, kq = (lane >> 4) * 8;
  // the lane's plane rows as 32-bit byte offsets from the planes' (uniform)
  // bases; a token row past t reads row t - 1: its products are computed and
  // dropped (the launcher checks that a plane fits 32-bit offsets)
  uint32_t xo[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
    xo[j] = 2u * ((uint32_t)min(t0 + 16 * (TJ * wave + j) + col, a.t - 1) * (uint32_t)a.kpad + (uint32_t)kq);
  const char* xhb = (const char*)a.xh;
  const char* xlb = (const char*)a.xl;

  float4_t acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  Frag<T> f{};
  auto fetch_w = [&](int st) {
    const int u = st * 4 + wj;
    if (w_ok && u < U) f = load_unit<T>(wm, n0 - sb + wr, u);
  };
  fetch_w(s_lo);
  for (int s = s_lo; s < s_hi; ++s) {
    // this stage's activation operands (awaited after the weight staging)
    half8_t bh[kGK / 32][TJ], bl[kGK / 32][TJ];
#pragma unroll
    for (int ks = 0; ks < kGK / 32; ++ks)
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const uint32_t o = xo[j] + 2u * (uint32_t)(s * kGK + ks * 32);
        bh[ks][j] = *(const half8_t*)(xhb + o);
        bl[ks][j] = *(const half8_t*)(xlb + o);
      }
    // weights: the unit's 32 values at their K offsets, hi and lo
    const int u = s * 4 + wj;
    float v[32];
    if (w_ok && u < U) {
      dequant_unit<T>(f, u, v, wsc);  // W * 2^ws (the unit's factors scaled: exact)
    } else {
#pragma unroll
      for (int e = 0; e < 32; ++e) v[e] = 0.f;
    }
    // the next stage's unit goes out as soon as this one is decoded (the last
    // stage requests itself again rather than branching on the stage index)
    fetch_w(min(s + 1, s_hi - 1));
    __syncthreads();  // the previous stage's tile is consumed
    _Float16* rh = wh + wr * kGS;
    _Float16* rl = wl + wr * kGS;
#pragma unroll
    for (int e = 0; e < 32; e += 4) {
      const int kk = (u < U ? unit_col<T>(u, e) : 32 * u + e) - s * kGK;
      half4_t h, l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sv = v[e + i];
        h[i] = (_Float16)sv;
        l[i] = (_Float16)(sv - (float)h[i]);
      }
      *(half4_t*)(rh + kk) = h;
      *(half4_t*)(rl + kk) = l;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kGK / 32; ++ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half8_t ah = *(const half8_t*)(wh + (16 * i + col) * kGS + ks * 32 + kq);
        const half8_t al = *(const half8_t*)(wl + (16 * i + col) * kGS + ks * 32 + kq);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc[i][j] = mfma32(ah, bh[ks][j], acc[i][j]);
          acc[i][j] = mfma32(ah, bl[ks][j], acc[i][j]);
          acc[i][j] = mfma32(al, bh[ks][j], acc[i][j]);
        }
      }
    }
  }
  // lane holds rows 4 * (lane / 16) + 0..3 of each row tile, token lane % 16
  const float wun = ldexpf(1.0f, -a.ws);
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    const int tt = t0 + 16 * (TJ * wave + j) + col;
    if (tt >= a.t) continue;
    const float sc = wun * a.xscale[tt];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + 16 * i + 4 * (lane >> 4);
      float* y = a.y + (size_t)tt * a.ldy + n;
      float* pp = a.part + ((size_t)blockIdx.z * a.t + tt) * N + n;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (n + q >= N) break;
        const float v = acc[i][j][q] * sc;
        if (a.ksplit > 1 || a.defer)
          pp[q] = v;
        else
          y[q] = a.epi == GEMM_ADD ? __fadd_rn(y[q], v) : v;
      }
    }
  }
}

// ---- decode-batch GEMM (at most 64 token rows) ------------------------------------
//
// With 64 or fewer token rows the GEMM streams weights: every weight is used
// by at most 64 products, so staging dequantized tiles through LDS (k_gemm)
// costs more than the products. Here each wave owns 64 weight rows x all 64
// token rows over a quarter of the workgroup's K range, with no LDS for the
// operands: the x planes are loaded straight into MFMA A operands (lane l:
// token l % 16 of each 16-token tile, k 8 (l / 16) .. + 8 of the 32-k step)
// and the weights are dequantized in registers into B operands (lane l: row
// l % 16 of each 16-row tile, the same 8 k), as fp16 hi + lo of W 2^ws; three
// MFMAs per step (Ah Bh + Al Bh + Ah Bl). The lane's weight bytes for its 8 k
// are consecutive in the striped rows: Q4_K sub-blocks 2c and 2c+1 share the
// bytes qs[32c + 8g .. + 8] (low / high nibbles), Q6_K's four 32-k quarters of
// a 128-k half share ql and qh bytes the same way, so the loads of a block
// (64 k of Q4_K, 128 k of Q6_K) are used whole. The four waves' sums meet in
// LDS at the end (in wave order) and the workgroup writes its K split's partial.

constexpr int kSkRows = 64;  // weight rows per wave (and per workgroup)
constexpr int kSkRed = kSkRows + 4;  // k_gemm_sk1's LDS row stride of the per-wave tiles (bank spread)

__device__ __forceinline__ half8_t pack8(const float (&w)[8]) {
  half8_t h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (_Float16)w[i];
  return h;
}
// hi = fp16(w), lo = fp16(w - hi)
__device__ __forceinline__ void split8(const float (&w)[8], half8_t& h, half8_t& l) {
  h = pack8(w);
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = w[i] - (float)h[i];
  l = pack8(r);
}
__device__ __forceinline__ float nib(uint32_t w, int i) { return (float)((w >> (4 * i)) & 15u); }

// A block is 64 k: two 32-k steps whose weights the lane reads from one run of
// bytes (Q4_K: sub-blocks 2c and 2c + 1 of qs[32c + 8g .. + 8], low and high
// nibbles; Q6_K: quarters p and p + 2 of a 128-k half, low and high nibbles of
// ql run p, the half's qh bits 2p and 2p + 4).
template <int T>
struct SkBlock;  // the lane's weight bytes of one block for one row
template <>
struct SkBlock<QT_Q4_K> {
  uint2 qs;      // qs[32c + 8g .. + 8]
  uint4 hdr;     // the super-block header (d, dmin, scales)
};
template <>
struct SkBlock<QT_Q6_K> {
  uint2 ql;      // ql[64h + 32p + 8g .. + 8]
  uint2 qh;      // qh[32h + 8g .. + 8]
  uint2 sc;      // the half's 8 scales sc[8h .. + 8]
  uint32_t d;
};
constexpr int kSkBlockK = 64;

// First column of step s2 (0 or 1) of block blk.
template <int T>
__device__ __forceinline__ int sk_col(int blk, int s2) {
  if constexpr (T == QT_Q4_K) return 64 * blk + 32 * s2;
  // Q6_K block blk: super-block blk / 4, half (blk / 2) % 2, run p = blk % 2; quarter p + 2 s2
  return 256 * (blk >> 2) + 128 * ((blk >> 1) & 1) + 32 * ((blk & 1) + 2 * s2);
}

template <int T>
__device__ __forceinline__ SkBlock<T> sk_load(const QMat& w, int row, int blk, int g) {
  const size_t K = (size_t)w.k;
  SkBlock<T> b;
  if constexpr (T == QT_Q4_K) {
    b.qs = ldg2(w.s0 + row * (K / 2) + 32 * blk + 8 * g);
    b.hdr = ldg4(w.s1 + row * (K / 16) + 16 * (blk >> 2));
  } else {
    const int sb = blk >> 2, h = (blk >> 1) & 1, p = blk & 1;
    b.ql = ldg2(w.s0 + row * (K / 2) + 128 * sb + 64 * h + 32 * p + 8 * g);
    b.qh = ldg2(w.s1 + row * (K / 4) + 64 * sb + 32 * h + 8 * g);
    b.sc = ldg2(w.s2 + row * (K / 16) + 16 * sb + 8 * h);
    b.d = ld_u16(w.s3 + 2 * (row * (K / 256) + sb));
  }
  return b;
}

// The lane's 8 weights (times 2^ws) of step s2 of the block.
template <int T>
__device__ __forceinline__ void sk_weights(const SkBlock<T>& b, int blk, int s2, int g, float wsc, float (&w)[8]) {
  if constexpr (T == QT_Q4_K) {
    // sub-block j = 2c + s2 of the super-block: nibble s2 of the lane's bytes
    const int j = ((blk & 3) << 1) + s2;
    uint32_t sc, m;
    scale_min(j, b.hdr.y, b.hdr.z, b.hdr.w, &sc, &m);
    const float dsc = h2f(b.hdr.x) * (float)sc * wsc, dm = h2f(b.hdr.x >> 16) * (float)m * wsc;
    // four codes per word at once: byte i = nibble s2 of the lane's byte i
    const uint32_t c0 = (b.qs.x >> (4 * s2)) & 0x0f0f0f0fu, c1 = (b.qs.y >> (4 * s2)) & 0x0f0f0f0fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = fmaf(dsc, ub(c0, i), -dm);
      w[4 + i] = fmaf(dsc, ub(c1, i), -dm);
    }
  } else {
    // quarter q = p + 2 s2 of the half: nibble s2 of the ql run, qh bits 2q;
    // the lane's 8 k lie in sub-block 2q + (g >> 1) of the half
    const int q = (blk & 1) + 2 * s2;
    const int si = 2 * q + (g >> 1);
    const uint32_t sw = si < 4 ? b.sc.x : b.sc.y;
    const float dsc = h2f(b.d) * (float)(int8_t)((sw >> (8 * (si & 3))) & 0xffu) * wsc, off = -32.0f * dsc;
    // four 6-bit codes per word at once (byte i: low 4 bits from ql, bits 4-5 from qh)
    const uint32_t c0 = ((b.ql.x >> (4 * s2)) & 0x0f0f0f0fu) | (((b.qh.x >> (2 * q)) & 0x03030303u) << 4);
    const uint32_t c1 = ((b.ql.y >> (4 * s2)) & 0x0f0f0f0fu) | (((b.qh.y >> (2 * q)) & 0x03030303u) << 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[i] = fmaf(dsc, ub(c0, i), off);
      w[4 + i] = fmaf(dsc, ub(c1, i), off);
    }
  }
}

template <int T>
__global__ __launch_bounds__(kWg, 2) void k_gemm_sk(GemmArgs a) {
  extern __shared__ __align__(16) float ssm[];
  constexpr int BK = kSkBlockK;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * kSkRows;
  const int N = a.n_all ? a.n_all : a.w.n;
  const int seg = a.n_all ? (n0 >= a.n2 ? 2 : (n0 >= a.n1 ? 1 : 0)) : 0;
  const int sb0 = seg == 2 ? a.n2 : (seg == 1 ? a.n1 : 0);
  QMat wm = a.w;
#define CHONK_PICK_W(f) wm.f = seg == 2 ? a.w3.f : (seg == 1 ? a.w2.f : a.w.f)
  CHONK_PICK_W(s0);
  CHONK_PICK_W(s1);
  CHONK_PICK_W(s2);
  CHONK_PICK_W(s3);
  CHONK_PICK_W(n);
#undef CHONK_PICK_W
  // this workgroup's blocks (split blockIdx.z of ksplit), then this wave's quarter
  const int nblk = a.w.k / BK;
  const int z_lo = (int)((int64_t)nblk * blockIdx.z / a.ksplit), z_hi = (int)((int64_t)nblk * (blockIdx.z + 1) / a.ksplit);
  const int b_lo = z_lo + (z_hi - z_lo) * wave / 4, b_hi = z_lo + (z_hi - z_lo) * (wave + 1) / 4;
  const float wsc = ldexpf(1.0f, a.ws);
  // rows of the lane in the matrix (clamped: a ragged tile loads a valid row, its sums are dropped)
  int rows[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) rows[rt] = min(n0 + 16 * rt + r16, N - 1) - sb0;
  // token rows of the lane's A operands, clamped: rows past a.t load a valid row
  // and their sums are never written
  int xrow[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) xrow[tt] = min(16 * tt + r16, a.t - 1);
  // the epilogue's operand scales, requested up front (read from LDS at the end)
  if (tid < a.t) ssm[4 * 64 * kSkRows + tid] = a.xscale[tid];

  float4_t acc[4][4];  // [token tile][row tile]: lane holds tokens 16 tt + 4 g + i, row 16 rt + r16
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = float4_t{0.f, 0.f, 0.f, 0.f};

  SkBlock<T> cur[4];
  if (b_lo < b_hi) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) cur[rt] = sk_load<T>(wm, rows[rt], b_lo, g);
  }
  for (int blk = b_lo; blk < b_hi; ++blk) {
    // the next block's bytes are requested before this one is reduced (the
    // last block reloads itself, so that the loads stay unconditional)
    SkBlock<T> nxt[4];
    const int bn = min(blk + 1, b_hi - 1);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) nxt[rt] = sk_load<T>(wm, rows[rt], bn, g);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int k0 = sk_col<T>(blk, s2) + 8 * g;  // this lane's 8 k of the step
      half8_t ah[4], al[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const size_t off = (size_t)xrow[tt] * a.kpad + k0;
        ah[tt] = *gbl((const half8_t*)(a.xh + off));
        al[tt] = *gbl((const half8_t*)(a.xl + off));
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float w[8];
        sk_weights<T>(cur[rt], blk, s2, g, wsc, w);
        half8_t bh, bl;
        split8(w, bh, bl);
        // (the four token tiles' chains interleaved: no MFMA waits on the one before it)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bh, acc[tt][rt]);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(al[tt], bh, acc[tt][rt]);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bl, acc[tt][rt]);
      }
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) cur[rt] = nxt[rt];
  }
  // the four waves' sums, added in wave order: [wave][token][row] floats
  float* red = ssm;
  float* xs = ssm + 4 * 64 * kSkRows;  // the token rows' operand scales
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wave * 64 + 16 * tt + 4 * g + i) * kSkRows + 16 * rt + r16] = acc[tt][rt][i];
  __syncthreads();
  // thread (tg, r) writes row n0 + r of tokens tg, tg + 4, ...: one coalesced
  // 256-byte run per token and store instruction
  const int r = tid & 63, tg = tid >> 6, n = n0 + r;
  if (n < N) {
    const float wun = ldexpf(1.0f, -a.ws);
    for (int t = tg; t < a.t; t += 4) {
      const int e = t * kSkRows + r;
      const float v = (((red[e] + red[64 * kSkRows + e]) + red[2 * 64 * kSkRows + e]) + red[3 * 64 * kSkRows + e]) *
                      (wun * xs[t]);
      if (a.ksplit > 1 || a.defer) {
        a.part[((size_t)blockIdx.z * a.t + t) * N + n] = v;
      } else if (a.epi == GEMM_ADD) {
        float* y = a.y + (size_t)t * a.ldy + n;
        *y = __fadd_rn(*y, v);
      } else {
        a.y[(size_t)t * a.ldy + n] = v;
      }
    }
  }
}

// The same with exactly one 64-k block per wave (the K split of the decode
// step's layer GEMMs): every load of the wave — its x operands, copied
// straight into its own 16 KiB of LDS, and its weight bytes — is issued at
// entry and awaited once, so the wave pays one memory round trip before its
// two steps of products. LDS per wave: [plane][step][token][32 halves].
template <int T>
__global__ __launch_bounds__(kWg, 2) void k_gemm_sk1(GemmArgs a) {
  extern __shared__ __align__(16) float ssm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * kSkRows;
  const int N = a.n_all ? a.n_all : a.w.n;
  const int seg = a.n_all ? (n0 >= a.n2 ? 2 : (n0 >= a.n1 ? 1 : 0)) : 0;
  const int sb0 = seg == 2 ? a.n2 : (seg == 1 ? a.n1 : 0);
  QMat wm = a.w;
#define CHONK_PICK_W(f) wm.f = seg == 2 ? a.w3.f : (seg == 1 ? a.w2.f : a.w.f)
  CHONK_PICK_W(s0);
  CHONK_PICK_W(s1);
  CHONK_PICK_W(s2);
  CHONK_PICK_W(s3);
  CHONK_PICK_W(n);
#undef CHONK_PICK_W
  // this wave's block: one per wave, the workgroup's four in a row
  const int blk = (int)blockIdx.z * 4 + wave;
  _Float16* xw = (_Float16*)ssm + (size_t)wave * (2 * 2 * 64 * 32);  // this wave's x operands
  float* xs = ssm + 4 * 64 * kSkRed;                                 // the token rows' operand scales
  // x: 16 copies of 1 KiB (16 tokens x 64 bytes each); lane l moves token
  // 16 i + l / 4, piece l % 4 (token rows past a.t repeat the last row: their
  // sums are never written)
  {
    const int tok = lane >> 2, pc = lane & 3;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = min(16 * i + tok, a.t - 1);
          const _Float16* src = (p ? a.xl : a.xh) + (size_t)t * a.kpad + sk_col<T>(blk, s2) + 8 * pc;
          __builtin_amdgcn_global_load_lds((gmem_void*)src, (lds_void*)(xw + ((p * 2 + s2) * 64 + 16 * i) * 32), 16,
                                           0, 0);
        }
  }
  const float wsc = ldexpf(1.0f, a.ws);
  SkBlock<T> bk[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) bk[rt] = sk_load<T>(wm, min(n0 + 16 * rt + r16, N - 1) - sb0, blk, g);
  if (tid < a.t) xs[tid] = a.xscale[tid];
  __builtin_amdgcn_s_waitcnt(0);  // (the copies into LDS land before they are read)
  __syncthreads();
  float4_t acc[4][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    half8_t ah[4], al[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      ah[tt] = *(const half8_t*)(xw + ((0 * 2 + s2) * 64 + 16 * tt + r16) * 32 + 8 * g);
      al[tt] = *(const half8_t*)(xw + ((1 * 2 + s2) * 64 + 16 * tt + r16) * 32 + 8 * g);
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      float w[8];
      sk_weights<T>(bk[rt], blk, s2, g, wsc, w);
      half8_t bh, bl;
      split8(w, bh, bl);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bh, acc[tt][rt]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(al[tt], bh, acc[tt][rt]);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bl, acc[tt][rt]);
    }
  }
  __syncthreads();  // every wave has read its x operands (the area is reused below)
  // the four waves' tiles [wave][token][row] (rows padded to kSkRed floats, so
  // that neither the writes below nor the 16-byte reads after them collide on
  // LDS banks); then thread (token tid / 4, rows 16 (tid % 4) .. + 15) sums its
  // 16 outputs over the waves with 16-byte reads and stores them with 16-byte
  // stores — one pass instead of 16 dependent rounds of single floats
  float* red = ssm;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wave * 64 + 16 * tt + 4 * g + i) * kSkRed + 16 * rt + r16] = acc[tt][rt][i];
  __syncthreads();
  const int t = tid >> 2, q = tid & 3;
  if (t < a.t) {
    const float sc = ldexpf(1.0f, -a.ws) * xs[t];
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float* e = red + t * kSkRed + 16 * q + 4 * j;
      const float4 w0 = *(const float4*)e, w1 = *(const float4*)(e + 64 * kSkRed);
      const float4 w2 = *(const float4*)(e + 2 * 64 * kSkRed), w3 = *(const float4*)(e + 3 * 64 * kSkRed);
      v[j] = make_float4((((w0.x + w1.x) + w2.x) + w3.x) * sc, (((w0.y + w1.y) + w2.y) + w3.y) * sc,
                         (((w0.z + w1.z) + w2.z) + w3.z) * sc, (((w0.w + w1.w) + w2.w) + w3.w) * sc);
    }
    const int nq = n0 + 16 * q;
    float* dst = a.part + ((size_t)blockIdx.z * a.t + t) * N + nq;
    if (nq + 16 <= N && (N & 3) == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) *(float4*)(dst + 4 * j) = v[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float o[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2)
          if (nq + 4 * j + e2 < N) dst[4 * j + e2] = o[e2];
      }
    }
  }
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
// The same for a matrix with many row groups (the lm_head): a workgroup owns
// 4 x 64 weight rows over the whole K, the four waves sharing each 64-k block
// of x operands, copied into LDS one block ahead (two buffers; each wave
// copies a quarter); every wave writes its own rows' results. Per block:
// weights of the next block and its x copies are issued, then this block's
// copies are awaited (s_waitcnt counts the loads issued since) and the waves
// meet at a barrier before the products.
template <int T>
__global__ __launch_bounds__(kWg, 2) void k_gemm_lm(GemmArgs a) {
  extern __shared__ __align__(16) float ssm[];
  constexpr int W = T == QT_Q4_K ? 8 : 16;  // weight loads per block and wave (4 row tiles)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * (4 * kSkRows) + wave * kSkRows;  // this wave's rows
  const int N = a.w.n, nblk = a.w.k / kSkBlockK;
  _Float16* xb = (_Float16*)ssm;  // [buffer][plane][step][token][32 halves]
  float* xs = (float*)(xb + 2 * (2 * 2 * 64 * 32));
  const float wsc = ldexpf(1.0f, a.ws);
  int rows[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) rows[rt] = min(n0 + 16 * rt + r16, N - 1);
  // x of block b into buffer b & 1: this wave's four of its sixteen 1-KiB copies
  const int tok = lane >> 2, pc = lane & 3;
  auto copy_x = [&](int b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = wave * 4 + j, p = c >> 3, s2 = (c >> 2) & 1, i = c & 3;
      const int t = min(16 * i + tok, a.t - 1);
      const _Float16* src = (p ? a.xl : a.xh) + (size_t)t * a.kpad + sk_col<T>(b, s2) + 8 * pc;
      __builtin_amdgcn_global_load_lds((gmem_void*)src,
                                       (lds_void*)(xb + (((b & 1) * 4 + p * 2 + s2) * 64 + 16 * i) * 32), 16, 0, 0);
    }
  };
  if (tid < a.t) xs[tid] = a.xscale[tid];
  SkBlock<T> cur[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) cur[rt] = sk_load<T>(a.w, rows[rt], 0, g);
  __builtin_amdgcn_sched_barrier(0);
  copy_x(0);
  __builtin_amdgcn_sched_barrier(0);
  float4_t acc[4][4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) acc[tt][rt] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int b = 0; b < nblk; ++b) {
    // the next block's weights, then its x copies (the last block copies
    // itself into the other buffer, which is not read again: the loop body
    // stays branch-free, so every wait counts exactly)
    const int bn = min(b + 1, nblk - 1);
    SkBlock<T> nxt[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) nxt[rt] = sk_load<T>(a.w, rows[rt], bn, g);
    __builtin_amdgcn_sched_barrier(0);
    copy_x(bn);
    __builtin_amdgcn_sched_barrier(0);
    // this block's copies have landed once at most the loads issued after
    // them are outstanding: the next block's W weight loads and 4 copies
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(W + 4));
    // (a bare barrier: __syncthreads would also wait for the loads in flight)
    lds_barrier();
    const _Float16* xc = xb + (size_t)(b & 1) * 4 * 64 * 32;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      half8_t ah[4], al[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        ah[tt] = *(const half8_t*)(xc + ((0 * 2 + s2) * 64 + 16 * tt + r16) * 32 + 8 * g);
        al[tt] = *(const half8_t*)(xc + ((1 * 2 + s2) * 64 + 16 * tt + r16) * 32 + 8 * g);
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        float w[8];
        sk_weights<T>(cur[rt], b, s2, g, wsc, w);
        half8_t bh, bl;
        split8(w, bh, bl);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bh, acc[tt][rt]);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(al[tt], bh, acc[tt][rt]);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) acc[tt][rt] = mfma32(ah[tt], bl, acc[tt][rt]);
      }
    }
    lds_barrier();  // every wave has read buffer b & 1 before block b + 2's copies overwrite it
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) cur[rt] = nxt[rt];
  }
  const float wun = ldexpf(1.0f, -a.ws);
  const bool add = a.epi == GEMM_ADD;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * tt + 4 * g + i;
      if (t >= a.t) continue;
      const float sc = wun * xs[t];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const int n = n0 + 16 * rt + r16;
        if (n >= N) continue;
        float* y = a.y + (size_t)t * a.ldy + n;
        const float v = acc[tt][rt][i] * sc;
        if (add)
          *y = __fadd_rn(*y, v);
        else
          *y = v;
      }
    }
}

size_t gemm_lm_shared_bytes() { return sizeof(_Float16) * 2 * (2 * 2 * 64 * 32) + sizeof(float) * 64; }

size_t gemm_sk_shared_bytes() { return sizeof(float) * (4 * 64 * kSkRed + 64); }

// The decode-batch GEMM applies: at most 64 token rows and a K-quant type it covers.
bool gemm_sk_applies(const GemmArgs& a) {
  static const bool off = [] {
    const char* v = std::getenv("CHONK_GEMM");
    return v && std::strcmp(v, "tiles") == 0;
  }();
  return !off && a.t >= 1 && a.t <= 64 && (a.w.type == QT_Q4_K || a.w.type == QT_Q6_K) && a.w.k % 256 == 0 &&
         a.kpad >= a.w.k;
}

// K split of a decode-batch GEMM: about 256 workgroups (one per CU), at least
// one block per wave.
int gemm_sk_split(const GemmArgs& a, int row_groups) {
  const int nblk = a.w.k / kSkBlockK;
  int ks = std::max(1, std::min(kMaxDeferSplit, (256 + row_groups - 1) / row_groups));
  while (ks > 1 && nblk / ks < 4) --ks;
  return ks;
}

hipError_t launch_gemm_sk(const GemmArgs& a, int n_rows, hipStream_t s) {
  const dim3 grid((n_rows + kSkRows - 1) / kSkRows, 1, a.ksplit);
  const size_t sh = gemm_sk_shared_bytes();
  if (a.w.type == QT_Q4_K)
    hipLaunchKernelGGL(k_gemm_sk<QT_Q4_K>, grid, dim3(kWg), sh, s, a);
  else
    hipLaunchKernelGGL(k_gemm_sk<QT_Q6_K>, grid, dim3(kWg), sh, s, a);
  return hipGetLastError();
}

// y[t][n] (=|+=) the K-split partial sums, added in split order.
__global__ __launch_bounds__(kWg) void k_gemm_reduce(GemmArgs a) {
  const int64_t total = (int64_t)a.t * a.w.n;
  for (int64_t i = (int64_t)blockIdx.x * kWg + threadIdx.x; i < total; i += (int64_t)gridDim.x * kWg) {
    float v = a.part[i];
    for (int z = 1; z < a.ksplit; ++z) v += a.part[(int64_t)z * total + i];
    const int64_t t = i / a.w.n, n = i - t * a.w.n;
    float* y = a.y + t * a.ldy + n;
    *y = a.epi == GEMM_ADD ? __fadd_rn(*y, v) : v;
  }
}

// ---- per-token glue ---------------------------------------------------------------

// Embedding rows of the prompt tokens times the embedding scale.
__global__ __launch_bounds__(kWg) void k_pf_embed(QMat embed, const int32_t* tok, float scale, int k, float* x) {
  const int t = blockIdx.x;
  const int id = tok[t];
  with_type(embed.type, [&]<int TE>() {
    for (int u = threadIdx.x; u < k / 32; u += kWg) {
      const Frag<TE> f = load_unit<TE>(embed, id, u);
      float v[32];
      dequant_unit<TE>(f, u, v);
#pragma unroll
      for (int e = 0; e < 32; ++e) x[(size_t)t * k + unit_col<TE>(u, e)] = __fmul_rn(v[e], scale);
    }
  });
}

// x = clamp(x + RMSNorm(d) * w, +-65000) per token row (the Gemma-3 sandwich
// residual, as the decode prologue PRO_RES_NORM computes it).
__global__ __launch_bounds__(kWg) void k_pf_norm_add(const float* d, const float* w, float eps, int k, float* x) {
  __shared__ float red[8];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float* dr = d + (size_t)t * k;
  float* xr = x + (size_t)t * k;
  float ss = 0.f;
  for (int i = tid; i < k; i += kWg) ss += dr[i] * dr[i];
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)k + eps);
  for (int i = tid; i < k; i += kWg) {
    const float nd = __fmul_rn(__fmul_rn(dr[i], inv), w[i]);
    xr[i] = fminf(fmaxf(__fadd_rn(xr[i], nd), -65000.0f), 65000.0f);
  }
}

// act = silu(g) * u or gelu_tanh(g) * u per element, then the split of the row
// into fp16 planes (one workgroup per token row).
__global__ __launch_bounds__(kRowT) void k_pf_glu_split(PfGluArgs a) {
  warm_kernarg<(int)(sizeof(PfGluArgs))>();  // (dependent argument rounds hit the scalar cache)
  // element tid + kRowT * e of the row is v[e] (at most 4 * kRowT elements)
  __shared__ float red[kRowW];
  const int t = blockIdx.x, tid = threadIdx.x;
  float* y = a.act + (size_t)t * a.k;
  float gv[4], uv[4], v[4];
  part_row4<kRowT>(a.pg, t, tid, gv);
  part_row4<kRowT>(a.pu, t, tid, uv);
  float mx = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = tid + kRowT * e;
    v[e] = 0.f;
    if (i < a.k) {
      v[e] = a.gelu ? __fmul_rn(gelu_tanh(gv[e]), uv[e]) : silu_mul(gv[e], uv[e]);
      y[i] = v[e];
      mx = fmaxf(mx, fabsf(v[e]));
    }
  }
  mx = rowt_max(mx, red);
  int ex = 0;
  (void)frexpf(mx, &ex);
  const int rs = max(min(14 - ex, 60), -60);
  _Float16* xh = a.xh + (size_t)t * a.kpad;
  _Float16* xl = a.xl + (size_t)t * a.kpad;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = tid + kRowT * e;
    if (i < a.kpad) {
      const float sv = ldexpf(v[e], rs);
      const _Float16 h = (_Float16)sv;
      xh[i] = h;
      xl[i] = (_Float16)(sv - (float)h);
    }
  }
  if (tid == 0) a.xscale[t] = __builtin_isfinite(mx) ? ldexpf(1.0f, -rs) : __int_as_float(0x7fc00000);
}

__device__ __forceinline__ int row_pos(const KvAddr& k, int t) { return k.row_pos ? k.row_pos[t] : k.p0 + t; }
__device__ __forceinline__ int row_seq(const KvAddr& k, int t) { return k.row_seq ? k.row_seq[t] : k.seq0; }
// element offset of (sequence, kv head, position)'s K/V row
__device__ __forceinline__ size_t kv_row(const KvAddr& k, int kv_heads, int hd, int seq, int kv, int pos) {
  if (!k.pages) return ((size_t)kv * k.ctx + pos) * hd;
  const int page = k.pages[(size_t)seq * k.max_pages + pos / kKvPage];
  return (((size_t)page * kv_heads + kv) * kKvPage + (pos & (kKvPage - 1))) * hd;
}

// Per-head q/k RMSNorm and rotary embedding of every prompt row (position
// p0 + t), the new k and v into the cache. One wave per (row, head): workgroup
// (t, y) holds heads 4y .. 4y + 3 of the q heads followed by the kv heads. A
// lane owns rotary pairs p = lane + 64 j and gathers their two elements (and,
// for a kv head, its v dims) straight from the projections' partial sums, every
// load issued at once. Same operation order as the decode attention's phase B.
// The rotated q goes to the q part of the row for the attention kernels.
__global__ __launch_bounds__(kWg) void k_pf_rope_kv(PfRopeArgs a) {
  constexpr int NP = 2;  // pairs per lane: head_dim <= 256
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = blockIdx.y * 4 + wave;
  const int nh = a.heads + a.kv_heads;
  if (hh >= nh) return;
  const int pos = row_pos(a.kv, t);
  const int hd = a.hd, half = hd / 2;
  const bool is_k = hh >= a.heads;
  const int kv = hh - a.heads;
  float* row = a.qkv + (size_t)t * a.ld;
  const int col = is_k ? a.heads * hd + kv * hd : hh * hd;  // the head's columns in the q|k|v row
  const PartSum& P = is_k ? a.pk : a.pq;
  const int pcol = is_k ? kv * hd : hh * hd;                 // ... in its projection's result
  int ia[NP], ib[NP];
  float x0[NP], x1[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int d = min(lane + 64 * j, half - 1);
    ia[j] = a.interleaved ? 2 * d : d;
    ib[j] = a.interleaved ? 2 * d + 1 : d + half;
  }
  if (P.p) {
    // both elements of every pair in one round of loads
    int jj[2 * NP];
    float xx[2 * NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      jj[2 * j] = pcol + ia[j];
      jj[2 * j + 1] = pcol + ib[j];
    }
    part_gather<2 * NP>(P, t, jj, xx);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      x0[j] = xx[2 * j];
      x1[j] = xx[2 * j + 1];
    }
  } else {
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      x0[j] = row[col + ia[j]];
      x1[j] = row[col + ib[j]];
    }
  }
  float r = 1.0f;
  if (a.qn_w) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NP; ++j)
      if (lane + 64 * j < half) ss += x0[j] * x0[j] + x1[j] * x1[j];
    ss = wave_sum(ss);
    r = 1.0f / sqrtf(ss / (float)hd + a.eps);
  }
  const float* w = is_k ? a.kn_w : a.qn_w;
  size_t base = 0;
  if (is_k) base = kv_row(a.kv, a.kv_heads, hd, row_seq(a.kv, t), kv, pos);
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int d = lane + 64 * j;
    if (d >= half) continue;
    float v0 = x0[j], v1 = x1[j];
    if (a.qn_w) {
      v0 = __fmul_rn(__fmul_rn(v0, r), w[ia[j]]);
      v1 = __fmul_rn(__fmul_rn(v1, r), w[ib[j]]);
    }
    const float ang = __fmul_rn((float)pos, a.rope_inv[d]);
    const float co = cosf(ang), si = sinf(ang);
    const float y0 = __fsub_rn(__fmul_rn(v0, co), __fmul_rn(v1, si));
    const float y1 = __fadd_rn(__fmul_rn(v0, si), __fmul_rn(v1, co));
    if (is_k) {
      if (a.kv16) {
        ((__half*)a.kv.kc)[base + ia[j]] = __float2half_rn(y0);
        ((__half*)a.kv.kc)[base + ib[j]] = __float2half_rn(y1);
      } else {
        ((float*)a.kv.kc)[base + ia[j]] = y0;
        ((float*)a.kv.kc)[base + ib[j]] = y1;
      }
    } else {
      row[col + ia[j]] = y0;
      row[col + ib[j]] = y1;
    }
  }
  if (is_k) {
    const int vcol = (a.heads + a.kv_heads) * hd + kv * hd;
    // lane's dims lane + 64 i (head_dim <= 256), every load issued at once
    int jv[4];
    float vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) jv[i] = min(lane + 64 * i, hd - 1);
    if (a.pv.p) {
#pragma unroll
      for (int i = 0; i < 4; ++i) jv[i] += kv * hd;
      part_gather<4>(a.pv, t, jv, vv);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) vv[i] = row[vcol + jv[i]];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d >= hd) continue;
      if (a.kv16)
        ((__half*)a.kv.vc)[base + d] = __float2half_rn(vv[i]);
      else
        ((float*)a.kv.vc)[base + d] = vv[i];
    }
  }
}

// Causal attention of every prompt row: one workgroup per (token, q head),
// keys [start, p0 + t] of the cache in blocks of 256 (one per thread), an
// online softmax across blocks. q is the rotated row left by k_pf_rope_kv.
__global__ __launch_bounds__(kWg) void k_pf_attn(PfAttnArgs a) {
  __shared__ float qs[256];
  __shared__ float red[8];
  __shared__ float wsh[kWg];
  __shared__ float part[kWg];
  const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int G = a.heads / a.kv_heads, kv = h / G;
  const int hd = a.hd;
  const int pos = row_pos(a.kv, t);
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const float* q = a.qkv + (size_t)t * a.ld + h * hd;
  for (int d = tid; d < hd; d += kWg) qs[d] = q[d];
  __syncthreads();
  const size_t head_base = (size_t)kv * a.kv.ctx * hd;
  float M = -INFINITY, L = 0.f;
  // output dims: thread tid owns dim (tid % hd) for key slice tid / hd
  const int nsl = kWg / hd, my_d = tid % hd, my_sl = tid / hd;
  float o = 0.f;
  for (int b0 = start; b0 <= pos; b0 += kWg) {
    const int p = b0 + tid;
    float s = -INFINITY;
    if (p <= pos) {
      float acc = 0.f;
      if (a.kv16) {
        const __half* kr = (const __half*)a.kv.kc + head_base + (size_t)p * hd;
        for (int d = 0; d < hd; d += 8) {
          const uint4 w4 = *(const uint4*)(kr + d);
          const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc += qs[d + 2 * i] * h2f(w[i]);
            acc += qs[d + 2 * i + 1] * h2f(w[i] >> 16);
          }
        }
      } else {
        const float* kr = (const float*)a.kv.kc + head_base + (size_t)p * hd;
        for (int d = 0; d < hd; ++d) acc += qs[d] * kr[d];
      }
      s = acc * a.scale;
    }
    float mb = wave_max(s);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = mb;
    __syncthreads();
    mb = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float e = p <= pos ? expf(s - mb) : 0.f;
    wsh[tid] = e;
    float lb = wave_sum(e);
    __syncthreads();
    if ((tid & 63) == 0) red[4 + (tid >> 6)] = lb;
    __syncthreads();
    lb = (red[4] + red[5]) + (red[6] + red[7]);
    const float Mn = fmaxf(M, mb);
    const float ro = M == -INFINITY ? 0.f : expf(M - Mn), rb = expf(mb - Mn);
    // weighted V of this block for my dim over my slice of the keys
    float ob = 0.f;
    const int nk = min(kWg, pos + 1 - b0);
    for (int kk = my_sl; kk < nk; kk += nsl) {
      const size_t vi = head_base + (size_t)(b0 + kk) * hd + my_d;
      const float vv = a.kv16 ? __half2float(((const __half*)a.kv.vc)[vi]) : ((const float*)a.kv.vc)[vi];
      ob += wsh[kk] * vv;
    }
    part[tid] = ob;
    __syncthreads();
    if (tid < hd) {
      float sb = 0.f;
      for (int sl = 0; sl < nsl; ++sl) sb += part[sl * hd + tid];
      o = o * ro + sb * rb;
    }
    L = L * ro + lb * rb;
    M = Mn;
    __syncthreads();
  }
  if (tid < hd) a.out[(size_t)t * a.ldo + h * hd + tid] = o * (1.0f / L);
}

// Causal attention of the prompt rows on the matrix cores (fp16 K/V cache):
// one workgroup per (block of 64 / G tokens, kv head); its 64 query rows
// (token, q head of the group) are four waves of 16. The products run
// transposed so that no operand needs a shuffle: per block of 64 keys,
//   S^T = K Q^T  (v_mfma 16x16x32: K rows from LDS, q split into fp16 hi + lo),
// whose accumulator layout (lane: query lane % 16, keys 4 (lane / 16) + i of
// each 16-key tile) is the B operand layout of the 16x16x16 product, so
//   O^T += V^T P^T  (P split into hi + lo; V^T staged in LDS, V exact)
// takes P straight from the registers, and every lane keeps the running
// maximum, sum and output of its own query. Scores are kept in log2 units
// (scale * log2 e folded into one multiply) and the exponent base is only
// raised when a block's maximum exceeds it by more than 8 (P <= 2^8 stays
// exact enough in fp16 hi + lo and the sums in fp32), so the output rescale
// is skipped by the whole wave on most blocks; blocks that no query of the
// wave sees partly masked skip the masking. The next block's K and V are
// loaded into registers while the current one is multiplied; workgroups
// with the most keys (the last tokens) are dispatched first, and workgroup
// ids step through the kv heads fastest: consecutive ids go to different XCDs
// (id mod 8), so with 8 kv heads each XCD's L2 holds one head's K/V.
constexpr int kFaKeys = 64;

__device__ __forceinline__ float4_t mfma16(half4_t a, half4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// max / sum over the four lanes of one query (lanes l, l ^ 16, l ^ 32, l ^ 48)
__device__ __forceinline__ float xquad_max(float v) {
  float a, b;
  swap16(v, a, b);
  v = fmaxf(a, b);
  swap32(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xquad_sum(float v) {
  float a, b;
  swap16(v, a, b);
  v = a + b;
  swap32(v, a, b);
  return a + b;
}

template <int HD, bool PAGED>
__global__ __launch_bounds__(kWg) void k_pf_fattn(PfAttnArgs a) {
  extern __shared__ __align__(16) _Float16 fsm[];
  constexpr int KS = HD + 8, VS = kFaKeys + 8;
  constexpr int NKP = HD / 32;                   // K pieces (8 halves) per thread and block
  constexpr int NVI = HD >= 64 ? HD / 64 : 1;    // V items (2 keys x 8 dims) per thread and block
  constexpr int VITEMS = (kFaKeys / 2) * (HD / 8);
  _Float16* ks = fsm;                  // [64 keys][KS]
  _Float16* vt = ks + kFaKeys * KS;    // [HD dims][VS]   (V transposed)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // rows of one workgroup share a sequence: one token per workgroup when
  // every row has its own
  const int G = a.heads / a.kv_heads, TW = a.kv.row_seq ? 1 : 64 / G;
  const int ntiles = gridDim.x / a.kv_heads;
  // query tiles in complementary pairs: workgroups q and q + hi (dispatched
  // one dispatch round apart, so that one CU holds both while the grid is two
  // rounds) take tiles ntiles - 1 - q and q, whose causal key ranges sum to a
  // constant
  const int q = (int)blockIdx.x / a.kv_heads, hi = ntiles - ntiles / 2;
  const int kv = blockIdx.x % a.kv_heads, t0 = (q < hi ? ntiles - 1 - q : q - hi) * TW;
  const int col = lane & 15, quad = lane >> 4;
  const int seq = row_seq(a.kv, t0);
  const __half* kc = (const __half*)a.kv.kc;
  const __half* vc = (const __half*)a.kv.vc;

  // this lane's query: row 16 * wave + col of the workgroup (token, head);
  // its B operand of S^T (dims 32 k + 8 quad .. + 8), hi and lo halves
  const int qr = 16 * wave + col, qt = t0 + qr / G;
  const bool qok = qr < TW * G && qt < a.rows;
  half8_t qh[HD / 32], ql[HD / 32];
  {
    const float* q = a.qkv + (size_t)(qok ? qt : t0) * a.ld + (kv * G + qr % G) * HD;
#pragma unroll
    for (int k = 0; k < HD / 32; ++k) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = q[32 * k + 8 * quad + i];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = qok ? v[i] : 0.f;
        qh[k][i] = (_Float16)x;
        ql[k][i] = (_Float16)(x - (float)qh[k][i]);
      }
    }
  }
  const int qpos = qok ? row_pos(a.kv, qt) : -1;
  const int qstart = (a.window != 0 && qpos + 1 > a.window) ? qpos + 1 - a.window : 0;
  // the wave's key range seen by every one of its queries (unused rows excluded)
  const int wpos_min = (int)-wave_max(-(float)(qok ? qpos : 1 << 24));
  const int wstart_max = (int)wave_max((float)(qok ? qstart : 0));
  const float sl2 = a.scale * 1.44269504088896341f;
  const int t_last = min(t0 + TW, a.rows) - 1;
  const int pos_hi = row_pos(a.kv, t_last), pos_lo = row_pos(a.kv, t0);
  const int st_lo = (a.window != 0 && pos_lo + 1 > a.window) ? pos_lo + 1 - a.window : 0;
  const int kb_lo = st_lo / kFaKeys, kb_hi = pos_hi / kFaKeys;

  // staging: K piece (key, 8 dims) and V item (key pair, 8 dims) of the thread
  uint4 kreg[NKP], vreg[NVI][2];
  // block kb's first K/V row (workgroup-uniform) and the last row of the block
  // that may be addressed (the cache ends inside the block)
  auto block_base = [&](int kb) -> size_t {
    if constexpr (PAGED) {
      const int page = ld_scalar(a.kv.pages + (size_t)seq * a.kv.max_pages + kb);
      return ((size_t)page * a.kv_heads + kv) * kKvPage * HD;
    } else {
      return ((size_t)kv * a.kv.ctx + kb * kFaKeys) * HD;
    }
  };
  auto key_cap = [&](int kb) -> int { return PAGED ? kFaKeys - 1 : min(kFaKeys - 1, a.kv.ctx - 1 - kb * kFaKeys); };
  // Keys past the block's last position were never written (fresh pages can
  // hold NaN bit patterns, and P = 0 times NaN is NaN): staged as zeros.
  auto fetch = [&](int kb) {
    const int k0 = kb * kFaKeys, cap = key_cap(kb);
    const size_t base = block_base(kb);
    const __half* kb0 = kc + base;
    const __half* vb0 = vc + base;
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int piece = tid + kWg * j, key = piece / (HD / 8), d8 = (piece % (HD / 8)) * 8;
      const uint4 v = ldg4(kb0 + (uint32_t)(min(key, cap) * HD + d8));
      kreg[j] = k0 + key <= pos_hi ? v : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < NVI; ++j) {
      const int item = min(tid + kWg * j, VITEMS - 1), kp = item % (kFaKeys / 2), d8 = (item / (kFaKeys / 2)) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = 2 * kp + h;
        const uint4 v = ldg4(vb0 + (uint32_t)(min(key, cap) * HD + d8));
        vreg[j][h] = k0 + key <= pos_hi ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int j = 0; j < NKP; ++j) {
      const int piece = tid + kWg * j, key = piece / (HD / 8), d8 = (piece % (HD / 8)) * 8;
      *(uint4*)(ks + key * KS + d8) = kreg[j];
    }
#pragma unroll
    for (int j = 0; j < NVI; ++j) {
      const int item = tid + kWg * j, kp = item % (kFaKeys / 2), d8 = (item / (kFaKeys / 2)) * 8;
      if (item < VITEMS) {
        // dims d8 .. d8 + 7 of keys 2 kp and 2 kp + 1 as eight (key, key + 1) pairs
        const uint32_t* w0 = (const uint32_t*)&vreg[j][0];
        const uint32_t* w1 = (const uint32_t*)&vreg[j][1];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          *(uint32_t*)(vt + (d8 + 2 * d) * VS + 2 * kp) = (w0[d] & 0xffffu) | (w1[d] << 16);
          *(uint32_t*)(vt + (d8 + 2 * d + 1) * VS + 2 * kp) = (w0[d] >> 16) | (w1[d] & 0xffff0000u);
        }
      }
    }
  };

  float m_use = -INFINITY, l_run = 0.f;  // exponent base (log2 units) and running sum of the lane's query
  float4_t o[HD / 16];  // O^T tiles: dims 16 dt + 4 quad + i of the lane's query
#pragma unroll
  for (int d = 0; d < HD / 16; ++d) o[d] = float4_t{0.f, 0.f, 0.f, 0.f};

  fetch(kb_lo);
  for (int kb = kb_lo; kb <= kb_hi; ++kb) {
    const int k0 = kb * kFaKeys;
    __syncthreads();  // the previous block's K / V^T are consumed
    stage();
    __syncthreads();
    fetch(min(kb + 1, kb_hi));  // the next block (the last one again at the end: cache hits)
    // S^T for the block's 64 keys x the wave's 16 queries (four 16 x 16 tiles)
    float s[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < HD / 32; ++k) {
        const half8_t kk = *(const half8_t*)(ks + (16 * kt + col) * KS + 32 * k + 8 * quad);
        acc = mfma32(kk, qh[k], acc);
        acc = mfma32(kk, ql[k], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kt][i] = acc[i] * sl2;
    }
    if (!(k0 >= wstart_max && k0 + kFaKeys - 1 <= wpos_min)) {
      // some query of the wave sees only part of the block
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + 16 * kt + 4 * quad + i;
          s[kt][i] = key >= qstart && key <= qpos ? s[kt][i] : -INFINITY;
        }
    }
    float mb = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mb = fmaxf(mb, s[kt][i]);
    mb = xquad_max(mb);
    const bool upd = mb > m_use + 8.0f;
    const float alpha = !upd ? 1.0f : (m_use == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_use - mb));
    m_use = upd ? mb : m_use;
    const float base = m_use == -INFINITY ? 0.f : m_use;  // masked scores give exp2(-inf) = 0
    float lb = 0.f;
    half4_t ph[4], pl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(s[kt][i] - base);
        lb += p;
        ph[kt][i] = (_Float16)p;
        pl[kt][i] = (_Float16)(p - (float)ph[kt][i]);
      }
    l_run = l_run * alpha + xquad_sum(lb);
    if (__builtin_amdgcn_ballot_w64(upd) != 0) {
#pragma unroll
      for (int d = 0; d < HD / 16; ++d) o[d] *= alpha;
    }
    // O^T += V^T P^T over the block's keys (four 16-key steps)
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const half4_t vv = *(const half4_t*)(vt + (16 * d + col) * VS + 16 * kt + 4 * quad);
        o[d] = mfma16(vv, ph[kt], o[d]);
        o[d] = mfma16(vv, pl[kt], o[d]);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the last redundant fetch has returned
  // out[token][head * HD + dim]: the lane's query, dims 16 d + 4 quad .. + 4
  if (qok) {
    float* out = a.out + (size_t)qt * a.ldo + (kv * G + qr % G) * HD;
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int d = 0; d < HD / 16; ++d)
      *(float4*)(out + 16 * d + 4 * quad) = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
  }
}

// Decode attention of batch rows over paged K/V. One workgroup per (kv head,
// row, segment) walks a segment of the row's pages [start, pos] with the
// decode attention's layout: a page's K rows in registers (four lanes per
// position), its V rows in registers (wave w holds dims [w*HD/4, (w+1)*HD/4)
// of every position, a lane 2 or 4 dims of every PG-th position); the next
// page's rows are requested before the current page is reduced. The softmax
// runs online over the pages (running maximum and sum per head, the
// accumulators rescaled when the maximum grows). With one segment per row the
// workgroup writes the attention output; otherwise a partial [max, sum,
// acc[hd]] per head for k_bd_merge.
template <int HD, bool ROPE>
__global__ __launch_bounds__(kWg) void k_bd_walk(PfAttnArgs a, float* part, int max_pages, int nseg, PfRopeArgs ra) {
  warm_kernarg<(int)(sizeof(PfAttnArgs) + 2 * sizeof(void*) + sizeof(PfRopeArgs))>();  // (dependent argument rounds hit the scalar cache)
  constexpr int DPT = HD / 4;  // K dims per lane
  constexpr int NKV = DPT / 8;
  constexpr int VD = HD >= 256 ? 4 : 2, VW = VD / 2;
  constexpr int DW = HD / 4 / VD;  // lanes per V position row: 8 or 16
  constexpr int LDW = DW == 8 ? 3 : 4;
  constexpr int PG = 64 / DW, NP = kKvPage / PG;
  static_assert(kKvPage == 64 && (DW == 8 || DW == 16), "page geometry");
  __shared__ __align__(16) float q_s[8 * HD];
  __shared__ float wmx[4][8];
  __shared__ __align__(16) float ew[8][kKvPage];
  __shared__ float lsum[8];
  __shared__ int pt_s[64];  // the segment's page table entries (max_pages <= 64)
  const int kv = blockIdx.x, r = blockIdx.y, sg = blockIdx.z, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.heads / a.kv_heads;
  // With ROPE, the rotary/K-V write of this (row, kv head) comes first (the
  // arithmetic of k_pf_rope_kv): the G q heads, k and v, gathered from the
  // projections' partial sums, are G + 2 items over the waves; q goes to LDS,
  // k and v to the cache. Item `it`: four elements per lane (q/k: the two
  // elements of the lane's rotary pairs lane and lane + 64; v: dims lane + 64 e),
  // clamped so that every item issues the same loads. The first item's loads
  // go out before anything else.
  constexpr int NPR = 2;  // pairs per lane: head_dim <= 256
  constexpr int HALF = HD / 2;
  int ia[NPR], ib[NPR];
#pragma unroll
  for (int j = 0; j < NPR; ++j) {
    const int d = min(lane + 64 * j, HALF - 1);
    ia[j] = ra.interleaved ? 2 * d : d;
    ib[j] = ra.interleaved ? 2 * d + 1 : d + HALF;
  }
  // item it's partial sums and columns
  auto item_cols = [&](int it, int (&jj)[4]) -> const PartSum& {
    if (it == G + 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) jj[e] = kv * HD + min(lane + 64 * e, HD - 1);
      return ra.pv;
    }
    const int pcol = it == G ? kv * HD : (kv * G + it) * HD;
#pragma unroll
    for (int j = 0; j < NPR; ++j) {
      jj[2 * j] = pcol + ia[j];
      jj[2 * j + 1] = pcol + ib[j];
    }
    return it == G ? ra.pk : ra.pq;
  };
  const int it0 = min(wave, G + 1);
  int jj0[4];
  float w0[4][4];
  if constexpr (ROPE) part_issue<4>(item_cols(it0, jj0), r, jj0, w0);
  // The row's position and sequence and its page table entries are read
  // through the scalar cache (the scalar load counter is separate: waiting for
  // them never waits for the vector loads in flight), and the segment's
  // entries are staged in LDS for the page loop.
  const int pos = ld_scalar(a.kv.row_pos + r);
  const int start = (a.window != 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
  const int j_lo = start / kKvPage, np = pos / kKvPage - j_lo + 1;
  // this segment's pages [p_lo, p_hi) of the row's range
  const int p_lo = j_lo + np * sg / nseg, p_hi = j_lo + np * (sg + 1) / nseg;  // np, nseg <= 64
  const int seq = ld_scalar(a.kv.row_seq + r);
  const int* ptab = a.kv.pages + (size_t)seq * a.kv.max_pages;
  const int jnew = pos / kKvPage;  // the newest page (entries past it may be unassigned)
  const int pt_mine = ptab[min(p_lo + tid, jnew)];
  const int phys0 = ld_scalar(ptab + min(p_lo, jnew));
  const float* q = a.qkv + (size_t)r * a.ld + kv * G * HD;
  const int kp = 16 * wave + (lane >> 2), kd0 = (lane & 3) * DPT;
  const int pg = lane >> LDW, vd = wave * (HD / 4) + VD * (lane & (DW - 1));
  const int ei = (kp % PG) * NP + kp / PG;
  // a page's rows are addressed from a workgroup-uniform base with 32-bit
  // per-lane byte offsets (scalar base + vector offset loads: no 64-bit
  // address arithmetic per load)
  const uint32_t koff = 2u * (uint32_t)(kp * HD + kd0), voff = 2u * (uint32_t)(pg * HD + vd);
  auto load = [&](int phys, uint4 (&kr)[NKV], uint32_t (&vr)[NP][VW]) {
    const size_t pb = ((size_t)__builtin_amdgcn_readfirstlane(phys) * a.kv_heads + kv) * (kKvPage * HD * 2);
    const char* kb = (const char*)a.kv.kc + pb;
    const char* vb = (const char*)a.kv.vc + pb;
#pragma unroll
    for (int v = 0; v < NKV; ++v) kr[v] = ldg4(kb + koff + 16 * v);
#pragma unroll
    for (int t = 0; t < NP; ++t) {
      const char* p = vb + (2 * PG * HD) * t + voff;
      if constexpr (VW == 1) {
        vr[t][0] = ldg1(p);
      } else {
        const uint2 w = ldg2(p);
        vr[t][0] = w.x;
        vr[t][VW - 1] = w.y;
      }
    }
  };
  float mrun[8], o[8][VD];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    mrun[g] = -INFINITY;
#pragma unroll
    for (int k = 0; k < VD; ++k) o[g][k] = 0.f;
  }
  float lrun[8];  // wave g % 4's running sum of head g
#pragma unroll
  for (int g = 0; g < 8; ++g) lrun[g] = 0.f;
  auto page = [&](int j, uint4 (&kr)[NKV], uint32_t (&vr)[NP][VW]) {
    const int k0 = j * kKvPage;
    const bool valid = k0 + kp >= start && k0 + kp <= pos;
    float s[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) s[g] = 0.f;
#pragma unroll
    for (int v = 0; v < NKV; ++v) {
      const uint32_t w[4] = {kr[v].x, kr[v].y, kr[v].z, kr[v].w};
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if (g < G) {
          const float4 q0 = *(const float4*)(q_s + g * HD + kd0 + 8 * v);
          const float4 q1 = *(const float4*)(q_s + g * HD + kd0 + 8 * v + 4);
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
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        const float sc = group_sum<4>(s[g]);
        s[g] = valid ? sc * a.scale : -INFINITY;
        const float mw = wave_max(s[g]);
        if (lane == 0) wmx[wave][g] = mw;
      }
    }
    __syncthreads();  // the page maxima (and the previous page's weights are consumed)
    float alpha[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        const float mp = fmaxf(fmaxf(wmx[0][g], wmx[1][g]), fmaxf(wmx[2][g], wmx[3][g]));
        const float mn = fmaxf(mrun[g], mp);  // finite: every page of the range holds a position
        alpha[g] = exp_fast(mrun[g] - mn);     // 0 on the first page
        mrun[g] = mn;
        const float e = valid ? exp_fast(s[g] - mn) : 0.f;
        if ((lane & 3) == 0) ew[g][ei] = e;
      }
    }
    __syncthreads();  // the page's weights
    if (k0 < start || k0 + kKvPage - 1 > pos) {
#pragma unroll
      for (int t = 0; t < NP; ++t) {
        const int p = k0 + pg + PG * t;
        if (p < start || p > pos)
#pragma unroll
          for (int u = 0; u < VW; ++u) vr[t][u] = 0u;
      }
    }
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      if (g < G) {
        if (g % 4 == wave) lrun[g] = lrun[g] * alpha[g] + wave_sum(ew[g][lane]);
#pragma unroll
        for (int k = 0; k < VD; ++k) o[g][k] *= alpha[g];
#pragma unroll
        for (int t4 = 0; t4 < NP / 4; ++t4) {
          const float4 w4 = *(const float4*)(&ew[g][pg * NP + 4 * t4]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 4 * t4 + i;
            const float wt = i == 0 ? w4.x : i == 1 ? w4.y : i == 2 ? w4.z : w4.w;
#pragma unroll
            for (int u = 0; u < VW; ++u) {
              o[g][2 * u] = fmaf(wt, h2f(vr[t][u]), o[g][2 * u]);
              o[g][2 * u + 1] = fmaf(wt, h2f(vr[t][u] >> 16), o[g][2 * u + 1]);
            }
          }
        }
      }
    }
  };
  uint4 ka[NKV], kb2[NKV];
  uint32_t va[NP][VW], vb2[NP][VW];
  if constexpr (ROPE) {
    // (one segment) the first page is requested before the rotary work; when
    // it is the newest, it is requested again after the barrier below that
    // publishes the new row
    load(phys0, ka, va);
    const size_t base = (((size_t)ld_scalar(ptab + jnew) * ra.kv_heads + kv) * kKvPage + (pos & (kKvPage - 1))) * HD;
    auto item_do = [&](int it, const float (&xx)[4]) {
      if (it == G + 1) {
#pragma unroll
        for (int e = 0; e < HD / 64; ++e) ((__half*)ra.kv.vc)[base + lane + 64 * e] = __float2half_rn(xx[e]);
        return;
      }
      const bool is_k = it == G;
      const float x0[NPR] = {xx[0], xx[2]}, x1[NPR] = {xx[1], xx[3]};
      float rn = 1.0f;
      if (ra.qn_w) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NPR; ++j)
          if (lane + 64 * j < HALF) ss += x0[j] * x0[j] + x1[j] * x1[j];
        ss = wave_sum(ss);
        rn = 1.0f / sqrtf(ss / (float)HD + ra.eps);
      }
      const float* w = is_k ? ra.kn_w : ra.qn_w;
#pragma unroll
      for (int j = 0; j < NPR; ++j) {
        const int d = lane + 64 * j;
        if (d >= HALF) continue;
        float v0 = x0[j], v1 = x1[j];
        if (ra.qn_w) {
          v0 = __fmul_rn(__fmul_rn(v0, rn), w[ia[j]]);
          v1 = __fmul_rn(__fmul_rn(v1, rn), w[ib[j]]);
        }
        const float ang = __fmul_rn((float)pos, ra.rope_inv[d]);
        const float co = cosf(ang), si = sinf(ang);
        const float y0 = __fsub_rn(__fmul_rn(v0, co), __fmul_rn(v1, si));
        const float y1 = __fadd_rn(__fmul_rn(v0, si), __fmul_rn(v1, co));
        if (is_k) {
          ((__half*)ra.kv.kc)[base + ia[j]] = __float2half_rn(y0);
          ((__half*)ra.kv.kc)[base + ib[j]] = __float2half_rn(y1);
        } else {
          q_s[it * HD + ia[j]] = y0;
          q_s[it * HD + ib[j]] = y1;
        }
      }
    };
    if (wave < G + 2) {
      float xx[4];
      part_finish<4>(item_cols(it0, jj0), r, jj0, w0, xx);
      item_do(wave, xx);
    }
    for (int it = wave + 4; it < G + 2; it += 4) {  // groups above 2
      int jj[4];
      float xx[4];
      part_gather<4>(item_cols(it, jj), r, jj, xx);
      item_do(it, xx);
    }
    if (tid < 64) pt_s[tid] = pt_mine;
    __syncthreads();  // q and the page table in LDS; the new K/V row visible to this workgroup's loads
    if (p_lo == jnew) load(phys0, ka, va);
  } else {
    // q first: its loads complete before the page's, which stay in flight
    float qv[6];
#pragma unroll
    for (int c = 0; c < 6; ++c) qv[c] = tid + kWg * c < G * HD ? q[tid + kWg * c] : 0.f;
    if (p_lo < p_hi) load(phys0, ka, va);
#pragma unroll
    for (int c = 0; c < 6; ++c)
      if (tid + kWg * c < G * HD) q_s[tid + kWg * c] = qv[c];
    if (tid < 64) pt_s[tid] = pt_mine;
    __syncthreads();
  }
  // The next page's loads are issued unconditionally (the last page requests
  // itself again, a cache hit) so that the loop body has no branch around
  // them: the compiler's load-counter waits then count exactly and page j's
  // reduction waits for page j's rows only.
  for (int j = p_lo; j < p_hi; j += 2) {
    load(pt_s[min(j + 1, p_hi - 1) - p_lo], kb2, vb2);
    __builtin_amdgcn_sched_barrier(0);  // issued before page j's reduction starts
    page(j, ka, va);
    if (j + 1 >= p_hi) break;
    load(pt_s[min(j + 2, p_hi - 1) - p_lo], ka, va);
    __builtin_amdgcn_sched_barrier(0);
    page(j + 1, kb2, vb2);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the last redundant request has returned
#pragma unroll
  for (int g = 0; g < 8; ++g)
    if (g < G)
#pragma unroll
      for (int k = 0; k < VD; ++k) o[g][k] = pg_sum<DW>(o[g][k]);
  // lanes (pg, dw) write item pg + PG * it (head item / VD, dim vd + item % VD)
  if (nseg == 1) {
    if (lane == 0)
#pragma unroll
      for (int g = 0; g < 8; ++g)
        if (g < G && g % 4 == wave) lsum[g] = lrun[g];
    __syncthreads();
    const size_t col = (size_t)kv * G * HD;
    for (int it = 0; it * PG < G * VD; ++it) {
      const int item = it * PG + pg;
      float val = 0.f;
#pragma unroll
      for (int g = 0; g < 8; ++g)
#pragma unroll
        for (int k = 0; k < VD; ++k)
          if (g * VD + k == item) val = o[g][k];
      if (item < G * VD) {
        const size_t i = col + (item / VD) * HD + vd + item % VD;
        const float y = val / lsum[item / VD];
        if (a.oh) {
          // the next GEMM's operand planes at scale 1: hi + lo keeps ~22 bits
          // for |y| >= 2^-3; below that lo is an fp16 subnormal (absolute
          // spacing 2^-24), so the relative error grows to ~2^-24 / |y|
          // (2^-17 at 0.01, 2^-14 at 1e-3), still far inside the 1e-3 logits bar
          const _Float16 h = (_Float16)y;
          a.oh[(size_t)r * a.okpad + i] = h;
          a.ol[(size_t)r * a.okpad + i] = (_Float16)(y - (float)h);
        } else {
          a.out[(size_t)r * a.ldo + i] = y;
        }
      }
    }
    if (a.oh && kv == 0) {
      // the planes past the row's last column are zero; its scale is 1
      for (int i = a.heads * HD + tid; i < a.okpad; i += kWg) {
        a.oh[(size_t)r * a.okpad + i] = (_Float16)0.f;
        a.ol[(size_t)r * a.okpad + i] = (_Float16)0.f;
      }
      if (tid == 0) a.oscale[r] = 1.0f;
    }
  } else {
    const int rowf = attn_rowf(G, HD);
    float* out = part + (((size_t)r * a.kv_heads + kv) * max_pages + sg) * rowf;
    for (int it = 0; it * PG < G * VD; ++it) {
      const int item = it * PG + pg;
      float val = 0.f;
#pragma unroll
      for (int g = 0; g < 8; ++g)
#pragma unroll
        for (int k = 0; k < VD; ++k)
          if (g * VD + k == item) val = o[g][k];
      if (item < G * VD) out[(item / VD) * (HD + 2) + 2 + vd + item % VD] = val;
    }
    if (lane == 0)
#pragma unroll
      for (int g = 0; g < 8; ++g)
        if (g < G && g % 4 == wave) {
          out[g * (HD + 2)] = mrun[g];  // -inf for a segment without pages
          out[g * (HD + 2) + 1] = lrun[g];
        }
  }
}

// out row r, heads of kv head blockIdx.x: the segments' partials merged
// (weights exp(m_j - M), normalised by the merged sum).
template <int HD>
__global__ __launch_bounds__(kWg) void k_bd_merge(PfAttnArgs a, const float* part, int max_pages, int nseg) {
  __shared__ float w[8][64];
  __shared__ float inv[8];
  const int kv = blockIdx.x, r = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = a.heads / a.kv_heads;
  const int n = nseg;
  const int rowf = attn_rowf(G, HD);
  const float* base = part + ((size_t)r * a.kv_heads + kv) * max_pages * rowf;
  for (int g = wave; g < G; g += 4) {
    float M = -INFINITY;
    for (int j = lane; j < n; j += 64) M = fmaxf(M, base[(size_t)j * rowf + g * (HD + 2)]);
    M = wave_max(M);
    float L = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float mj = base[(size_t)j * rowf + g * (HD + 2)];
      const float f = mj == -INFINITY ? 0.f : expf(mj - M);
      w[g][j] = f;
      L += base[(size_t)j * rowf + g * (HD + 2) + 1] * f;
    }
    L = wave_sum(L);
    if (lane == 0) inv[g] = 1.0f / L;
  }
  __syncthreads();
  for (int i = tid; i < G * HD; i += kWg) {
    const int g = i / HD, d = i - g * HD;
    float acc = 0.f;
    for (int j = 0; j < n; ++j) acc += base[(size_t)j * rowf + g * (HD + 2) + 2 + d] * w[g][j];
    a.out[(size_t)r * a.ldo + (kv * G + g) * HD + d] = acc * inv[g];
  }
}

// Greedy id of each row of logits: the largest value, the lowest index on
// ties, NaN never chosen (argmax's better(), llama-wgsl-runtime.ts:3645-3791).
// Stage 1: kArgParts workgroups per row each reduce a slice to (value, id).
constexpr int kArgParts = 32;

__global__ __launch_bounds__(kWg) void k_row_argmax1(const float* logits, int vocab, float* pv, uint32_t* pi) {
  __shared__ float sv[kWg];
  __shared__ uint32_t si[kWg];
  const float* row = logits + (size_t)blockIdx.x * vocab;
  const int per = (vocab + kArgParts - 1) / kArgParts;
  const int lo = blockIdx.y * per, hi = min(vocab, lo + per);
  float bv = kNegBig;
  uint32_t bi = 0xffffffffu;
  for (int i = lo + threadIdx.x; i < hi; i += kWg) {
    const float v = row[i];
    if (better(v, (uint32_t)i, bv, bi)) {
      bv = v;
      bi = (uint32_t)i;
    }
  }
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int stride = kWg / 2; stride >= 1; stride >>= 1) {
    if ((int)threadIdx.x < stride && better(sv[threadIdx.x + stride], si[threadIdx.x + stride], sv[threadIdx.x],
                                            si[threadIdx.x])) {
      sv[threadIdx.x] = sv[threadIdx.x + stride];
      si[threadIdx.x] = si[threadIdx.x + stride];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pv[blockIdx.x * kArgParts + blockIdx.y] = sv[0];
    pi[blockIdx.x * kArgParts + blockIdx.y] = si[0];
  }
}

// Stage 2: one wave per row over the row's kArgParts candidates.
__global__ __launch_bounds__(64) void k_row_argmax2(const float* pv, const uint32_t* pi, int32_t* out) {
  __shared__ float sv[64];
  __shared__ uint32_t si[64];
  const int r = blockIdx.x, l = threadIdx.x;
  sv[l] = l < kArgParts ? pv[r * kArgParts + l] : kNegBig;
  si[l] = l < kArgParts ? pi[r * kArgParts + l] : 0xffffffffu;
  __syncthreads();
  for (int stride = 32; stride >= 1; stride >>= 1) {
    if (l < stride && better(sv[l + stride], si[l + stride], sv[l], si[l])) {
      sv[l] = sv[l + stride];
      si[l] = si[l + stride];
    }
    __syncthreads();
  }
  if (l == 0) out[r] = si[0] == 0xffffffffu ? 0 : (int32_t)si[0];
}

}  // namespace

// ---- host launchers ----------------------------------------------------------------

size_t gemm_shared_bytes() { return sizeof(_Float16) * (size_t)(2 * kGM) * kGS; }

// k_gemm addresses the activation planes with 32-bit byte offsets
bool gemm_planes_fit(const GemmArgs& a) { return a.t >= 1 && (int64_t)a.t * a.kpad * 2 <= (int64_t)UINT32_MAX; }

// k_gemm<type, tj> on the stream; false for a type without an instance
bool launch_gemm_tiles(const GemmArgs& a, int tj, dim3 grid, hipStream_t s) {
  const size_t sh = gemm_shared_bytes();
#define CHONK_GEMM_CASE(QT)                                                 \
  case QT:                                                                  \
    if (tj == 2)                                                            \
      hipLaunchKernelGGL((k_gemm<QT, 2>), grid, dim3(kWg), sh, s, a);       \
    else                                                                    \
      hipLaunchKernelGGL((k_gemm<QT, 1>), grid, dim3(kWg), sh, s, a);       \
    return true;
  switch (a.w.type) {
    CHONK_GEMM_CASE(QT_Q4_K)
    CHONK_GEMM_CASE(QT_Q5_K)
    CHONK_GEMM_CASE(QT_Q6_K)
    CHONK_GEMM_CASE(QT_Q8_0)
    CHONK_GEMM_CASE(QT_Q5_0)
    CHONK_GEMM_CASE(QT_Q5_1)
    default: return false;
  }
#undef CHONK_GEMM_CASE
}

size_t fattn_shared_bytes(int hd) {
  return sizeof(_Float16) * ((size_t)kFaKeys * (hd + 8) + (size_t)hd * (kFaKeys + 8));
}


hipError_t launch_gemm(const GemmArgs& a0, hipStream_t s) {
  GemmArgs a = a0;
  if (!a.n_all && gemm_sk_applies(a) && a.w.n >= 128 * 4 * kSkRows) {
    // many row groups (the lm_head): four per workgroup over the whole K, x shared in LDS
    const dim3 grid((a.w.n + 4 * kSkRows - 1) / (4 * kSkRows));
    if (a.w.type == QT_Q4_K)
      hipLaunchKernelGGL(k_gemm_lm<QT_Q4_K>, grid, dim3(kWg), gemm_lm_shared_bytes(), s, a);
    else
      hipLaunchKernelGGL(k_gemm_lm<QT_Q6_K>, grid, dim3(kWg), gemm_lm_shared_bytes(), s, a);
    return hipGetLastError();
  }
  if (!a.n_all && gemm_sk_applies(a)) {
    const int groups = (a.w.n + kSkRows - 1) / kSkRows;
    int ks = a.part ? gemm_sk_split(a, groups) : 1;
    while (ks > 1 && (int64_t)ks * a.t * a.w.n > a.part_cap) --ks;
    a.ksplit = ks;
    a.defer = 0;
    hipError_t e = launch_gemm_sk(a, a.w.n, s);
    if (e != hipSuccess || ks == 1) return e;
    const int64_t total = (int64_t)a.t * a.w.n;
    const int blocks = (int)std::min<int64_t>((total + kWg - 1) / kWg, 4096);
    hipLaunchKernelGGL(k_gemm_reduce, dim3(blocks), dim3(kWg), 0, s, a);
    return hipGetLastError();
  }
  if (!gemm_planes_fit(a)) return hipErrorInvalidValue;
  const int tj = gemm_tj(a.t), gt = gemm_tokens(tj);
  const int tiles = ((a.w.n + kGM - 1) / kGM) * ((a.t + gt - 1) / gt);
  const int nst = (a.w.k + kGK - 1) / kGK;
  a.ksplit = 1;
  if (a.part && tiles < 256) {
    int ks = std::min(nst, (256 + tiles - 1) / tiles);
    while (ks > 1 && (int64_t)ks * a.t * a.w.n > a.part_cap) --ks;
    a.ksplit = ks;
  }
  const dim3 grid((a.w.n + kGM - 1) / kGM, (a.t + gt - 1) / gt, a.ksplit);
  if (!launch_gemm_tiles(a, tj, grid, s)) return hipErrorInvalidValue;
  if (a.ksplit > 1) {
    const int64_t total = (int64_t)a.t * a.w.n;
    const int blocks = (int)std::min<int64_t>((total + kWg - 1) / kWg, 4096);
    hipLaunchKernelGGL(k_gemm_reduce, dim3(blocks), dim3(kWg), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_deferred(const GemmArgs& a0, float* region, int64_t region_cap, PartSum* out, hipStream_t s) {
  GemmArgs a = a0;
  const int N = a.n_all ? a.n_all : a.w.n;
  if (a.n_all) {
    // fused segments: one type and K, starts on tile boundaries, in order
    if (a.n1 <= 0 || a.n1 % kGM || a.n2 < a.n1 || a.n2 % kGM || a.n_all < a.n2 || a.w2.type != a.w.type ||
        a.w3.type != a.w.type || a.w2.k != a.w.k || a.w3.k != a.w.k || a.w.n != a.n1 ||
        (a.n2 > a.n1 && a.w2.n != a.n2 - a.n1) || (a.n_all > a.n2 && a.w3.n != a.n_all - a.n2))
      return hipErrorInvalidValue;
  }
  if ((int64_t)a.t * N > region_cap) return hipErrorInvalidValue;
  if (gemm_sk_applies(a)) {
    // one 64-k block per wave when the partial sums of that split fit
    const int ks1 = a.w.k / kSkBlockK / 4;
    const bool one = ks1 <= kMaxDeferSplit && (int64_t)ks1 * a.t * N <= region_cap;
    int ks = one ? ks1 : gemm_sk_split(a, (N + kSkRows - 1) / kSkRows);
    while (ks > 1 && (int64_t)ks * a.t * N > region_cap) --ks;
    a.ksplit = ks;
    a.part = region;
    a.defer = 1;
    hipError_t e;
    if (one) {
      const dim3 grid((N + kSkRows - 1) / kSkRows, 1, ks);
      if (a.w.type == QT_Q4_K)
        hipLaunchKernelGGL(k_gemm_sk1<QT_Q4_K>, grid, dim3(kWg), gemm_sk_shared_bytes(), s, a);
      else
        hipLaunchKernelGGL(k_gemm_sk1<QT_Q6_K>, grid, dim3(kWg), gemm_sk_shared_bytes(), s, a);
      e = hipGetLastError();
    } else {
      e = launch_gemm_sk(a, N, s);
    }
    out->p = region;
    out->n = N;
    out->ld = N;
    out->ks = ks;
    out->zs = (int64_t)a.t * N;
    return e;
  }
  if (!gemm_planes_fit(a)) return hipErrorInvalidValue;
  const int tj = gemm_tj(a.t), gt = gemm_tokens(tj);
  const int tiles = ((N + kGM - 1) / kGM) * ((a.t + gt - 1) / gt);
  const int nst = (a.w.k + kGK - 1) / kGK;
  // split K until about four workgroups per CU are queued (passes of 128-row
  // tiles; two with 64-row tiles); a decode batch (one row tile) runs faster
  // with half the CUs busy, as fewer, longer-running
  // workgroups amortise the stage pipeline's start (64 rows of the Qwen3-0.6B
  // shapes: 3.86 ms per step at 128, 3.99 at 512, 4.39 at 64)
  const int target = a.t <= 64 ? 128 : (tj == 2 ? 1024 : 512);
  int ks = tiles < target ? std::min(std::min(nst, kMaxDeferSplit), (target + tiles - 1) / tiles) : 1;
  while (ks > 1 && (int64_t)ks * a.t * N > region_cap) --ks;
  a.ksplit = ks;
  a.part = region;
  a.defer = 1;
  const dim3 grid((N + kGM - 1) / kGM, (a.t + gt - 1) / gt, ks);
  if (!launch_gemm_tiles(a, tj, grid, s)) return hipErrorInvalidValue;
  out->p = region;
  out->n = N;
  out->ld = N;
  out->ks = ks;
  out->zs = (int64_t)a.t * N;
  return hipGetLastError();
}

hipError_t init_gemm_attributes() {
  const size_t sh = gemm_shared_bytes();
  const void* fns[12] = {(const void*)k_gemm<QT_Q4_K, 1>, (const void*)k_gemm<QT_Q5_K, 1>, (const void*)k_gemm<QT_Q6_K, 1>,
                         (const void*)k_gemm<QT_Q8_0, 1>, (const void*)k_gemm<QT_Q5_0, 1>, (const void*)k_gemm<QT_Q5_1, 1>,
                         (const void*)k_gemm<QT_Q4_K, 2>, (const void*)k_gemm<QT_Q5_K, 2>, (const void*)k_gemm<QT_Q6_K, 2>,
                         (const void*)k_gemm<QT_Q8_0, 2>, (const void*)k_gemm<QT_Q5_0, 2>, (const void*)k_gemm<QT_Q5_1, 2>};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sh);
    if (e != hipSuccess) return e;
  }
  for (const void* f : {(const void*)k_gemm_sk<QT_Q4_K>, (const void*)k_gemm_sk<QT_Q6_K>,
                        (const void*)k_gemm_sk1<QT_Q4_K>, (const void*)k_gemm_sk1<QT_Q6_K>}) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_sk_shared_bytes());
    if (e != hipSuccess) return e;
  }
  const void* fa[8] = {(const void*)k_pf_fattn<32, false>,  (const void*)k_pf_fattn<64, false>,
                       (const void*)k_pf_fattn<128, false>, (const void*)k_pf_fattn<256, false>,
                       (const void*)k_pf_fattn<32, true>,   (const void*)k_pf_fattn<64, true>,
                       (const void*)k_pf_fattn<128, true>,  (const void*)k_pf_fattn<256, true>};
  const int hds[4] = {32, 64, 128, 256};
  for (int i = 0; i < 8; ++i) {
    const hipError_t e =
        hipFuncSetAttribute(fa[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)fattn_shared_bytes(hds[i & 3]));
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_pf_split(const PfSplitArgs& a, int rows, hipStream_t s) {
  if (a.kpad > 4 * kRowT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pf_split, dim3(rows), dim3(kRowT), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_pf_embed(const QMat& embed, const int32_t* tok, float scale, int k, float* x, int rows,
                           hipStream_t s) {
  hipLaunchKernelGGL(k_pf_embed, dim3(rows), dim3(kWg), 0, s, embed, tok, scale, k, x);
  return hipGetLastError();
}
hipError_t launch_pf_norm_add(const float* d, const float* w, float eps, int k, float* x, int rows, hipStream_t s) {
  hipLaunchKernelGGL(k_pf_norm_add, dim3(rows), dim3(kWg), 0, s, d, w, eps, k, x);
  return hipGetLastError();
}
hipError_t launch_pf_glu_split(const PfGluArgs& a, int rows, hipStream_t s) {
  if (a.kpad > 4 * kRowT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pf_glu_split, dim3(rows), dim3(kRowT), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_pf_rope_kv(const PfRopeArgs& a, int rows, hipStream_t s) {
  const int nh = a.heads + a.kv_heads;
  if (a.hd > 256) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_pf_rope_kv, dim3(rows, (nh + 3) / 4), dim3(kWg), 0, s, a);
  return hipGetLastError();
}
hipError_t launch_pf_attn(const PfAttnArgs& a, int rows, hipStream_t s) {
  const int G = a.heads / a.kv_heads;
  if (!a.kv16 || G > 16) {
    if (a.kv.pages || a.kv.row_seq) return hipErrorInvalidValue;  // paged rows need the fp16 cache
    hipLaunchKernelGGL(k_pf_attn, dim3(rows, a.heads), dim3(kWg), 0, s, a);
    return hipGetLastError();
  }
  PfAttnArgs b = a;
  b.rows = rows;
  const int tw = a.kv.row_seq ? 1 : 64 / G;
  const dim3 grid((rows + tw - 1) / tw * a.kv_heads);
  const size_t sh = fattn_shared_bytes(a.hd);
  const bool paged = a.kv.pages != nullptr;
#define CHONK_FA(H)                                                              \
  if (paged)                                                                     \
    hipLaunchKernelGGL((k_pf_fattn<H, true>), grid, dim3(kWg), sh, s, b);        \
  else                                                                           \
    hipLaunchKernelGGL((k_pf_fattn<H, false>), grid, dim3(kWg), sh, s, b);
  switch (a.hd) {
    case 32: CHONK_FA(32) break;
    case 64: CHONK_FA(64) break;
    case 128: CHONK_FA(128) break;
    case 256: CHONK_FA(256) break;
    default: return hipErrorInvalidValue;
  }
#undef CHONK_FA
  return hipGetLastError();
}

}  // namespace chonk

namespace chonk {
hipError_t launch_row_argmax(const float* logits, int vocab, int rows, float* scratch, int32_t* out, hipStream_t s) {
  float* pv = scratch;
  uint32_t* pi = (uint32_t*)(scratch + (size_t)rows * kArgParts);
  hipLaunchKernelGGL(k_row_argmax1, dim3(rows, kArgParts), dim3(kWg), 0, s, logits, vocab, pv, pi);
  hipLaunchKernelGGL(k_row_argmax2, dim3(rows), dim3(64), 0, s, pv, pi, out);
  return hipGetLastError();
}
}  // namespace chonk

namespace chonk {
int bd_attn_segments(int rows, int kv_heads, int max_pages) {
  // enough (kv head, row, segment) workgroups to cover the device; with one
  // segment the walk writes the output (and may do the rotary/K-V write)
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return std::max(1, std::min(max_pages, (2 * cus + rows * kv_heads - 1) / std::max(1, rows * kv_heads)));
}

hipError_t launch_bd_attn(const PfAttnArgs& a0, int rows, float* part, int64_t part_cap, hipStream_t s, bool* planes,
                          const PfRopeArgs* rope) {
  PfAttnArgs a = a0;
  a.rows = rows;
  const int G = a.heads / a.kv_heads;
  const int mp = a.kv.max_pages;
  const int nseg = bd_attn_segments(rows, a.kv_heads, mp);
  if (nseg <= 0 || (rope && nseg != 1)) return hipErrorInvalidValue;
  PfRopeArgs ra{};
  if (rope) ra = *rope;
  if (rope && (!ra.pq.p || !ra.pk.p || !ra.pv.p)) return hipErrorInvalidValue;  // the partial sums are read
  if (!a.kv16 || !a.kv.pages || !a.kv.row_seq || !a.kv.row_pos || G > 8 || G * a.hd > 1536 || mp > 64 ||
      (nseg > 1 && (int64_t)rows * a.kv_heads * mp * attn_rowf(G, a.hd) > part_cap))
    return hipErrorInvalidValue;
  if (nseg > 1) a.oh = nullptr;  // the merge writes a.out
  if (a.oh && (!a.ol || !a.oscale || a.okpad < a.heads * a.hd)) return hipErrorInvalidValue;
  *planes = a.oh != nullptr;
  const dim3 g1(a.kv_heads, rows, nseg), g2(a.kv_heads, rows);
#define CHONK_BD_CASE(HH)                                                                     \
  case HH:                                                                                    \
    if (rope)                                                                                 \
      hipLaunchKernelGGL((k_bd_walk<HH, true>), g1, dim3(kWg), 0, s, a, part, mp, nseg, ra);  \
    else                                                                                      \
      hipLaunchKernelGGL((k_bd_walk<HH, false>), g1, dim3(kWg), 0, s, a, part, mp, nseg, ra); \
    if (nseg > 1) hipLaunchKernelGGL(k_bd_merge<HH>, g2, dim3(kWg), 0, s, a, part, mp, nseg); \
    return hipGetLastError();
  switch (a.hd) {
    CHONK_BD_CASE(64)
    CHONK_BD_CASE(128)
    CHONK_BD_CASE(256)
    default: return hipErrorInvalidValue;
  }
#undef CHONK_BD_CASE
}
}  // namespace chonk

