// Batched (many-token) kernels: operand split, dequant-fused MFMA GEMM and the
// per-token glue of a prompt processed as T rows at once (prefill.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"

namespace chonk {

enum GemmEpi : int32_t { GEMM_STORE = 0, GEMM_ADD = 1 };

// y[t][n] (=|+=) 2^-ws * xscale[t] * sum_k (xh + xl)[t][k] * (W 2^ws)[n][k]
struct GemmArgs {
  QMat w;                 // striped weights, N = w.n rows of K = w.k
  // a fused launch over up to three matrices of one type and K (e.g. q | k | v):
  // output rows [0, n1) come from w, [n1, n2) from w2, [n2, n_all) from w3; the
  // segment starts are multiples of the 64-row tile. n_all = 0: w alone.
  QMat w2, w3;
  int32_t n1, n2, n_all, pad0;
  const _Float16* xh;     // [t][kpad] activation planes, zero past K
  const _Float16* xl;
  const float* xscale;    // [t]
  float* y;               // [t][ldy]
  int32_t ldy, t, kpad, epi;
  int32_t ws;             // weight exponent
  int32_t ksplit;         // K partitions (grid z); > 1 needs `part`
  float* part;            // [ksplit][t][w.n] partial sums, reduced in order by the launcher
  int64_t part_cap;       // floats available in part
  int32_t defer;          // 1: always leave partials in part (launch_gemm_deferred)
};

// Where a row batch's K/V live: the engine's contiguous cache
// ([kv_heads][ctx][hd] per layer, pages == null), or pages of 64 positions
// ([page][kv_heads][64][hd]) through a per-sequence page table.
struct KvAddr {
  void *kc, *vc;
  int32_t ctx;
  const int32_t* pages;   // [seq][max_pages] physical page ids, or null
  int32_t max_pages;
  int32_t seq0;           // sequence of every row when row_seq is null
  const int32_t* row_seq; // [rows] per-row sequence, or null
  const int32_t* row_pos; // [rows] per-row position, or null (p0 + row)
  int32_t p0;
};
constexpr int kKvPage = 64;

// A GEMM result left as K-split partial sums: value(t, j) = sum over z < ks
// of p[z * zs + t * n + j], added in z order (the consumer kernel adds them).
struct PartSum {
  const float* p;         // null: absent
  int32_t n, ks;          // valid columns, K splits
  int64_t zs;             // floats between splits
  int32_t ld, pad0;       // floats between rows (>= n: a column range of a fused result)
};

struct PfSplitArgs {
  const float* x;         // [rows][ldx]
  int32_t ldx, k, kpad;
  const float* w;         // RMSNorm weight [k], or null for a plain split
  float eps;
  _Float16 *xh, *xl;      // [rows][kpad]
  float* xscale;          // [rows]
  // residual update first (x must then be writable): x += add, or with
  // add_w (the Gemma-3 sandwich) x = clamp(x + RMSNorm(add) * add_w, +-65000)
  PartSum add;
  const float* add_w;
};

struct PfGluArgs {
  PartSum pg, pu;         // gate and up rows [rows][k] (deferred GEMM results)
  float* act;             // [rows][k]
  int32_t k, kpad, gelu;
  _Float16 *xh, *xl;
  float* xscale;
};

struct PfRopeArgs {
  float* qkv;             // [rows][ld]: q | k | v (gathered from pq, pk, pv when given)
  PartSum pq, pk, pv;
  int32_t ld, hd, heads, kv_heads, interleaved, kv16;
  const float *qn_w, *kn_w;  // per-head RMSNorm weights (null: none)
  float eps;
  const float* rope_inv;  // [hd/2]
  KvAddr kv;
};

struct PfAttnArgs {
  const float* qkv;       // rotated q rows
  int32_t ld;
  float* out;             // [rows][ldo]
  int32_t ldo, heads, kv_heads, hd, window, kv16;
  int32_t rows;           // rows of the pass (set by the launcher)
  float scale;
  KvAddr kv;
  // batched decode: the next GEMM's operand planes [rows][okpad] (hi, lo) and
  // row scales, written instead of `out` when set and the rows are not split
  // into segments (the output of attention needs no scaling: |x| <= max |V|)
  _Float16* oh;
  _Float16* ol;
  float* oscale;
  int32_t okpad;
};

// K padded for the GEMM's activation planes.
constexpr int gemm_kpad(int k) { return (k + 127) / 128 * 128; }

size_t gemm_shared_bytes();
hipError_t init_gemm_attributes();
// Picks the K split for a launch (at least ~256 workgroups when the partial
// buffer allows) and launches the GEMM and, when split, the ordered reduction.
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// The GEMM with its result left as partial sums in `region` (capacity in
// floats): the K split is chosen as in launch_gemm within the region, and no
// reduction is launched; *out describes the partials for the consumer.
hipError_t launch_gemm_deferred(const GemmArgs& a, float* region, int64_t region_cap, PartSum* out, hipStream_t s);
hipError_t launch_pf_split(const PfSplitArgs& a, int rows, hipStream_t s);
hipError_t launch_pf_embed(const QMat& embed, const int32_t* tok, float scale, int k, float* x, int rows,
                           hipStream_t s);
hipError_t launch_pf_norm_add(const float* d, const float* w, float eps, int k, float* x, int rows, hipStream_t s);
hipError_t launch_pf_glu_split(const PfGluArgs& a, int rows, hipStream_t s);
hipError_t launch_pf_rope_kv(const PfRopeArgs& a, int rows, hipStream_t s);
hipError_t launch_pf_attn(const PfAttnArgs& a, int rows, hipStream_t s);
// Decode attention of rows with their own sequences (kv.row_seq) over paged
// K/V: per-page partials in `part`, then a merge per (row, kv head).
// Segments per row of the batched decode attention (1: one workgroup walks all
// of a (row, kv head)'s pages; 0: no device).
int bd_attn_segments(int rows, int kv_heads, int max_pages);
// *planes: whether the launch wrote a.oh / a.ol / a.oscale (else a.out). With
// `rope` (only when bd_attn_segments is 1) the attention also does that
// launch's rotary/K-V write, reading q, k and v from the projections.
hipError_t launch_bd_attn(const PfAttnArgs& a, int rows, float* part, int64_t part_cap, hipStream_t s, bool* planes,
                          const PfRopeArgs* rope);
// Greedy id per row of logits [rows][vocab] (the reference's argmax ordering);
// scratch holds 64 floats per row.
hipError_t launch_row_argmax(const float* logits, int vocab, int rows, float* scratch, int32_t* out, hipStream_t s);

}  // namespace chonk
