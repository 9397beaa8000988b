// Kernel argument blocks and launchers of the decode step.
//
// One decode step of an L-layer model is 5L + 2 launches:
//   per layer  qkv      RMSNorm (or embedding gather / residual re-norm) fused
//                       into the q|k|v dequant-matvec
//              attn     qk-norm + RoPE + K/V store + split-K GQA attention with
//                       an in-kernel last-arriver combine
//              oproj    o-projection (+ residual add)
//              gateup   RMSNorm + gate|up matvec + SiLU/GELU-tanh product
//              down     down projection (+ residual add)
//   final      lmhead   final RMSNorm + lm_head matvec + per-256-id group
//                       argmax with the repetition penalty (ARGMAX_STAGE1)
//              select   global argmax (ARGMAX_STAGE2) or the candidate
//                       sampler, token bookkeeping, position advance
#pragma once

#include "device_common.h"

namespace chonk {

enum ProMode : int32_t {
  PRO_PLAIN = 0,         // xs = in
  PRO_NORM = 1,          // xs = rmsnorm(in) * w_norm
  PRO_EMBED_NORM = 2,    // r = embed(hist[pos]) * scale; WG0 writes r; xs = rmsnorm(r) * w_norm
  PRO_RES_NORM = 3,      // r = clamp(in + rmsnorm(delta) * w_delta, +-65000); WG0 writes r; xs = rmsnorm(r) * w_norm
  PRO_GATE = 4,          // v = in * silu(gate_z); xs = rmsnorm(v) * w_norm (granitehybrid Mamba2 gated norm)
  PRO_LN = 5,            // xs = layernorm(in) * w_norm + norm_b (GPT-2)
  PRO_EMBED_LN = 6,      // r = embed(hist[pos]) + pos_embd[pos]; WG0 writes r; xs = layernorm(r) * w_norm + norm_b
  PRO_CONV = 7,          // xs = C * (s1 * w0 + s2 * w1 + (B * x) * w2), B | C | x = conv_proj (lfm2)
};

enum EpiMode : int32_t {
  EPI_STORE = 0,    // out[n] = acc
  EPI_ADD = 1,      // out[n] = add[n] + acc
  EPI_GLU_SILU = 2, // out[n] = silu(gate_n) * up_n
  EPI_GLU_GELU = 3, // out[n] = gelu_tanh(gate_n) * up_n
  EPI_LOGITS = 4,   // logits[n] = acc; group candidate per 256 rows (lfm2: per residue class mod 256)
  EPI_GELU = 5,     // out[n] = gelu_tanh(acc + bias[n]) (GPT-2 MLP up projection)
  EPI_TAG = 6,      // ((uint64_t*)out)[n] = {acc, tag_epoch[n / tag_div]}: q|k|v rows of the fused attention launch
};

struct MvSeg {
  QMat w;            // matrix (GLU: gate)
  QMat w2;           // GLU: up
  float* out;
  const float* add;  // EPI_ADD residual input
  const float* bias; // added to each row's sum first when set (GPT-2 linear biases)
  int32_t n_out;     // output rows
  int32_t tile;      // output rows per workgroup
  int32_t lpr;       // lanes per row (power of two, <= 64)
  int32_t wg_begin;  // first workgroup of this segment
  int32_t tag_div;   // EPI_TAG: rows per kv head (the row's tag is tag_epoch[row / tag_div])
};

struct MvArgs {
  MvSeg seg[3];
  int32_t nseg;
  int32_t pro;
  int32_t epi;
  int32_t k;              // activation length
  const float* in;
  const float* delta;
  const float* w_delta;
  const float* w_norm;
  float* res_out;
  QMat embed;
  float embed_scale;
  float eps;
  const int32_t* hist;
  int32_t vocab;
  int32_t advance_pos;    // WG0 advances st->pos when done (steps without logits)
  int32_t row_kernel;     // 1: one output row per lane group (k_mvr_*, planned by plan_seg_row)
  const float* norm_b;    // PRO_LN / PRO_EMBED_LN: LayerNorm bias
  const float* pos_embd;  // PRO_EMBED_LN: learned position table [context][k]
  int32_t sanitize;       // EPI_ADD: NaN -> 0, clamp to +-10000 (GPT-2 residual)
  int32_t gpt_argmax;     // EPI_LOGITS: the GPT-2 runtime's group argmax (strict >, left slot kept)
  const uint32_t* pen_bits;
  const DevSampling* samp;
  Candidate* cand;
  DevState* st;
  // lfm2 short convolution: the PRO_CONV prologue reads the state, a later
  // launch of the same layer (conv_commit) shifts it once every reader is done
  const float* conv_proj;  // [3 * conv_n] this token's in_proj rows B | C | x
  const float* conv_w;     // [conv_n][3] depthwise taps
  float* conv_s1;          // [conv_n] B * x two positions back
  float* conv_s2;          // [conv_n] B * x one position back
  int32_t conv_n;          // channels (the hidden size)
  int32_t conv_commit;     // WG0 sets s1 = s2, s2 = B * x
  int32_t lfm_classes;     // EPI_LOGITS: rows stored class-major, workgroup c computes ids c, c + 256, ...
  int32_t lm_lanes;        // EPI_LOGITS: seg[0].w is the lane-interleaved copy (k_lm_lanes, 256 ids per workgroup)
  const float* gate_z;     // PRO_GATE: the gate z (the first k rows of the Mamba2 in_proj output)
  float add_scale;         // EPI_ADD: out = add + acc * add_scale when non-zero (granitehybrid's 0.246)
  float logit_scale;       // EPI_LOGITS: logits = acc * logit_scale when non-zero (granitehybrid's 1/3)
  const uint32_t* tag_epoch;  // EPI_TAG: the attention's per-kv-head epochs
};

// One Mamba2 step of a granitehybrid layer (granite-wgsl-runtime.ts:1476-1562):
// the causal 4-tap convolution + silu of the xBC channels and the selective
// scan of every (head, channel) over its 128 states. Workgroup (n, y) owns head
// n's channels 8y .. 8y+7; every workgroup evaluates the convolution of the
// shared B and C channels itself.
struct SsmArgs {
  const float* proj;       // [inner + conv + heads] in_proj output: z | xBC | dt
  const float* conv_w;     // [conv][4] taps
  const float* conv_b;     // [conv]
  float* conv_state;       // [2][conv][3]: each channel's last three inputs, the buffer chosen by position parity
  const float* dt_bias;    // [heads]
  const float* a_neg;      // [heads] A = -exp(A_log)
  const float* d;          // [heads]
  float* ssm_state;        // [heads][32][128]
  float* y;                // [inner] scan output
  DevState* st;
  int32_t inner, conv, heads;
};

struct AttnArgs {
  const float* qkv;       // q[heads*hd] | k[kv*hd] | v[kv*hd]
  const float* qn_w;      // per-head q RMSNorm weight (null: none)
  const float* kn_w;
  const float* rope_inv;  // [hd/2] theta^(-2d/hd), f32
  void* kc;               // [kv_heads][C][hd], half or float
  void* vc;
  float* part;            // [kv_heads][nchunk] rows of G*(hd+2) floats padded to 4, uncached memory
  uint32_t* cnt;          // [kv_heads], uncached memory: k_attention's arrival counters (zero
                          // between launches), k_attn_dec's per-head epochs
  uint64_t* tpart;        // k_attn_dec: [kv_heads][nchunk] rows of tagged words
  const uint64_t* qkv_tag;  // fused q|k|v + attention launch: q | k | v as tagged words (qkv unused)
  const float2* rope_cs;  // k_attn_dec: [ctx][hd/2] (cos, sin) of the rotary angles
  float* out;             // [heads*hd]
  DevState* st;
  int32_t heads, kv_heads, hd, ctx, window, chunk, nchunk;
  uint32_t theta;         // Math.round(ropeTheta)
  int32_t interleaved, kv_f16;
  int32_t merge_floats;   // LDS floats available for staging chunk partials
  int32_t spec_kv;        // request the chunk's K/V before the position is known
  int32_t sub;            // k_attn_dec: 64-position sub-chunks walked by one workgroup
  int32_t tpp;            // threads per position in the score phase (power of two)
  int32_t variant;        // 0: k_attention; 1: k_attn_dec (fp16 cache, 64-position chunks)
  int32_t kv_delay;       // fused q|k|v + attention launch: 10 ns ticks before the K/V requests
  float eps, scale;
};

// Floats (or tagged words) per attention chunk partial: per head [max, sum,
// acc[hd]], padded to a 16-byte multiple.
__host__ __device__ constexpr int attn_rowf(int G, int hd) { return (G * (hd + 2) + 3) & ~3; }

struct SelArgs {
  const Candidate* cand;
  int32_t gpt_argmax;     // greedy stage 2 with the GPT-2 runtime's tree (strict >, left slot kept)
  int32_t groups;
  int32_t vocab;
  int32_t ctx;
  const DevSampling* samp;
  uint32_t* pen_bits;
  uint32_t* seen_bits;
  int32_t* hist;          // [ctx + 1]
  int32_t* gen;           // [ctx + 1]
  DevState* st;
};

// Words {f32 value, u32 epoch} written and read with agent-scope atomics: a
// consumer in another workgroup waits for a value by polling the word itself
// until it carries the launch's epoch (no counters, no cache maintenance).
typedef uint64_t tagged_t;

// Launch parameter helpers -------------------------------------------------------
size_t mv_shared_bytes(int k, int max_tile_rows);
size_t attn_shared_bytes(int group, int hd, int chunk, int nchunk, int kv_elem);
int attn_merge_floats(int group, int hd, int nchunk);
// Largest chunk (positions per attention workgroup) the kernel supports for hd.
int attn_max_chunk(int hd);
int attn_threads_per_position(int hd, int chunk, int kv_elem);
int pick_lpr(int units);

// Raises the dynamic LDS limit of the kernels; call once per device before launching.
hipError_t init_kernel_attributes();
// Dynamic LDS bytes a launch may request after init_kernel_attributes().
size_t lds_limit();
// Units of 32 weights a lane of the one-row-per-lane-group matvec handles at most.
constexpr int kRowUnits = 4;
hipError_t launch_matvec(const MvArgs& a, int grid, size_t shmem, hipStream_t s);
hipError_t launch_attention(const AttnArgs& a, size_t shmem, hipStream_t s);
hipError_t launch_ssm(const SsmArgs& a, hipStream_t s);
// The register-resident decode attention (attn_decode.hip): fp16 cache,
// head_dim 64/128/256, GQA group <= 8 (group x head_dim <= 1536), at most 128
// chunks of attn_dec_chunk() positions over the context.
bool attn_dec_supported(int group, int hd, int ctx, int kv_f16);
int attn_dec_chunk();
// 64-position sub-chunks per k_attn_dec workgroup at a context, with at most
// min(128, per_head) workgroups per kv head.
int attn_dec_sub(int ctx, int per_head);
size_t attn_dec_shared_bytes(int group, int hd, int nchunk);
// Workgroups of k_attn_dec that fit on the device at once (its active chunks
// wait for each other, so the whole grid must be resident); 0 for an instance
// that spills registers to scratch, which the engine then does not use.
int attn_dec_resident(int device, int group, int hd, size_t shmem, bool walk);
hipError_t launch_attn_dec(const AttnArgs& a, size_t shmem, hipStream_t s);
// The fused q|k|v matvec + decode attention launch (k_qkv_attn): the matvec's
// nq workgroups (m planned for the row kernel, EPI_TAG, PRO_NORM) ahead of the
// attention's kv_heads * nchunk. Resident workgroups of the instance for
// (group, hd) at `shmem` bytes of LDS on the device (0: no such instance).
int qkv_attn_resident(int device, int group, int hd, size_t shmem);
hipError_t launch_qkv_attn(const MvArgs& m, int nq, const AttnArgs& a, size_t shmem, hipStream_t s);
// cs[p][d] = (cos, sin)(p * inv[d]) for p < ctx, d < half.
hipError_t launch_rope_cs(const float* inv, int half, int ctx, float2* cs, hipStream_t s);
hipError_t launch_select(const SelArgs& a, hipStream_t s);

// Test / utility kernels
hipError_t launch_dequant(const QMat& w, float* out, hipStream_t s);
hipError_t launch_fill_kv(void* kc, void* vc, int kv_heads, int ctx, int hd, int pos, int kv_f16, uint64_t seed,
                          hipStream_t s);

}  // namespace chonk
