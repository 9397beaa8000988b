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
  int32_t pad_lfm;
  const float* gate_z;     // PRO_GATE: the gate z (the first k rows of the Mamba2 in_proj output)
  float add_scale;         // EPI_ADD: out = add + acc * add_scale when non-zero (granitehybrid's 0.246)
  float logit_scale;       // EPI_LOGITS: logits = acc * logit_scale when non-zero (granitehybrid's 1/3)
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

// Persistent decode step --------------------------------------------------------
//
// The whole token (every layer, lm_head, selection) as one launch of one
// workgroup per CU. Phases follow each other in the order of the step; a
// workgroup walks its tasks of every phase (task t of a phase runs on
// workgroup (t + rot) mod grid). Activations crossing workgroups are "tagged":
// 8-byte words {f32 value, u32 step epoch} written and read with agent-scope
// atomics, so a consumer waits for its inputs by polling the words themselves
// (no counters, no cache maintenance), with a bounded wait that aborts the step
// (DevState.error = 3) instead of hanging.
typedef uint64_t tagged_t;

enum PhaseKind : int32_t { PH_MV = 0, PH_ATTN = 1 };

struct StepPhase {
  int32_t kind;
  int32_t n_tasks;
  int32_t rot;
  int32_t nseg;
  // PH_MV: up to three matrices sharing the input (q | k | v); seg[i].wg_begin
  // is the segment's first task, seg[i].tile its rows per task.
  MvSeg seg[3];
  int32_t pro, epi, k, pad0;
  const tagged_t* in;      // input [k] (PRO_PLAIN, PRO_NORM, PRO_RES_NORM)
  const tagged_t* delta;   // PRO_RES_NORM: branch output to normalise and add
  const float* w_norm;
  const float* w_delta;
  tagged_t* res_out;       // PRO_EMBED_NORM / PRO_RES_NORM: residual [k], written in task slices
  const tagged_t* add;     // EPI_ADD: residual input [n_out]
  tagged_t* tout[3];       // per-segment tagged outputs (EPI_STORE / EPI_ADD / EPI_GLU_*)
  float* logits;           // EPI_LOGITS: plain logits [vocab]
  // PH_ATTN: one task per (kv head, chunk); q|k|v come from qkv_in. Every
  // chunk but the newest stores its partial in tpart ([kv][nchunk] rows of
  // attn_rowf words); the newest chunk's task merges them into attn_out.
  AttnArgs at;
  const tagged_t* qkv_in;
  tagged_t* attn_out;
  tagged_t* tpart;
};

// Record of the first wait that exceeded its time bound (diagnostics).
struct StepDebug {
  uint32_t claimed;        // set by the first workgroup that aborts
  int32_t wg, phase, task, index;
  uint32_t seen, want;     // tag found at `index` / tag expected
  int32_t pos;
  uint64_t abort_time;     // wall clock (100 MHz ticks)
  uint64_t start[1024];    // per-workgroup start time of the last step
};

// Wall-clock stamps per persistent-step task when tracing: matvec: start,
// input arrived, prologue done, input quantized, dot products done, next slot
// requested, epilogue stored, end; attention: start, input arrived, K rows
// loaded, chunk done, next slot requested, partial stored or heads merged,
// next slot requested (merging chunk), end.
constexpr int kStepStamps = 8;

// One task of a workgroup's list in the persistent step, resolved on the host
// from the phase table: a matvec task carries its rows, the slot layout of
// its weight rows and norm weights, the direct-to-LDS copies that fill that
// slot and the addresses of its tagged inputs and outputs, so the device
// reads one record per task instead of walking the phase's segments.
enum StepTaskKind : int32_t {
  STASK_MV = 0,    // matvec task whose rows and norm weights are in the slot
  STASK_ATTN = 1,  // attention task (kv head, chunk) = (t / nchunk, t % nchunk)
  STASK_LM = 2,    // lm_head task: rows streamed from memory, group argmax
};
struct StepDma {
  const uint8_t* src;
  int32_t dst, n16;  // slot offset, 16-byte units
};
constexpr int kStepMaxDma = 10;  // two norm weights + two matrices of up to four streams
struct alignas(16) StepTask {
  int32_t phase;         // index in the phase table; >= n_phases ends the list
  int32_t t;             // task index within the phase
  int32_t kind;          // StepTaskKind
  int32_t type, uc, k, lpr;
  int32_t t0, nt, glu;   // rows [t0, t0 + nt) of the segment
  int32_t pro, epi;
  int32_t res_lo, res_hi;  // residual slice stored by this task (PRO_EMBED_NORM / PRO_RES_NORM)
  int32_t n_dma;
  int32_t wn, wd;        // slot offsets of the norm weights (-1: none)
  int32_t data[2][4];    // slot offset of row t0 of each (matrix, stream) (-1: none)
  int32_t pad[3];
  const tagged_t* in;    // [k] unless PRO_EMBED_NORM
  const tagged_t* delta; // [k] for PRO_RES_NORM
  const tagged_t* add;   // EPI_ADD: residual words of rows [t0, t0 + nt)
  tagged_t* out;         // output words of rows [t0, t0 + nt)
  tagged_t* res_out;     // residual words [k] (the task stores [res_lo, res_hi))
  StepDma dma[kStepMaxDma];
  int32_t pad2[2];
};
static_assert(sizeof(StepTask) == 320, "StepTask is copied in 16-byte units");
constexpr int kStepDescRing = 8;  // task records a workgroup keeps in LDS (prefetched ahead)

struct StepArgs {
  const StepPhase* phases;
  const StepTask* tasks;   // [grid][task_stride]: each workgroup's tasks in order, then end records
  int32_t task_stride;
  int32_t n_phases;
  int32_t logits;          // 1: the step ends with token selection
  DevState* st;
  uint32_t* epoch;         // step epoch (tags); advanced by the last workgroup
  uint32_t* done;          // workgroups finished; reset by the last one
  QMat embed;
  float embed_scale;
  float eps;
  int32_t vocab;
  int32_t pad0;
  const int32_t* hist;
  const DevSampling* samp;
  const uint32_t* pen_bits;
  Candidate* cand;
  SelArgs sel;
  StepDebug* dbg;
  uint64_t* trace;         // optional wall-clock stamps: [n_phases + 1][grid] phase ends, then start;
                           // then [n_phases][grid][kStepStamps] per task (see k_step)
};

// Each task of the persistent step finds the inputs that do not depend on the
// previous phases (norm weights, its weight rows, its K/V chunk) in an LDS
// slot filled by direct-to-LDS loads issued during the workgroup's previous
// task; two slots of kStepSlotBytes alternate.
constexpr int kStepSlotBytes = 36 * 1024;

// Bytes per row of stream s of a [N][K] matrix of `type` in the striped layout
// (device_common.h); 0 for a stream the type does not use.
__host__ __device__ constexpr int stripe_row_bytes(int type, int k, int s) {
  switch (type) {
    case QT_Q4_K: return s == 0 ? k / 2 : s == 1 ? k / 16 : 0;
    case QT_Q5_K: return s == 0 ? k / 2 : s == 1 ? k / 16 : s == 2 ? k / 8 : 0;
    case QT_Q6_K: return s == 0 ? k / 2 : s == 1 ? k / 4 : s == 2 ? k / 16 : k / 128;
    case QT_Q8_0: return s == 0 ? k : s == 1 ? k / 16 : 0;
    case QT_Q5_0: return s == 0 ? k / 2 : s == 1 ? k / 8 : s == 2 ? k / 16 : 0;
    case QT_Q5_1: return s == 0 ? k / 2 : s == 1 ? k / 8 : k / 16;
  }
  return 0;
}

// Slot layout of a matvec task over rows [t0, t0 + nt) of a K-column matrix
// (two matrices for GLU): the norm weights (K floats each) first, then each
// stream's row range as a 16-byte-aligned copy. data[m][s] is the slot offset
// of row t0's first byte of stream s of matrix m; returns the slot bytes used.
struct MvSlot {
  int wn, wd;        // norm weight / residual-norm weight offsets (-1: none)
  int data[2][4];    // per matrix and stream: offset of row t0 (-1: none)
  int dst[2][4];     // slot offset of the copy (16-aligned)
  int src0[2][4];    // first byte (16-aligned) of the copied range within the stream
  int n16[2][4];     // 16-byte units copied
};
__host__ __device__ inline int mv_slot_layout(int type, int k, int t0, int nt, int nmat, int n_norms, MvSlot* m) {
  int off = 0;
  m->wn = n_norms > 0 ? off : -1;
  off += n_norms > 0 ? 4 * k : 0;
  m->wd = n_norms > 1 ? off : -1;
  off += n_norms > 1 ? 4 * k : 0;
  for (int j = 0; j < 2; ++j)
    for (int s = 0; s < 4; ++s) {
      const int rb = stripe_row_bytes(type, k, s);
      if (j >= nmat || rb == 0 || nt <= 0) {
        m->data[j][s] = -1;
        m->dst[j][s] = 0;
        m->src0[j][s] = 0;
        m->n16[j][s] = 0;
        continue;
      }
      const int b0 = t0 * rb, b1 = (t0 + nt) * rb;
      const int a0 = b0 & ~15, a1 = (b1 + 15) & ~15;
      m->src0[j][s] = a0;
      m->n16[j][s] = (a1 - a0) / 16;
      m->dst[j][s] = off;
      m->data[j][s] = off + (b0 - a0);
      off += a1 - a0;
    }
  return off;
}

// Slot layout of an attention task: rotary inverse frequencies [hd/2], q / k
// norm weights [hd] each, then K and V rows of the chunk indexed by chunk
// position (only the positions the task reads are copied).
struct AttnSlot {
  int inv, qn, kn, k, v;
};
__host__ __device__ inline int attn_slot_layout(int hd, int chunk, int kv_elem, AttnSlot* s) {
  s->inv = 0;
  s->qn = (hd / 2 * 4 + 15) & ~15;
  s->kn = s->qn + hd * 4;
  s->k = s->kn + hd * 4;
  s->v = s->k + chunk * hd * kv_elem;
  return s->v + chunk * hd * kv_elem;
}

// Dynamic LDS bytes of the persistent step for this model.
size_t step_shared_bytes(int max_k, int max_tile_rows, int group, int hd, int chunk, int nchunk, int kv_elem);
// Whether the persistent step is compiled for this GQA group / K/V type.
bool step_supported(int group, bool kv_f16);
// Workgroups of the persistent step resident per CU with `shmem` bytes of LDS (0: cannot run).
int step_occupancy(int group, bool kv_f16, size_t shmem);
// `a` and `phases` point to device memory holding the step's arguments and phase table.
hipError_t launch_step(const StepArgs* a, const StepPhase* phases, int group, bool kv_f16, int grid, size_t shmem,
                       hipStream_t s);

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
// wait for each other, so the whole grid must be resident).
int attn_dec_resident(int device, int group, int hd, size_t shmem, bool walk);
hipError_t launch_attn_dec(const AttnArgs& a, size_t shmem, hipStream_t s);
// cs[p][d] = (cos, sin)(p * inv[d]) for p < ctx, d < half.
hipError_t launch_rope_cs(const float* inv, int half, int ctx, float2* cs, hipStream_t s);
hipError_t launch_select(const SelArgs& a, hipStream_t s);

// Test / utility kernels
hipError_t launch_dequant(const QMat& w, float* out, hipStream_t s);
hipError_t launch_fill_kv(void* kc, void* vc, int kv_heads, int ctx, int hd, int pos, int kv_f16, uint64_t seed,
                          hipStream_t s);

}  // namespace chonk
