/*
 * ORACLE — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of the reference's llama-webgpu decode path
 * (src/lib/llama-wgsl-runtime.ts, src/lib/gguf.ts, src/lib/sampling.ts),
 * following the WGSL kernels' fp32 arithmetic and reduction orders. It is the
 * checker for the HIP path and the CPU baseline in bench.py; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (chonklm_amd) never links or calls it.
 *
 * Everything here is compiled with -ffp-contract=off so that a*b+c is two
 * roundings, as in the WGSL source.
 *
 * Parity pins (see tests/): block decode vs hand-built known-answer blocks and
 * an independent numpy decode; matvec vs float64 dot products; the whole
 * forward pass vs an independent float64 numpy decoder on tiny models;
 * argmax/sampling vs closed-form cases. The exact ulps of the WGSL built-ins
 * pow/sin/cos/exp/inverseSqrt/tanh are implementation-defined in the
 * reference and are "parity unpinned" beyond float64 closed forms.
 */
#ifndef CHONK_ORACLE_H
#define CHONK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element-wise block decode of n elements (row-major, n a multiple of the
 * block size) of GGML type `type` (6 Q5_0, 7 Q5_1, 8 Q8_0, 12 Q4_K, 13 Q5_K,
 * 14 Q6_K, 0 F32, 1 F16). Returns 0 on success. */
int orc_dequant(uint32_t type, const uint8_t* blocks, int64_t n, float* out);

/* The same decode row by row, as the oracle's matvec takes it (block scales
 * decoded once per block); equal to orc_dequant element for element. */
int orc_decode_rows(uint32_t type, const uint8_t* blocks, int64_t n_rows, int64_t row_len, float* out);

/* y[N] = W[N,K] x[K] in the WGSL order: 128 strided partial sums then a
 * stride 64..1 tree (llama-wgsl-runtime.ts:2412-2442). */
int orc_matvec(uint32_t type, const uint8_t* blocks, int64_t n_rows, int64_t row_len, const float* x,
               float* y, int n_threads);

/* Model ---------------------------------------------------------------- */
typedef struct orc_model orc_model;

typedef struct {
  int32_t vocab;        /* ModelDef.vocab */
  int32_t layers;       /* ModelDef.layers (alias construction only) */
  int32_t max_context;  /* ModelDef.maxContext */
  int32_t kv_f16;       /* 1: round K/V to binary16 on store (fp16 KV cache) */
  int32_t n_threads;
} orc_model_def;

typedef struct {
  double temperature;
  double top_p;
  int32_t top_k;
  double repetition_penalty;
} orc_sampling;

orc_model* orc_model_load(const char* gguf_path, const orc_model_def* def, char* err, size_t err_len);
void orc_model_free(orc_model* m);
int orc_model_context(const orc_model* m);
/* 1 for a GGUF of architecture gpt2 (gpt-wgsl-runtime.ts), else 0. */
int orc_model_is_gpt(const orc_model* m);
/* 1 for a GGUF of architecture lfm2 (lfm-wgsl-runtime.ts), else 0. */
int orc_model_is_lfm(const orc_model* m);
/* 1 when the model is a granitehybrid (Granite-4.0-H) decoder. */
int orc_model_is_granite(const orc_model* m);
/* Vocabulary of the loaded model (ModelDef.vocab, or token_embd's rows for gpt2). */
int orc_model_vocab(const orc_model* m);
int orc_model_position(const orc_model* m);
void orc_model_reset(orc_model* m);

/* runToken (llama-wgsl-runtime.ts:1025-1150; for gpt2 GptWgslEngine.runToken,
 * gpt-wgsl-runtime.ts:749-840; for lfm2 LfmWgslEngine.runToken,
 * lfm-wgsl-runtime.ts:727-809, which takes no penalty list). `uniform` is the sampler's
 * U in [0,1) (replaces Math.random). Returns 0, or -1 with err filled. */
int orc_model_run_token(orc_model* m, int32_t token, int32_t need_logits, const orc_sampling* s,
                        const int32_t* penalized, int64_t n_penalized, const int32_t* seen, int64_t n_seen,
                        double uniform, int32_t* out_token, char* err, size_t err_len);

/* Buffers of the last step. which: 0 logits[vocab], 1 residual[hidden]
 * (final hidden before the last norm), 2 final normed hidden[hidden],
 * 3 candidates (vocab/256 x {value f32, index u32}, 256 for lfm2) as raw 8-byte pairs,
 * 4 q after rope (last layer) [heads*hd], 5 attention output (last layer). */
int orc_model_read(const orc_model* m, int which, void* out, int64_t n_bytes);

/* Per-layer K/V cache rows at position t (float values after the optional
 * fp16 rounding): out[kv_heads*hd]. */
int orc_model_read_kv(const orc_model* m, int layer, int is_value, int pos, float* out);

/* Fills the K/V cache for positions [0, pos) with seeded values and sets the
 * position, so decode steps at long context can be timed without a prefill. */
int orc_model_fake_context(orc_model* m, int pos, uint64_t seed);

/* ARGMAX_STAGE1/2 over a logits vector: candidate pairs (optional, 8 bytes
 * per 256-id group) and the greedy token. */
int orc_argmax(const float* logits, int64_t vocab, const int32_t* penalized, int64_t n_penalized,
               double repetition_penalty, uint8_t* candidate_pairs, int32_t* token);

/* The GPT-2 runtime's ARGMAX_STAGE1/2 (strict-greater trees, padding index
 * 0, penalty whenever it is not 1; at most 65536 ids). */
int orc_argmax_gpt(const float* logits, int64_t vocab, const int32_t* penalized, int64_t n_penalized,
                   double repetition_penalty, uint8_t* candidate_pairs, int32_t* token);

/* The LFM runtime's selection over a logits vector: TOPK256_WGSL's 256
 * candidates (slot t: the first strictly greatest of ids t, t + 256, ...,
 * starting from (-3.402823e38, 0)) and ARGMAX_WGSL's token (a strict-greater
 * tree over those slots), lfm-wgsl-runtime.ts:1880-1947. */
int orc_lfm_select(const float* logits, int64_t vocab, uint8_t* candidate_pairs, int32_t* token);

/* sampleFromCandidateBuffer (sampling.ts:23-76) with Math.random() -> uniform. */
int32_t orc_sample_candidates(const uint8_t* candidate_pairs, int64_t n_groups, const orc_sampling* s,
                              const int32_t* seen, int64_t n_seen, double uniform);

/* Counter-based U[0,1): (splitmix64(seed + 0x9e37..*(step+1)) >> 11) * 2^-53. */
double orc_uniform(uint64_t seed, uint64_t step);

#ifdef __cplusplus
}
#endif

#endif
