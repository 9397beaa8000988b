/*
 * chonk.h — C ABI of the MI355X decode engine (libchonk.so).
 *
 * This is the drop-in boundary for the reference's llama-webgpu runtime. Each
 * entry point names the reference interface it replaces
 * (paths relative to the reference repository):
 *
 *   chonk_engine_create            loadLlamaWgslModel + LlamaWgslEngine.create
 *                                  (src/lib/llama-wgsl-runtime.ts:184-240, :669-919)
 *   chonk_engine_run_token         LlamaWgslEngine.runToken (:1025-1150)
 *   chonk_engine_prefill           the prompt loop of generateLlamaWgsl (:281-288),
 *                                  runToken(id, false) per token, as row batches
 *   chonk_engine_generate          generateLlamaWgsl (:242-314)
 *   chonk_engine_reset             LlamaWgslEngine.reset (:1011-1019)
 *   chonk_engine_reset_conversation resetLlamaWgslConversation (:320-324)
 *   chonk_engine_position          LlamaWgslEngine.position (:1021-1023)
 *   chonk_engine_destroy           disposeLlamaWgsl / LlamaWgslEngine.dispose (:316-318, :1152-1215)
 *   chonk_engine_read_logits       (new) logits readback for parity tests; the
 *                                  reference keeps logits GPU-only (:893)
 *
 * Conventions: plain pointers and sizes, no ownership transfer. Every function
 * returns CHONK_OK (0) or a negative status; the message of the last failure
 * is available from chonk_engine_last_error(engine) or, for calls without an
 * engine, chonk_last_error(). Messages reuse the reference's wording
 * ("Llama WGSL context exhausted at N tokens", "unsupported GGUF tensor type
 * X", "Llama GGUF WGSL does not support architecture X", ...).
 * An engine is not re-entrant: a call made while another call on the same
 * engine is in progress returns CHONK_EBUSY (the reference's `active` guard,
 * :1221-1224). Engines on different threads are independent: of the engines
 * on one GPU only the first that qualifies decodes with the spin-merging
 * attention (chunks of one launch wait for each other, so its grid must be
 * resident at once); engines created while it exists use the arrival-counter
 * attention, which never waits, so concurrent decoding cannot stall. The
 * spin-merging engine runs its q|k|v matvec inside the attention launch only
 * while it is the only engine on its GPU (separate launches otherwise).
 * A HIP error marks the engine lost; later calls that touch the device
 * (position, info and destroy still answer) fail fast with CHONK_ELOST
 * (the LFM runtime's deviceLost behaviour, lfm-wgsl-runtime.ts:704-707,
 * :729-731).
 */
#ifndef CHONK_H
#define CHONK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHONK_OK 0
#define CHONK_EINVAL -1      /* bad argument / unsupported model */
#define CHONK_EIO -2         /* file or shard read failure */
#define CHONK_EHIP -3        /* HIP runtime error (engine is now lost) */
#define CHONK_ECONTEXT -4    /* "Llama WGSL context exhausted at N tokens" */
#define CHONK_EBUSY -5       /* concurrent call on the same engine */
#define CHONK_ELOST -6       /* engine lost after an earlier HIP error */
#define CHONK_ENOMEM -7      /* device allocation failed */

#define CHONK_KV_F16 0       /* fp16 K/V cache (default) */
#define CHONK_KV_F32 1       /* fp32 K/V cache, the reference layout (:830-831) */

typedef struct chonk_engine chonk_engine;

/* The ModelDef fields the engine reads (src/lib/registry.ts:14-46). */
typedef struct {
  const char* id;                    /* ModelDef.id (diagnostics only) */
  int32_t vocab;                     /* ModelDef.vocab */
  int32_t layers;                    /* ModelDef.layers */
  int32_t max_context;               /* ModelDef.maxContext */
  const int32_t* eos_ids;            /* ModelDef.eosIds */
  int32_t n_eos;
  float default_repetition_penalty;  /* ModelDef.defaultRepetitionPenalty (0 = unset -> 1) */
  int32_t kv_dtype;                  /* CHONK_KV_F16 or CHONK_KV_F32 */
  int32_t device;                    /* HIP device ordinal */
} chonk_model_def;

/* SamplingOptions (src/lib/sampling.ts:1-7); seed replaces Math.random():
 * the uniform draw for the token sampled at position p is
 * (mix64(seed + 0x9E3779B97F4A7C15*(p+1)) >> 11) * 2^-53 with mix64 the
 * splitmix64 finaliser. */
typedef struct {
  double temperature;         /* default 0 */
  double top_p;               /* default 1 */
  int32_t top_k;              /* default 0 */
  double repetition_penalty;  /* default 1 */
  uint64_t seed;
} chonk_sampling;

typedef struct {
  int32_t hidden, ffn, vocab, layers, heads, kv_heads, head_dim, context;
  int32_t architecture;      /* 0 llama, 1 qwen3, 2 gemma3, 3 gpt2, 4 openelm, 5 lfm2, 6 granitehybrid */
  int32_t qk_norm, interleaved_rope, kv_dtype;
  uint64_t weight_bytes_per_token;  /* GGUF bytes of every matrix read per token (incl. lm_head + embedding row) */
  uint64_t device_bytes;            /* device memory held by the engine */
  int32_t kernels_per_step;         /* per-phase kernels of one decode step (chonk_engine_bench_kernel ids) */
  int32_t persistent_step;          /* always 0 (kept for layout: the one-launch step was retired) */
  int32_t noalloc_prefill_rows;     /* most tokens one chonk_engine_prefill_noalloc call takes (0: none) */
  int32_t spin_attention;           /* 1: decodes with the spin-merging attention (one engine per GPU) */
  int32_t fused_attention;          /* layers whose q|k|v matvec runs inside the attention launch */
} chonk_engine_info;

typedef struct {
  double prefill_ms;     /* wall time of the prompt steps */
  double decode_ms;      /* wall time of the generated steps */
  int32_t prompt_tokens;
  int32_t generated_tokens;
  double tokens_per_sec; /* generated / (prefill + decode), the reference's formula (:266, :312) */
} chonk_gen_stats;

const char* chonk_last_error(void);
const char* chonk_engine_last_error(const chonk_engine* e);

/* Loads a GGUF file, or a directory with manifest.json + NNNN.bin shards
 * (scripts/shard-gguf.mjs format), uploads the weights and allocates the K/V
 * cache of min(def->max_context, GGUF context_length) positions. */
int chonk_engine_create(const chonk_model_def* def, const char* path, chonk_engine** out);
/* Same from a caller buffer holding a whole GGUF file (copied). */
int chonk_engine_create_from_memory(const chonk_model_def* def, const void* gguf_bytes, size_t n_bytes,
                                    chonk_engine** out);
int chonk_engine_destroy(chonk_engine* e);
int chonk_engine_info_get(const chonk_engine* e, chonk_engine_info* out);

/* runToken: processes `token` at the current position; when need_logits is
 * non-zero, computes logits and selects the next token (greedy argmax, or
 * the candidate sampler when temperature > 0, top_p < 1 or top_k > 0). The
 * repetition penalty applies to `penalized` (the reference's
 * penalizedTokenIds; at most the last `context` ids are used) and, in the
 * candidate sampler, again to `seen` (seenIds). out_token receives 0 when
 * need_logits is zero. */
int chonk_engine_run_token(chonk_engine* e, int32_t token, int32_t need_logits, const chonk_sampling* s,
                           const int32_t* penalized, size_t n_penalized, const int32_t* seen, size_t n_seen,
                           int32_t* out_token);

/* Appends tokens[0, n) to the context without computing logits, with the
 * result of n calls of run_token(token, need_logits = 0) (the reference's
 * prompt loop, generateLlamaWgsl :281-288), computed as row batches: the
 * linear layers as dequant-fused MFMA GEMMs and a causal attention over the
 * cache. generate uses the same pass for all but the last prompt token. */
int chonk_engine_prefill(chonk_engine* e, const int32_t* tokens, size_t n);

/* chonk_engine_prefill without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). It is not for code under
 * HIP graph capture: the call copies the token ids to the device and waits
 * for its pass to finish before it returns.
 * The row buffers of the pass come from one 48 MiB device array per GPU,
 * reserved when the library is loaded on that GPU and held until the process
 * ends, instead of the ~50-60 MB that chonk_engine_prefill allocates on its
 * first call. One call takes at most chonk_engine_info.noalloc_prefill_rows
 * tokens (one pass; CHONK_EINVAL beyond that, or when the model's row buffers
 * do not fit). Every call on one GPU shares that GPU's array: calls of
 * engines on one GPU take turns on a per-GPU lock (a second thread's call
 * waits until the first has finished). Results equal chonk_engine_prefill's
 * to fp32 rounding (passes of a different row count change the GEMMs' K
 * split). */
int chonk_engine_prefill_noalloc(chonk_engine* e, const int32_t* tokens, size_t n);

/* generateLlamaWgsl: prefix reuse against the previous conversation, prompt
 * prefill, then up to max_new_tokens generated ids (stopping after an EOS
 * id), all on the device without a per-token host round trip. A negative
 * max_new_tokens means "not given" (128); 0 prefills only. The penalty list
 * is prompt + generated, as in the reference. out_ids receives
 * min(n, out_cap) ids; *n_out the count. */
int chonk_engine_generate(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new_tokens,
                          const chonk_sampling* s, int32_t* out_ids, size_t out_cap, size_t* n_out,
                          chonk_gen_stats* stats);

/* The same loop stepped from the host one token at a time (one readback per
 * token, as the reference does), for callers that stream tokens or cancel:
 * before each generated id is appended, callback(user, 0, 0) is the
 * reference's shouldStop() (non-zero stops); after it is appended,
 * callback(user, 1, id) is onToken. Results equal chonk_engine_generate's. */
typedef int32_t (*chonk_token_callback)(void* user, int32_t event, int32_t token);
int chonk_engine_generate_stepped(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new_tokens,
                                  const chonk_sampling* s, chonk_token_callback callback, void* user,
                                  int32_t* out_ids, size_t out_cap, size_t* n_out, chonk_gen_stats* stats);

/* Conversation cache of the last generate call (LoadedLlamaWgslModel's
 * cachedTokenIds / cachedNextId, :174-182): *n_cached ids are copied to ids
 * (up to cap); *next_id is cachedNextId or -1 when it is null. */
int chonk_engine_conversation(chonk_engine* e, int32_t* ids, size_t cap, size_t* n_cached, int32_t* next_id);

int chonk_engine_reset(chonk_engine* e);
int chonk_engine_reset_conversation(chonk_engine* e);
int chonk_engine_position(const chonk_engine* e, int32_t* out_pos);

/* Test hook (no counterpart in the reference, which cannot force a device
 * error): the engine's next kernel launch reports a HIP error. That call
 * returns CHONK_EHIP, the engine is marked lost, and every later call on it
 * that touches the device returns CHONK_ELOST (the LFM runtime's deviceLost rule,
 * lfm-wgsl-runtime.ts:704-707, :729-731); destroy still frees it. */
int chonk_engine_debug_fail_next_launch(chonk_engine* e);

/* Logits of the last step that computed them (vocab floats). */
int chonk_engine_read_logits(chonk_engine* e, float* out, size_t n);

/* Intermediate buffers of the last step, for parity tests:
 * 0 residual after the last layer [hidden], 1 attention output of the last
 * layer [heads*head_dim], 2 group candidates [ceil(vocab/256) x {f32, u32}],
 * 3 raw q|k|v projections of the last layer [qdim + 2 kvdim]. */
int chonk_engine_read_buffer(chonk_engine* e, int32_t which, void* out, size_t n_bytes);
/* K or V cache row of `layer` at position `pos` as floats [kv_heads*head_dim]. */
int chonk_engine_read_kv(chonk_engine* e, int32_t layer, int32_t is_value, int32_t pos, float* out);

/* Benchmark hooks -------------------------------------------------------
 * Runs `n_warmup` then `n_steps` greedy decode steps by graph replay from the
 * current state (the history token at the current position is consumed), timed
 * with HIP events on the engine stream. */
int chonk_engine_bench_decode(chonk_engine* e, int32_t n_warmup, int32_t n_steps, double* ms_total);
/* Average duration (microseconds) of one kernel of the decode step, launched
 * `reps` times back-to-back with the arguments it has in the step, timed with
 * HIP events on the engine stream. kernel_id indexes the step's launch list;
 * name receives its label (e.g. "L3.gateup q4_k"); bytes its algorithmic
 * bytes per launch. reps = 0 launches nothing (name and bytes only). */
int chonk_engine_bench_kernel(chonk_engine* e, int32_t kernel_id, int32_t reps, double* avg_us, char* name,
                              size_t name_len, uint64_t* bytes);
/* The same kernel timed launch by launch with HIP events, `reps` times with
 * the caches flushed first (a write of max(flush_bytes, 512 MiB) to a
 * benchmark buffer evicts L2 and the 256 MB Infinity Cache: *cold_us) and
 * `reps` times right after an identical launch (*warm_us). */
int chonk_engine_bench_kernel_cold(chonk_engine* e, int32_t kernel_id, int32_t reps, uint64_t flush_bytes,
                                   double* cold_us, double* warm_us);
/* Mean duration (microseconds) of one launch of the step kernels ids[0..n_ids)
 * when the list is launched back to back, `rounds` times, with the arguments
 * they have in the step, timed with HIP events on the engine stream. A list
 * of one phase of every layer (e.g. each layer's attention) meets its weights
 * and K/V rows as cold as the step does, unlike repeats of one launch. */
int chonk_engine_time_kernels(chonk_engine* e, const int32_t* ids, int32_t n_ids, int32_t rounds,
                              double* us_per_launch);
/* Writes `pos` synthetic positions into the K/V cache and sets the position,
 * so that long-context decode can be measured without a full prefill. */
int chonk_engine_fake_context(chonk_engine* e, int32_t pos, uint64_t seed);

/* Batched decoding (no counterpart in the reference, which runs one sequence
 * per engine) -----------------------------------------------------------------
 * Independent sequences over one engine's weights, each with its own paged
 * fp16 K/V cache (pages of 64 positions); one step advances any subset of the
 * sequences by one token, every linear layer a dequant-fused MFMA GEMM over
 * the batch rows. Greedy selection (argmax, no repetition penalty). The
 * engine's own conversation is not touched. */
typedef struct chonk_batch chonk_batch;
int chonk_batch_create(chonk_engine* e, int32_t max_seqs, int32_t max_tokens_per_seq, chonk_batch** out);
int chonk_batch_destroy(chonk_batch* b);
/* Starts sequence `seq` over: K/V of the prompt, and the greedy next id. */
int chonk_batch_prefill(chonk_batch* b, int32_t seq, const int32_t* tokens, size_t n, int32_t* next_id);
/* Appends tokens[i] to sequence seqs[i] (distinct) for i < n and returns each
 * sequence's greedy next id in next_ids[i]. */
int chonk_batch_step(chonk_batch* b, const int32_t* seqs, const int32_t* tokens, size_t n, int32_t* next_ids);
int chonk_batch_position(const chonk_batch* b, int32_t seq, int32_t* out_pos);
/* Logits of row `row` of the last prefill (row 0) or step. */
int chonk_batch_read_logits(chonk_batch* b, int32_t row, float* out, size_t n);

/* Kernel-level entry points (tests) ---------------------------------------
 * GGUF rows are given as raw block bytes in host memory; the call uploads
 * them with the engine's repacking, runs the kernel on `device`, and returns
 * the result to host memory. */
int chonk_dequant(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len,
                  float* out);
/* y[N] = W[N,K] x[K]; when reps > 0 also times `reps` back-to-back launches
 * and stores the mean microseconds in *avg_us. */
int chonk_matvec(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len,
                 const float* x, float* y, int32_t reps, double* avg_us);
/* Y[T,N] = X[T,K] W[N,K]^T with the batched pass's GEMM (fp16 hi/lo operand
 * split on the matrix cores, fp32 accumulation); x and y are row-major;
 * K <= 4096 and T <= 65536 (CHONK_EINVAL otherwise). When
 * reps > 0 also times `reps` launches (the operand split included) and
 * stores the mean microseconds in *avg_us. */
int chonk_gemm(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len,
               const float* x, int64_t n_tokens, float* y, int32_t reps, double* avg_us);

/* Model files --------------------------------------------------------------- */
typedef struct {
  const char* arch;      /* "llama" | "qwen3" | "gemma3" | "gpt2" | "openelm" */
  const char* recipe;    /* "q4_k_m" | "q8_0" | "q4_k" | "q6_k" | "q5_0" */
  int32_t hidden, layers, heads, kv_heads, head_dim, ffn, vocab, context_length;
  float rope_theta, norm_eps;
  int32_t sliding_window;
  uint64_t seed;
  float weight_std;      /* 0 -> 0.02 */
  float norm_std;        /* 0 -> 0.02 */
  /* openelm: per-layer head, kv-head and feed-forward counts, `layers` entries
   * each (null: heads / kv_heads / ffn for every layer) */
  const int32_t* layer_heads;
  const int32_t* layer_kv_heads;
  const int32_t* layer_ffn;
} chonk_synth_config;

/* Writes a seeded random-init decoder as GGUF (see the recipe in synth.h). */
int chonk_write_synthetic_gguf(const chonk_synth_config* c, const char* path, int32_t n_threads);
/* Splits a GGUF file into <out_dir>/NNNN.bin + manifest.json. */
int chonk_write_shards(const char* gguf_path, const char* out_dir, uint64_t shard_size, const char* quant);

#ifdef __cplusplus
}
#endif

#endif
