// Synthetic GGUF decoder models for tests and benchmarks.
//
// Weight init: linear weights mean 0, std weight_std (N(0, 0.02) by
// default); norm weights 1 + N(0, norm_std). Values come from a counter-based
// generator keyed on (seed, tensor name, element index), so files are
// reproducible for any thread count.
//
// Quantization recipe "q4_k_m" (llama.cpp llama_tensor_get_type, restated):
//   * default Q4_K;
//   * the output projection (the tied token_embd here) is Q6_K, or Q8_0 when
//     its row length is not a multiple of 256;
//   * attn_v and ffn_down are Q6_K on layers where
//     i < n/8 || i >= 7n/8 || (i - n/8) % 3 == 2;
//   * a fused attn_qkv is Q5_K;
//   * any K-quant whose row length is not a multiple of 256 falls back:
//     Q4_K -> Q5_0, Q6_K -> Q8_0, Q5_K -> Q5_1;
//   * 1-D norm weights stay F32.
// "q8_0": every matrix Q8_0. "q4_k"/"q6_k"/"q5_0": one type everywhere (with
// the K-quant fallback). "f32"/"f16": unquantized.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace chonk {

struct SynthConfig {
  std::string arch = "llama";  // llama | qwen3 | gemma3 | gpt2 | openelm | lfm2
  std::string name;
  int hidden = 576;
  int layers = 30;
  int heads = 9;
  int kv_heads = 3;
  int head_dim = 0;            // 0: hidden / heads and no key_length metadata
  int ffn = 1536;
  int vocab = 49152;
  int context_length = 8192;
  float rope_theta = 100000.f;
  float norm_eps = 1e-5f;
  int sliding_window = 0;      // gemma3 only
  std::string recipe = "q4_k_m";
  uint64_t seed = 1;
  float weight_std = 0.02f;
  float norm_std = 0.02f;
  // openelm: per-layer head, kv-head and feed-forward counts (empty: the
  // scalars above for every layer); written as the arrays
  // openelm.attention.head_count, .head_count_kv and .feed_forward_length.
  // lfm2: layer_kv_heads alone, 0 marking a short-convolution layer (written as
  // lfm2.attention.head_count_kv)
  std::vector<int> layer_heads, layer_kv_heads, layer_ffn;
};

uint32_t recipe_tensor_type(const std::string& recipe, const std::string& role, int layer, int n_layers,
                            uint64_t row_len);

void write_synthetic_gguf(const SynthConfig& c, const std::string& path, int n_threads);

}  // namespace chonk
