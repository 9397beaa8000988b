// Synthetic GGUF model writer: seeded random-init decoder weights quantized
// with the reference block quantizers under a llama.cpp-style type recipe.
//
// The tensor names, metadata keys and shapes are the ones the reference's
// manifest builder reads (src/lib/llama-wgsl-runtime.ts:326-425):
//   token_embd.weight, output_norm.weight, blk.N.{attn_norm, attn_q, attn_k,
//   attn_v, attn_output, attn_q_norm, attn_k_norm, ffn_norm, ffn_gate, ffn_up,
//   ffn_down, post_attention_norm, post_ffw_norm}.weight, and
//   <arch>.{block_count, embedding_length, feed_forward_length,
//   attention.head_count, attention.head_count_kv, attention.key_length,
//   context_length, rope.freq_base, attention.layer_norm_rms_epsilon},
//   gemma3.attention.sliding_window. Architecture openelm has one fused
//   blk.N.attn_qkv per layer (rows q | k | v) and per-layer head, kv-head and
//   feed-forward counts as metadata arrays (:331-416). Architecture lfm2
//   follows the LFM runtime's loader (src/lib/lfm-wgsl-runtime.ts:505-560):
//   blk.N.shortconv.{conv, in_proj, out_proj}.weight on convolution layers,
//   blk.N.attn_{q, k, v, output, q_norm, k_norm}.weight on attention layers,
//   token_embd_norm.weight as the final norm; the layer kinds are written as
//   lfm2.attention.head_count_kv, one entry per layer, 0 on convolution layers.
// Type recipe (Q4_K_M): llama.cpp's llama_tensor_get_type as restated in the
// header of synth.h. Architecture gpt2 follows the GPT runtime's manifest
// (src/lib/gpt-wgsl-runtime.ts:274-356; gpt2_plan below). Architecture
// granitehybrid follows the Granite runtime's loader
// (src/lib/granite-wgsl-runtime.ts:536-624; granite_plan below): Mamba2 layers
// (layer_kv_heads 0) hold blk.N.ssm_{in, out}.weight, ssm_conv1d.{weight, bias},
// ssm_dt.bias, ssm_a, ssm_d and ssm_norm.weight with the runtime's fixed ratios
// (inner size 2 * hidden, 32-wide heads, 128 states, 4 taps, one group).

#include "synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <thread>
#include <vector>

#include "ggml_types.h"
#include "gguf.h"
#include "quantize.h"

namespace chonk {
namespace {

inline uint64_t splitmix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

inline uint64_t name_hash(const std::string& s) {
  uint64_t h = 1469598103934665603ull;  // FNV-1a
  for (unsigned char c : s) h = (h ^ c) * 1099511628211ull;
  return h;
}

// Standard normal value for (stream, index) via Box-Muller on two
// counter-based uniforms; independent of thread scheduling.
inline float normal_at(uint64_t stream, uint64_t i) {
  const uint64_t a = splitmix64(stream ^ splitmix64(2 * i));
  const uint64_t b = splitmix64(stream ^ splitmix64(2 * i + 1));
  const double u1 = ((a >> 11) + 1) * (1.0 / 9007199254740993.0);  // (0, 1]
  const double u2 = (b >> 11) * (1.0 / 9007199254740992.0);        // [0, 1)
  return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

// Standard deviation of the synthetic short-convolution taps: large enough that
// the convolution branch moves the residual stream.
constexpr float kLfmConvStd = 0.5f;
// granitehybrid: the Granite runtime's fixed Mamba2 geometry (granite-wgsl-runtime.ts:526-533,
// :586-596) and the spread of the synthetic depthwise conv taps
constexpr uint64_t kGraniteHeadDim = 32, kGraniteState = 128;
constexpr float kGraniteConvStd = 0.25f;

bool use_more_bits(int i, int n) { return i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2; }

uint32_t fallback_type(uint32_t type, uint64_t row_len) {
  if (row_len % 256 == 0) return type;
  if (type == GGML_Q4_K) return GGML_Q5_0;
  if (type == GGML_Q6_K) return GGML_Q8_0;
  if (type == GGML_Q5_K) return GGML_Q5_1;
  return type;
}

struct TensorPlan {
  std::string name;
  uint64_t rows;     // N
  uint64_t row_len;  // K
  uint32_t type;
  float mean;        // weights = mean + std * normal
  float std;
};

}  // namespace

uint32_t recipe_tensor_type(const std::string& recipe, const std::string& role, int layer, int n_layers,
                            uint64_t row_len) {
  if (role == "norm") return GGML_F32;
  if (recipe == "f32") return GGML_F32;
  if (recipe == "f16") return GGML_F16;
  if (recipe == "q8_0") return row_len % 32 == 0 ? GGML_Q8_0 : GGML_F16;
  if (recipe == "q4_k" || recipe == "q6_k" || recipe == "q5_0") {
    const uint32_t t = recipe == "q4_k" ? GGML_Q4_K : recipe == "q6_k" ? GGML_Q6_K : GGML_Q5_0;
    return fallback_type(t, row_len);
  }
  if (recipe != "q4_k_m") throw std::runtime_error("unknown quantization recipe " + recipe);
  uint32_t t = GGML_Q4_K;
  if (role == "output") {
    t = row_len % 256 != 0 ? GGML_Q8_0 : GGML_Q6_K;
  } else if (role == "attn_v" || role == "ffn_down") {
    if (use_more_bits(layer, n_layers)) t = GGML_Q6_K;
  } else if (role == "attn_qkv") {
    t = GGML_Q5_K;
  }
  return fallback_type(t, row_len);
}

// The tensor plan of a GPT-2 decoder as the reference's GPT runtime reads it
// (src/lib/gpt-wgsl-runtime.ts:274-356): learned position table, LayerNorm
// weights and biases, fused q|k|v and biases on every linear layer, a separate
// output matrix.
std::vector<TensorPlan> gpt2_plan(const SynthConfig& c) {
  const uint64_t H = (uint64_t)c.hidden, F = (uint64_t)c.ffn;
  std::vector<TensorPlan> plan;
  plan.push_back({"token_embd.weight", (uint64_t)c.vocab, H, recipe_tensor_type(c.recipe, "output", -1, c.layers, H),
                  0.f, c.weight_std});
  plan.push_back({"position_embd.weight", (uint64_t)c.context_length, H, GGML_F32, 0.f, c.weight_std});
  for (int i = 0; i < c.layers; ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    auto lin = [&](const std::string& role, uint64_t n, uint64_t k) {
      plan.push_back({p + role + ".weight", n, k, recipe_tensor_type(c.recipe, role, i, c.layers, k), 0.f, c.weight_std});
      plan.push_back({p + role + ".bias", 1, n, GGML_F32, 0.f, c.weight_std});
    };
    auto ln = [&](const std::string& role) {
      plan.push_back({p + role + ".weight", 1, H, GGML_F32, 1.f, c.norm_std});
      plan.push_back({p + role + ".bias", 1, H, GGML_F32, 0.f, c.norm_std});
    };
    ln("attn_norm");
    lin("attn_qkv", 3 * H, H);
    lin("attn_output", H, H);
    ln("ffn_norm");
    lin("ffn_up", F, H);
    lin("ffn_down", H, F);
  }
  plan.push_back({"output_norm.weight", 1, H, GGML_F32, 1.f, c.norm_std});
  plan.push_back({"output_norm.bias", 1, H, GGML_F32, 0.f, c.norm_std});
  plan.push_back({"output.weight", (uint64_t)c.vocab, H, recipe_tensor_type(c.recipe, "output", -1, c.layers, H), 0.f,
                  c.weight_std});
  return plan;
}

// The tensor plan of a Granite-4.0-H hybrid decoder (granite-wgsl-runtime.ts:
// 536-624): per layer attn_norm, ffn_norm, the SwiGLU matrices, and either a
// Mamba2 block or NoPE attention; token_embd doubles as the output projection.
// ssm_a holds -exp(A_log) (negative), ssm_dt.bias sits near softplus^-1 of a
// small step, ssm_d near 1.
std::vector<TensorPlan> granite_plan(const SynthConfig& c, const std::vector<int>& lkv, int head_dim) {
  const uint64_t H = (uint64_t)c.hidden, F = (uint64_t)c.ffn;
  const uint64_t inner = 2 * H, conv = inner + 2 * kGraniteState, nh = inner / kGraniteHeadDim;
  std::vector<TensorPlan> plan;
  plan.push_back({"token_embd.weight", (uint64_t)c.vocab, H, recipe_tensor_type(c.recipe, "output", -1, c.layers, H),
                  0.f, c.weight_std});
  for (int i = 0; i < c.layers; ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    auto lin = [&](const std::string& role, uint64_t n, uint64_t k) {
      plan.push_back({p + role + ".weight", n, k, recipe_tensor_type(c.recipe, role, i, c.layers, k), 0.f,
                      c.weight_std});
    };
    auto vec = [&](const std::string& name, uint64_t n, float mean, float std) {
      plan.push_back({p + name, 1, n, GGML_F32, mean, std});
    };
    vec("attn_norm.weight", H, 1.f, c.norm_std);
    if (lkv[(size_t)i] == 0) {
      lin("ssm_in", inner + conv + nh, H);
      plan.push_back({p + "ssm_conv1d.weight", conv, 4, GGML_F32, 0.f, kGraniteConvStd});
      vec("ssm_conv1d.bias", conv, 0.f, c.weight_std);
      vec("ssm_dt.bias", nh, -4.f, 0.5f);
      vec("ssm_a", nh, -4.f, 0.5f);
      vec("ssm_d", nh, 1.f, 0.1f);
      vec("ssm_norm.weight", inner, 1.f, c.norm_std);
      lin("ssm_out", H, inner);
    } else {
      const uint64_t qdim = (uint64_t)c.heads * head_dim, kvdim = (uint64_t)lkv[(size_t)i] * head_dim;
      lin("attn_q", qdim, H);
      lin("attn_k", kvdim, H);
      lin("attn_v", kvdim, H);
      lin("attn_output", H, qdim);
    }
    vec("ffn_norm.weight", H, 1.f, c.norm_std);
    lin("ffn_gate", F, H);
    lin("ffn_up", F, H);
    lin("ffn_down", H, F);
  }
  plan.push_back({"output_norm.weight", 1, H, GGML_F32, 1.f, c.norm_std});
  return plan;
}

void write_synthetic_gguf(const SynthConfig& c, const std::string& path, int n_threads) {
  const std::string& a = c.arch;
  if (a != "llama" && a != "qwen3" && a != "gemma3" && a != "gpt2" && a != "openelm" && a != "lfm2" &&
      a != "granitehybrid")
    throw std::runtime_error("synthetic writer: unsupported arch " + a);
  if (c.hidden <= 0 || c.layers <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.ffn <= 0 || c.vocab <= 0)
    throw std::runtime_error("synthetic writer: non-positive dimension");
  const bool granite = a == "granitehybrid";
  // (a 0 kv-head entry marks an lfm2 convolution layer or a granitehybrid Mamba2 layer)
  const bool openelm = a == "openelm", lfm = a == "lfm2" || granite;
  auto per_layer = [&](const std::vector<int>& v, int fallback, const char* what, bool zero_ok) {
    if (v.empty()) return std::vector<int>((size_t)c.layers, fallback);
    if (!openelm && !(lfm && zero_ok))
      throw std::runtime_error(std::string("synthetic writer: per-layer ") + what + " needs arch openelm");
    if ((int)v.size() != c.layers) throw std::runtime_error(std::string("synthetic writer: ") + what + " length != layers");
    for (int x : v)
      if (x < 0 || (x == 0 && !(lfm && zero_ok))) throw std::runtime_error("synthetic writer: non-positive dimension");
    return v;
  };
  const std::vector<int> lh = per_layer(c.layer_heads, c.heads, "heads", false);
  // lfm2: 0 kv heads marks a short-convolution layer
  const std::vector<int> lkv = per_layer(c.layer_kv_heads, c.kv_heads, "kv_heads", true);
  const std::vector<int> lff = per_layer(c.layer_ffn, c.ffn, "ffn", false);
  for (int i = 0; i < c.layers; ++i)
    if (lkv[(size_t)i] > 0 && lh[(size_t)i] % lkv[(size_t)i] != 0)
      throw std::runtime_error("synthetic writer: heads not a multiple of kv_heads");
  if (openelm && c.head_dim <= 0) throw std::runtime_error("synthetic writer: openelm needs head_dim");
  const int head_dim = c.head_dim > 0 ? c.head_dim : c.hidden / c.heads;
  const uint64_t H = (uint64_t)c.hidden;
  const bool gemma = a == "gemma3";
  const bool qk_norm = a == "qwen3" || gemma || openelm || lfm;
  const float w_std = c.weight_std;
  const float n_std = c.norm_std;

  std::vector<TensorPlan> plan;
  if (a == "gpt2") plan = gpt2_plan(c);
  if (granite) {
    if (c.recipe != "q4_k_m" && c.recipe != "q8_0")
      throw std::runtime_error("synthetic writer: granitehybrid files are Q4_K_M or Q8_0");
    if (c.hidden % 16 != 0) throw std::runtime_error("synthetic writer: granitehybrid hidden must be a multiple of 16");
    plan = granite_plan(c, lkv, head_dim);
  }
  // tied embeddings: token_embd doubles as the output projection ("output" role)
  if (a != "gpt2" && !granite) plan.push_back({"token_embd.weight", (uint64_t)c.vocab, H,
                  recipe_tensor_type(c.recipe, "output", -1, c.layers, H), 0.f, w_std});
  for (int i = 0; i < (a == "gpt2" || granite ? 0 : c.layers); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    auto lin = [&](const std::string& role, uint64_t n, uint64_t k) {
      plan.push_back({p + role + ".weight", n, k, recipe_tensor_type(c.recipe, role, i, c.layers, k), 0.f, w_std});
    };
    auto norm = [&](const std::string& role, uint64_t n) { plan.push_back({p + role + ".weight", 1, n, GGML_F32, 1.f, n_std}); };
    const uint64_t qdim = (uint64_t)lh[(size_t)i] * head_dim, kvdim = (uint64_t)lkv[(size_t)i] * head_dim;
    const uint64_t F = (uint64_t)lff[(size_t)i];
    norm("attn_norm", H);
    if (lfm && lkv[(size_t)i] == 0) {
      // short convolution: in_proj rows B | C | x, a 3-tap depthwise filter per channel
      plan.push_back({p + "shortconv.conv.weight", H, 3, GGML_F32, 0.f, kLfmConvStd});
      lin("shortconv.in_proj", 3 * H, H);
      lin("shortconv.out_proj", H, H);
      norm("ffn_norm", H);
      lin("ffn_gate", F, H);
      lin("ffn_up", F, H);
      lin("ffn_down", H, F);
      continue;
    }
    if (openelm) {
      lin("attn_qkv", qdim + 2 * kvdim, H);
    } else {
      lin("attn_q", qdim, H);
      lin("attn_k", kvdim, H);
      lin("attn_v", kvdim, H);
    }
    lin("attn_output", H, qdim);
    if (qk_norm) {
      norm("attn_q_norm", (uint64_t)head_dim);
      norm("attn_k_norm", (uint64_t)head_dim);
    }
    if (gemma) norm("post_attention_norm", H);
    norm("ffn_norm", H);
    lin("ffn_gate", F, H);
    lin("ffn_up", F, H);
    lin("ffn_down", H, F);
    if (gemma) norm("post_ffw_norm", H);
  }
  if (a != "gpt2" && !granite)
    plan.push_back({lfm ? "token_embd_norm.weight" : "output_norm.weight", 1, H, GGML_F32, 1.f, n_std});

  GgufWriter w;
  w.set_string("general.architecture", a);
  w.set_string("general.name", c.name.empty() ? "synthetic-" + a : c.name);
  w.set_u32("general.file_type", c.recipe == "q8_0" ? 7u : c.recipe == "q4_k_m" ? 15u : 0u);
  w.set_u32(a + ".context_length", (uint32_t)c.context_length);
  w.set_u32(a + ".embedding_length", (uint32_t)c.hidden);
  w.set_u32(a + ".block_count", (uint32_t)c.layers);
  if (lfm) {
    w.set_u32(a + ".feed_forward_length", (uint32_t)c.ffn);
    w.set_u32(a + ".attention.head_count", (uint32_t)c.heads);
    w.set_u32_array(a + ".attention.head_count_kv", std::vector<uint32_t>(lkv.begin(), lkv.end()));
    if (granite) {
      // llama.cpp's granitehybrid keys (the Granite runtime itself reads only
      // general.architecture and general.file_type, :359-371)
      w.set_u32(a + ".ssm.conv_kernel", 4u);
      w.set_u32(a + ".ssm.state_size", (uint32_t)kGraniteState);
      w.set_u32(a + ".ssm.group_count", 1u);
      w.set_u32(a + ".ssm.inner_size", (uint32_t)(2 * H));
      w.set_u32(a + ".ssm.time_step_rank", (uint32_t)(2 * H / kGraniteHeadDim));
      w.set_f32(a + ".embedding_scale", 12.f);
      w.set_f32(a + ".residual_scale", 0.246f);
      w.set_f32(a + ".logit_scale", 3.f);
      w.set_f32(a + ".attention.scale", 0.015625f);
      w.set_f32(a + ".attention.layer_norm_rms_epsilon", c.norm_eps);
    } else {
      w.set_u32(a + ".shortconv.l_cache", 3u);
    }
  } else if (openelm) {
    auto u32s = [](const std::vector<int>& v) { return std::vector<uint32_t>(v.begin(), v.end()); };
    w.set_u32_array(a + ".feed_forward_length", u32s(lff));
    w.set_u32_array(a + ".attention.head_count", u32s(lh));
    w.set_u32_array(a + ".attention.head_count_kv", u32s(lkv));
  } else {
    w.set_u32(a + ".feed_forward_length", (uint32_t)c.ffn);
    w.set_u32(a + ".attention.head_count", (uint32_t)c.heads);
    if (a != "gpt2") w.set_u32(a + ".attention.head_count_kv", (uint32_t)c.kv_heads);
  }
  if (a == "gpt2") w.set_f32("gpt2.attention.layer_norm_epsilon", c.norm_eps);
  if (c.head_dim > 0) {
    w.set_u32(a + ".attention.key_length", (uint32_t)head_dim);
    w.set_u32(a + ".attention.value_length", (uint32_t)head_dim);
  }
  if (a != "gpt2" && !granite) {
    w.set_u32(a + ".rope.dimension_count", (uint32_t)head_dim);
    w.set_f32(a + ".rope.freq_base", c.rope_theta);
    w.set_f32(a + ".attention.layer_norm_rms_epsilon", c.norm_eps);
  }
  w.set_u32(a + ".vocab_size", (uint32_t)c.vocab);
  if (gemma) w.set_u32("gemma3.attention.sliding_window", (uint32_t)c.sliding_window);

  const int nt = std::max(1, n_threads);
  for (size_t ti = 0; ti < plan.size(); ++ti) {
    const TensorPlan& t = plan[ti];
    TypeTraits tt;
    type_traits(t.type, &tt);
    const uint64_t row_bytes = t.row_len / tt.block_elems * tt.block_bytes;
    std::vector<uint8_t> data(row_bytes * t.rows);
    const uint64_t stream = splitmix64(c.seed ^ name_hash(t.name));
    std::vector<std::thread> pool;
    std::vector<std::string> errors(nt);
    for (int th = 0; th < nt; ++th) {
      pool.emplace_back([&, th]() {
        std::vector<float> row(t.row_len);
        for (uint64_t r = th; r < t.rows; r += nt) {
          for (uint64_t k = 0; k < t.row_len; ++k) row[k] = t.mean + t.std * normal_at(stream, r * t.row_len + k);
          if (!quantize_rows(t.type, row.data(), data.data() + r * row_bytes, (int64_t)t.row_len)) {
            errors[th] = "quantization failed for " + t.name;
            return;
          }
        }
      });
    }
    for (auto& th : pool) th.join();
    for (const auto& e : errors)
      if (!e.empty()) throw std::runtime_error(e);
    std::vector<uint64_t> shape = t.rows == 1 ? std::vector<uint64_t>{t.row_len} : std::vector<uint64_t>{t.row_len, t.rows};
    w.add_tensor(t.name, shape, t.type, std::move(data));
  }
  w.write(path);
}

}  // namespace chonk
