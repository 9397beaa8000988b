// Decode engine: GGUF -> device upload, K/V cache, step graphs, C ABI.
//
// Host semantics follow the reference's llama-webgpu runtime
// (src/lib/llama-wgsl-runtime.ts):
//   loadLlamaWgslModel / buildGgufLlamaManifest   :184-240, :326-425
//   LlamaWgslEngine.create (buffers, K/V cache)   :669-919
//   runToken (op order per architecture)          :1025-1150
//   generateLlamaWgsl (prefix reuse, loop, tok/s) :242-314
//   reset / position / dispose                    :1011-1023, :1152-1215
//   argmax penalty list                           :1647-1665
// and src/lib/sampling.ts:9-16 (needsSamplingReadback).
//
// MI355X design: every weight matrix is repacked once into striped streams
// (device_common.h); one decode step is a fixed list of 5L+2 kernel launches
// that read the position and token from device memory, captured once into a
// hipGraph per step kind (with / without logits) and replayed. Device-driven
// generation appends sampled ids on the device and checks EOS there, so a
// whole generate call needs no per-token host round trip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../host/ggml_types.h"
#include "../host/gguf.h"
#include "../host/synth.h"
#include "chonk.h"
#include "kernels.h"
#include "prefill.h"

// Row buffers of the no-allocation prompt pass (chonk_engine_prefill_noalloc):
// one array per GPU the library runs on, held until the process ends. Host
// code never uses this name as an address: the device address comes from
// hipGetSymbolAddress, once per device (scratch_address).
constexpr size_t kNoAllocScratchBytes = (size_t)48 << 20;
constexpr int kMultiSteps = 8;  // decode steps per multi-step graph
// CHONK_MULTI=0 replays every step as its own graph
bool multi_off() {
  static const bool off = [] {
    const char* v = std::getenv("CHONK_MULTI");
    return v && v[0] == '0';
  }();
  return off;
}
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace chonk {
namespace {

thread_local std::string g_last_error;

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIP_OK(expr)                                                                               \
  do {                                                                                             \
    hipError_t e_ = (expr);                                                                        \
    if (e_ != hipSuccess)                                                                          \
      throw Error(CHONK_EHIP, std::string("HIP error ") + hipGetErrorString(e_) + " at " #expr);  \
  } while (0)

// ---- repacking GGUF blocks into stripes -------------------------------------------

struct Stripes {
  std::vector<uint8_t> s[4];
};

Stripes repack(uint32_t type, const uint8_t* raw, int64_t N, int64_t K) {
  TypeTraits t;
  if (!type_traits(type, &t) || !t.quantized) throw Error(CHONK_EINVAL, "not a GGUF quant type: " + type_name(type));
  const int64_t nb = N * (K / t.block_elems);
  Stripes st;
  auto put = [](std::vector<uint8_t>& v, const uint8_t* p, size_t n) { v.insert(v.end(), p, p + n); };
  for (int i = 0; i < 4; ++i) st.s[i].reserve((size_t)(nb * t.block_bytes));
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* p = raw + b * t.block_bytes;
    switch (type) {
      case GGML_Q4_K: put(st.s[0], p + 16, 128); put(st.s[1], p, 16); break;
      case GGML_Q5_K: put(st.s[0], p + 48, 128); put(st.s[1], p, 16); put(st.s[2], p + 16, 32); break;
      case GGML_Q6_K: put(st.s[0], p, 128); put(st.s[1], p + 128, 64); put(st.s[2], p + 192, 16); put(st.s[3], p + 208, 2); break;
      case GGML_Q8_0: put(st.s[0], p + 2, 32); put(st.s[1], p, 2); break;
      case GGML_Q5_0: put(st.s[0], p + 6, 16); put(st.s[1], p + 2, 4); put(st.s[2], p, 2); break;
      case GGML_Q5_1: put(st.s[0], p + 8, 16); put(st.s[1], p + 4, 4); put(st.s[2], p, 2); put(st.s[3], p + 2, 2); break;
      default: throw Error(CHONK_EINVAL, "unsupported GGUF tensor type " + type_name(type));
    }
  }
  return st;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Uncached device memory for cross-workgroup exchange (attention partials and
// arrival counters). Once a kernel has read such memory it is never freed:
// blocks return to a per-device free list and are reused by later engines.
class UncachedPool {
 public:
  void* take(int device, size_t bytes) {
    std::lock_guard<std::mutex> l(mu_);
    auto& fl = free_[device];
    for (size_t i = 0; i < fl.size(); ++i) {
      if (fl[i].second >= bytes) {
        void* p = fl[i].first;
        sizes_[p] = fl[i].second;
        fl.erase(fl.begin() + (long)i);
        return p;
      }
    }
    void* p = nullptr;
    HIP_OK(hipExtMallocWithFlags(&p, align256(bytes), hipDeviceMallocUncached));
    sizes_[p] = align256(bytes);
    return p;
  }
  void give_back(int device, void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> l(mu_);
    free_[device].emplace_back(p, sizes_[p]);
  }

 private:
  std::mutex mu_;
  std::map<int, std::vector<std::pair<void*, size_t>>> free_;
  std::map<void*, size_t> sizes_;
};

UncachedPool& uncached_pool() {
  static UncachedPool* pool = new UncachedPool();  // process lifetime, never destroyed
  return *pool;
}

// Device memory arena: one allocation, bump-allocated 256-byte aligned.
class Arena {
 public:
  void reserve(size_t bytes) {
    HIP_OK(hipMalloc(&base_, bytes ? bytes : 256));
    cap_ = bytes;
  }
  void* take(size_t bytes) {
    const size_t n = align256(bytes);
    if (off_ + n > cap_) throw Error(CHONK_ENOMEM, "device arena exhausted");
    void* p = (uint8_t*)base_ + off_;
    off_ += n;
    return p;
  }
  void release() {
    if (base_) (void)hipFree(base_);
    base_ = nullptr;
  }
  size_t capacity() const { return cap_; }

 private:
  void* base_ = nullptr;
  size_t cap_ = 0, off_ = 0;
};

struct DevMat {
  QMat q{};
  uint64_t gguf_bytes = 0;  // bytes of the N rows as stored in GGUF
  int ws = 0;               // GEMM weight exponent: |W| * 2^ws stays below 2^14
};

// ---- model description (buildGgufLlamaManifest) ---------------------------------

struct TensorRef {
  const GgufTensorInfo* info = nullptr;
};

struct LayerCfg {
  uint32_t theta = 10000;
  int window = 0;
  int heads = 0, kv_heads = 0, ffn = 0;  // openelm varies them per layer
  bool conv = false;                     // lfm2: a gated short-convolution layer instead of attention
  bool mamba = false;                    // granitehybrid: a Mamba2 layer instead of attention
};

struct ModelCfg {
  std::string arch;
  bool gemma = false, interleaved = false, qk_norm = false;
  bool openelm = false;  // fused attn_qkv, per-layer heads / kv heads / feed-forward width
  int gmax = 1;          // largest GQA group of any layer
  bool gpt = false;  // GGUF architecture gpt2: the reference's GPT runtime (gpt-wgsl-runtime.ts)
  bool lfm = false;  // GGUF architecture lfm2: the reference's LFM runtime (lfm-wgsl-runtime.ts)
  bool granite = false;  // GGUF architecture granitehybrid: the reference's Granite runtime (granite-wgsl-runtime.ts)
  int ssm_inner = 0, ssm_conv = 0, ssm_heads = 0;  // granitehybrid Mamba2: inner size, xBC channels, heads
  float res_scale = 0, logit_scale = 0;            // granitehybrid: residual x0.246, logits x1/3 (0: none)
  int pos_rows = 0;  // gpt2: rows of the learned position table (gpt2.context_length)
  int hidden = 0, ffn = 0, vocab = 0, layers = 0, heads = 0, kv_heads = 0, hd = 0, ctx = 0;
  float eps = 1e-5f, qk_eps = 1e-5f, scale = 0, embed_scale = 1;
  std::vector<LayerCfg> layer;
};

double meta_number(const GgufFile& g, const std::string& key, const double* fallback) {
  const GgufValue* v = g.value(key);
  if (v && v->is_number()) return v->number;
  if (fallback) return *fallback;
  throw Error(CHONK_EINVAL, "GGUF metadata " + key + " is missing or not numeric");
}

// A numeric array of metadata (ggufNumberArray, llama-wgsl-runtime.ts:474-486).
std::vector<int> meta_array(const GgufFile& g, const std::string& key) {
  const GgufValue* v = g.value(key);
  if (!v || v->type != GV_ARRAY) throw Error(CHONK_EINVAL, "GGUF metadata " + key + " is missing or not a numeric array");
  std::vector<int> out;
  for (size_t i = 0; i < v->array.size(); ++i) {
    if (!v->array[i].is_number())
      throw Error(CHONK_EINVAL, "GGUF metadata " + key + "[" + std::to_string(i) + "] is not numeric");
    out.push_back((int)v->array[i].number);
  }
  return out;
}

ModelCfg build_config(const GgufFile& g, const chonk_model_def& def) {
  ModelCfg c;
  const GgufValue* a = g.value("general.architecture");
  if (!a || a->type != GV_STRING) throw Error(CHONK_EINVAL, "GGUF metadata general.architecture is missing or not a string");
  c.arch = a->str;
  if (c.arch == "gpt2") {
    // manifestFromGguf (gpt-wgsl-runtime.ts:274-356)
    c.gpt = true;
    c.layers = (int)meta_number(g, "gpt2.block_count", nullptr);
    c.hidden = (int)meta_number(g, "gpt2.embedding_length", nullptr);
    c.ffn = (int)meta_number(g, "gpt2.feed_forward_length", nullptr);
    c.heads = (int)meta_number(g, "gpt2.attention.head_count", nullptr);
    c.pos_rows = (int)meta_number(g, "gpt2.context_length", nullptr);
    const double eps_default = 1e-5;
    c.eps = (float)meta_number(g, "gpt2.attention.layer_norm_epsilon", &eps_default);
    if (c.heads <= 0 || c.hidden % c.heads)
      throw Error(CHONK_EINVAL, "GPT WGSL: hidden " + std::to_string(c.hidden) + " is not divisible by heads");
    c.hd = c.hidden / c.heads;
    if (c.hd != 64)
      throw Error(CHONK_EINVAL, "GPT WGSL: only 64-wide GPT-2 heads are implemented, got " + std::to_string(c.hd));
    c.kv_heads = c.heads;
    const GgufTensorInfo* te = g.find("token_embd.weight");
    if (!te || te->shape.size() != 2) throw Error(CHONK_EINVAL, "GPT WGSL: missing token_embd.weight");
    c.vocab = (int)te->shape[1];
    if ((c.vocab + 255) / 256 > 256)
      throw Error(CHONK_EINVAL, "GPT WGSL argmax supports at most 65536 vocab entries, got " + std::to_string(c.vocab));
    c.ctx = std::min(def.max_context, c.pos_rows);
    c.scale = (float)(1.0 / std::sqrt((double)c.hd));  // INV_SQRT_HEAD_DIM (:1066)
    c.layer.assign(c.layers, LayerCfg{0, 0, c.heads, c.kv_heads, c.ffn});  // no rotary embedding
    if (c.layers <= 0 || c.ffn <= 0 || c.vocab <= 0 || c.ctx <= 0)
      throw Error(CHONK_EINVAL, "model has a non-positive dimension or context");
    return c;
  }
  if (c.arch == "lfm2") {
    // The LFM runtime (lfm-wgsl-runtime.ts:313-340, :457-580) fixes the
    // LFM2.5-350M shape in code; here the dimensions come from the file and the
    // constants stay the reference's: eps 1e-5 on every RMSNorm (:1567-1639,
    // :1763), rope base 1e6 with split halves (:1739-1742), three conv taps
    // (:1641-1672), the embedding as lm_head (:512-519), context = the
    // definition's maxContext (:461). A layer holding shortconv.conv.weight is
    // a convolution layer (lfm2.attention.head_count_kv is 0 there).
    c.lfm = true;
    c.layers = (int)meta_number(g, "lfm2.block_count", nullptr);
    c.hidden = (int)meta_number(g, "lfm2.embedding_length", nullptr);
    c.ffn = (int)meta_number(g, "lfm2.feed_forward_length", nullptr);
    c.heads = (int)meta_number(g, "lfm2.attention.head_count", nullptr);
    std::vector<int> lkv;
    const GgufValue* kv = g.value("lfm2.attention.head_count_kv");
    if (kv && kv->type == GV_ARRAY) {
      lkv = meta_array(g, "lfm2.attention.head_count_kv");
      if ((int)lkv.size() != c.layers)
        throw Error(CHONK_EINVAL, "LFM GGUF lfm2.attention.head_count_kv has " + std::to_string(lkv.size()) +
                                      " entries for " + std::to_string(c.layers) + " layers");
    } else {
      lkv.assign((size_t)std::max(0, c.layers), (int)meta_number(g, "lfm2.attention.head_count_kv", nullptr));
    }
    const double hd_default = std::floor((double)c.hidden / std::max(1, c.heads));
    c.hd = (int)meta_number(g, "lfm2.attention.key_length", &hd_default);
    c.vocab = def.vocab;
    c.ctx = def.max_context;
    c.eps = c.qk_eps = 1e-5f;
    c.qk_norm = true;
    c.scale = (float)(1.0 / std::sqrt((double)c.hd));
    c.kv_heads = 0;
    for (int i = 0; i < c.layers; ++i) {
      LayerCfg L;
      L.theta = 1000000;
      L.conv = g.find("blk." + std::to_string(i) + ".shortconv.conv.weight") != nullptr;
      L.heads = c.heads;
      L.kv_heads = L.conv ? c.heads : lkv[(size_t)i];  // (a convolution layer has no heads; kept valid)
      L.ffn = c.ffn;
      if (!L.conv) c.kv_heads = std::max(c.kv_heads, L.kv_heads);
      c.layer.push_back(L);
    }
    if (c.layers <= 0 || c.hidden <= 0 || c.heads <= 0 || c.ffn <= 0 || c.vocab <= 0 || c.ctx <= 0)
      throw Error(CHONK_EINVAL, "model has a non-positive dimension or context");
    if (c.kv_heads <= 0) throw Error(CHONK_EINVAL, "LFM GGUF has no attention layer");
    for (LayerCfg& L : c.layer) {
      if (L.conv) L.kv_heads = c.kv_heads;
      if (L.kv_heads <= 0 || L.heads % L.kv_heads != 0 || L.heads / L.kv_heads > 8)
        throw Error(CHONK_EINVAL, "GQA group size must divide heads and be at most 8");
      c.gmax = std::max(c.gmax, L.heads / L.kv_heads);
    }
    if (c.hd != 32 && c.hd != 64 && c.hd != 128 && c.hd != 256)
      throw Error(CHONK_EINVAL, "head_dim " + std::to_string(c.hd) + " is not supported (32, 64, 128 or 256)");
    // the convolution prologue holds a row of at most 4096 channels in registers;
    // the class-major lm_head gives each of the 256 argmax slots one workgroup
    if (c.hidden > 4096 || c.hidden % 4 != 0)
      throw Error(CHONK_EINVAL, "LFM hidden size must be a multiple of 4 and at most 4096");
    if (c.vocab > 65536)
      throw Error(CHONK_EINVAL, "LFM argmax supports at most 65536 vocab entries, got " + std::to_string(c.vocab));
    return c;
  }
  if (c.arch == "granitehybrid") {
    // The Granite runtime (granite-wgsl-runtime.ts:309-371, :526-624) fixes the
    // Granite-4.0-H-350M shape in code; here the dimensions come from the
    // tensor shapes with the same fixed SSM head width (32), state size (128),
    // 4 conv taps and head_dim 64, and the constants stay the reference's: eps
    // 1e-5, embedding x12, residual x0.246, attention scores x0.015625 without
    // rotary embedding, logits x1/3, 4096 positions. A layer holding
    // blk.N.ssm_in.weight is a Mamba2 layer (the registry's layerTypes,
    // registry.ts:48-53, list the same layers).
    c.granite = true;
    const std::string id = def.id ? def.id : "";
    const GgufValue* ft = g.value("general.file_type");
    const int file_type = ft && ft->is_number() ? (int)ft->number : -1;
    if (file_type != 7 && file_type != 15)  // validateGraniteGguf (:359-371)
      throw Error(CHONK_EINVAL, "Granite WGSL " + id + ": expected GGUF Q8_0 or Q4_K_M file_type, got " +
                                    std::to_string(file_type));
    for (const char* name : {"token_embd.weight", "output_norm.weight", "blk.0.attn_norm.weight"})
      if (!g.find(name)) throw Error(CHONK_EINVAL, "Granite WGSL " + id + ": GGUF missing tensor " + name);
    for (const GgufTensorInfo& t : g.tensors)  // dtypeForGgmlType (:373-390)
      if (t.type != GGML_F32 && t.type != GGML_F16 && t.type != GGML_Q8_0 && t.type != GGML_Q4_K &&
          t.type != GGML_Q6_K)
        throw Error(CHONK_EINVAL, "Granite WGSL unsupported GGML tensor type " + type_name(t.type));
    const GgufTensorInfo* te = g.find("token_embd.weight");
    if (te->shape.size() != 2) throw Error(CHONK_EINVAL, "Granite WGSL tensor token_embd.weight is not a matrix");
    c.hidden = (int)te->shape[0];
    c.vocab = (int)te->shape[1];
    int nl = 0;
    while (g.find("blk." + std::to_string(nl) + ".attn_norm.weight")) ++nl;
    c.layers = nl;
    c.hd = 64;
    c.ctx = 4096;
    c.eps = c.qk_eps = 1e-5f;
    c.scale = 0.015625f;
    c.embed_scale = 12.0f;
    c.res_scale = 0.246f;
    c.logit_scale = (float)0.3333333333333333;
    c.heads = c.kv_heads = c.ffn = 0;
    auto rows = [&](const std::string& name) -> int {
      const GgufTensorInfo* t = g.find(name);
      if (!t || t->shape.size() != 2) throw Error(CHONK_EINVAL, "Granite WGSL manifest missing tensor " + name);
      return (int)t->shape[1];
    };
    for (int i = 0; i < nl; ++i) {
      const std::string p = "blk." + std::to_string(i) + ".";
      LayerCfg L;
      L.theta = 0;  // STORE_KV_WGSL stores k as projected: no rotary embedding
      L.mamba = g.find(p + "ssm_in.weight") != nullptr;
      L.ffn = rows(p + "ffn_gate.weight");
      c.ffn = std::max(c.ffn, L.ffn);
      if (L.mamba) {
        // the inner size is out_proj's row length
        const GgufTensorInfo* so = g.find(p + "ssm_out.weight");
        if (!so || so->shape.size() != 2)
          throw Error(CHONK_EINVAL, "Granite WGSL manifest missing tensor " + p + "ssm_out.weight");
        const int inner = (int)so->shape[0];
        if (c.ssm_inner && inner != c.ssm_inner)
          throw Error(CHONK_EINVAL, "Granite WGSL: the SSM inner size differs between layers");
        c.ssm_inner = inner;
      } else {
        L.heads = rows(p + "attn_q.weight") / c.hd;
        L.kv_heads = rows(p + "attn_k.weight") / c.hd;
        c.heads = std::max(c.heads, L.heads);
        c.kv_heads = std::max(c.kv_heads, L.kv_heads);
      }
      c.layer.push_back(L);
    }
    if (c.layers <= 0 || c.hidden <= 0 || c.ffn <= 0 || c.vocab <= 0)
      throw Error(CHONK_EINVAL, "model has a non-positive dimension or context");
    if (c.kv_heads <= 0) throw Error(CHONK_EINVAL, "Granite WGSL GGUF has no attention layer");
    for (LayerCfg& L : c.layer) {
      if (L.mamba) {  // (kept valid for the attention geometry; a Mamba2 layer has no heads)
        L.heads = c.heads;
        L.kv_heads = c.kv_heads;
      }
      if (L.kv_heads <= 0 || L.heads % L.kv_heads != 0 || L.heads / L.kv_heads > 8)
        throw Error(CHONK_EINVAL, "GQA group size must divide heads and be at most 8");
      c.gmax = std::max(c.gmax, L.heads / L.kv_heads);
    }
    if (c.ssm_inner) {
      // the Mamba2 kernel's geometry: 32-wide heads, 128 states, one group
      if (c.ssm_inner % 32 != 0 || c.ssm_inner > 4096)
        throw Error(CHONK_EINVAL, "Granite WGSL: the SSM inner size must be a multiple of 32 and at most 4096");
      c.ssm_heads = c.ssm_inner / 32;
      c.ssm_conv = c.ssm_inner + 2 * 128;
    }
    if (c.hidden > 4096 || c.hidden % 32 != 0)
      throw Error(CHONK_EINVAL, "Granite WGSL hidden size must be a multiple of 32 and at most 4096");
    // the class-major lm_head: one workgroup per residue class of at most 512 ids
    if (c.vocab > 131072)
      throw Error(CHONK_EINVAL, "Granite WGSL argmax supports at most 131072 vocab entries, got " + std::to_string(c.vocab));
    return c;
  }
  if (c.arch != "qwen3" && c.arch != "llama" && c.arch != "gemma3" && c.arch != "openelm")
    throw Error(CHONK_EINVAL, "Llama GGUF WGSL does not support architecture " + c.arch);
  c.gemma = c.arch == "gemma3";
  c.openelm = c.arch == "openelm";
  c.interleaved = c.arch == "llama";
  const std::string p = c.arch + ".";
  c.layers = (int)meta_number(g, p + "block_count", nullptr);
  c.hidden = (int)meta_number(g, p + "embedding_length", nullptr);
  // openelm: per-layer arrays, the scalars are their maxima (buildGgufLlamaManifest, :373-380)
  std::vector<int> lh, lkv, lff;
  if (c.openelm) {
    lh = meta_array(g, p + "attention.head_count");
    lkv = meta_array(g, p + "attention.head_count_kv");
    lff = meta_array(g, p + "feed_forward_length");
    if (lh.empty() || lkv.empty() || lff.empty()) throw Error(CHONK_EINVAL, "openelm per-layer metadata arrays are empty");
    c.heads = *std::max_element(lh.begin(), lh.end());
    c.kv_heads = *std::max_element(lkv.begin(), lkv.end());
    c.ffn = *std::max_element(lff.begin(), lff.end());
  } else {
    c.heads = (int)meta_number(g, p + "attention.head_count", nullptr);
    c.kv_heads = (int)meta_number(g, p + "attention.head_count_kv", nullptr);
    c.ffn = (int)meta_number(g, p + "feed_forward_length", nullptr);
  }
  const double hd_default = std::floor((double)c.hidden / std::max(1, c.heads));
  c.hd = (int)meta_number(g, p + "attention.key_length", &hd_default);
  c.vocab = def.vocab;
  const double ctx_default = def.max_context;
  const int gguf_ctx = (int)meta_number(g, p + "context_length", &ctx_default);
  c.ctx = std::min(def.max_context, std::min(def.max_context, gguf_ctx));
  const double eps_default = 1e-5;
  c.eps = (float)meta_number(g, p + "attention.layer_norm_rms_epsilon", &eps_default);
  c.qk_eps = c.eps;
  c.qk_norm = g.find("blk.0.attn_q_norm.weight") && g.find("blk.0.attn_k_norm.weight");
  c.scale = (float)(1.0 / std::sqrt((double)c.hd));
  c.embed_scale = c.gemma ? (float)std::sqrt((double)c.hidden) : 1.0f;
  const double theta_default = 10000, gtheta_default = 1000000, win_default = 0;
  const double theta = c.gemma ? 10000.0 : meta_number(g, p + "rope.freq_base", &theta_default);
  const double gtheta = c.gemma ? meta_number(g, "gemma3.rope.freq_base", &gtheta_default) : 0;
  const int window = c.gemma ? (int)meta_number(g, "gemma3.attention.sliding_window", &win_default) : 0;
  // validateLayerArray (:1815-1821)
  for (const auto* v : {&lh, &lkv, &lff})
    if (c.openelm && (int)v->size() != c.layers)
      throw Error(CHONK_EINVAL, "Llama WGSL manifest layer array length " + std::to_string(v->size()) + " != layers " +
                                    std::to_string(c.layers));
  for (int i = 0; i < c.layers; ++i) {
    LayerCfg L;
    const double th = c.gemma ? (i % 6 == 5 ? gtheta : 10000.0) : theta;
    L.theta = (uint32_t)std::llround(th);
    L.window = c.gemma ? (i % 6 == 5 ? 0 : window) : 0;
    L.heads = c.openelm ? lh[(size_t)i] : c.heads;
    L.kv_heads = c.openelm ? lkv[(size_t)i] : c.kv_heads;
    L.ffn = c.openelm ? lff[(size_t)i] : c.ffn;
    c.layer.push_back(L);
  }
  // limits of this engine's kernels
  if (c.layers <= 0 || c.hidden <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.ffn <= 0 || c.vocab <= 0 || c.ctx <= 0)
    throw Error(CHONK_EINVAL, "model has a non-positive dimension or context");
  for (const LayerCfg& L : c.layer) {
    if (L.heads <= 0 || L.kv_heads <= 0 || L.ffn <= 0)
      throw Error(CHONK_EINVAL, "model has a non-positive dimension or context");
    if (L.heads % L.kv_heads != 0 || L.heads / L.kv_heads > 8)
      throw Error(CHONK_EINVAL, "GQA group size must divide heads and be at most 8");
    c.gmax = std::max(c.gmax, L.heads / L.kv_heads);
  }
  // the packed q|k|v path normalises q and k (llama-wgsl-runtime.ts:1071-1084)
  if (c.openelm && !c.qk_norm) throw Error(CHONK_EINVAL, "Llama WGSL layer is missing attention projection weights");
  if (c.hd != 32 && c.hd != 64 && c.hd != 128 && c.hd != 256)
    throw Error(CHONK_EINVAL, "head_dim " + std::to_string(c.hd) + " is not supported (32, 64, 128 or 256)");
  if ((c.vocab + 255) / 256 > 4096) throw Error(CHONK_EINVAL, "vocab above 1048576 is not supported");
  if (c.gemma && !c.qk_norm) throw Error(CHONK_EINVAL, "Gemma WGSL layer is missing required weights");
  return c;
}

// ---- the engine ------------------------------------------------------------------

struct LayerDev {
  DevMat q, k, v, o, gate, up, down;
  DevMat conv_in, conv_out;  // lfm2 convolution layer: in_proj (rows B | C | x) and out_proj
  float* conv_w = nullptr;   // [hidden][3] taps
  float *conv_s1 = nullptr, *conv_s2 = nullptr;  // B * x two positions and one position back
  DevMat qkv;  // gpt2: fused q|k|v
  // granitehybrid Mamba2 layer: in_proj (rows z | xBC | dt), out_proj, conv taps
  // [conv][4] and bias, per-head dt bias / A / D, gated-norm weight; state
  DevMat ssm_in, ssm_out;
  float *c1d_w = nullptr, *c1d_b = nullptr, *dt_b = nullptr, *a_neg = nullptr, *d_w = nullptr, *ssm_norm = nullptr;
  float *ssm_state = nullptr, *mconv_state = nullptr;  // [heads][32][128], [2][conv][3]
  // gpt2: LayerNorm biases (in_norm / post_norm hold the weights) and linear biases
  float *in_norm_b = nullptr, *post_norm_b = nullptr, *qkv_b = nullptr, *o_b = nullptr, *up_b = nullptr,
        *down_b = nullptr;
  float *in_norm = nullptr, *post_norm = nullptr, *pre_ffn_norm = nullptr, *post_ffn_norm = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr;
  void *kc = nullptr, *vc = nullptr;
};

struct Launch {
  // QKVATTN: the q|k|v matvec (mv, nq workgroups) and the decode attention (at)
  // in one launch (k_qkv_attn)
  enum Kind { MV, ATTN, SEL, SSM, QKVATTN } kind = MV;
  MvArgs mv{};
  SsmArgs ssm{};
  AttnArgs at{};
  SelArgs sel{};
  int grid = 0;
  int nq = 0;  // QKVATTN: the matvec's workgroups, ahead of the attention's
  size_t shmem = 0;
  std::string name;
  uint64_t weight_bytes = 0;  // GGUF weight bytes read (matvec)
  int layer = -1;
};

}  // namespace
}  // namespace chonk

using namespace chonk;

struct chonk_engine {
  chonk_model_def def{};
  std::string model_id;
  std::vector<int32_t> eos;
  ModelCfg cfg;
  int device = 0;
  hipStream_t stream = nullptr;
  Arena weights, state;
  std::vector<LayerDev> layers;
  DevMat embed, lm_head;
  DevMat lm_lanes;  // the lm_head's lane-interleaved copy (k_lm_lanes); s0 null when absent
  float* final_norm = nullptr;
  float *final_norm_b = nullptr, *pos_embd = nullptr;  // gpt2: final LayerNorm bias, position table
  size_t kv_elem = 2;
  // activations
  float *resA = nullptr, *resB = nullptr, *delta = nullptr, *qkv = nullptr, *attn = nullptr, *ff = nullptr,
        *logits = nullptr, *part = nullptr;
  float* conv_proj = nullptr;  // lfm2: [3 * hidden] in_proj output of the current convolution layer
  float *mproj = nullptr, *my = nullptr;  // granitehybrid: Mamba2 in_proj output, scan output
  Candidate* cand = nullptr;
  uint32_t* cnt = nullptr;
  void* uncached = nullptr;       // part + cnt, from the uncached pool
  bool use_graph = true;
  DevState* st = nullptr;
  DevSampling* samp = nullptr;
  int32_t *hist = nullptr, *gen = nullptr;
  uint32_t *pen_bits = nullptr, *seen_bits = nullptr;
  int groups = 0, chunk = 0, nchunk = 0;
  bool dec_attn = false;          // per-phase attention: k_attn_dec over dnchunk chunks
  int dnchunk = 0;                // workgroup chunks of dsub x 64 positions
  int dsub = 1;
  tagged_t* dpart = nullptr;      // k_attn_dec chunk rows
  // the q|k|v matvec inside the attention launch (k_qkv_attn): its rows as
  // tagged words, [heads * hd | kv_heads * hd | kv_heads * hd]
  bool fuse_qkv = false;
  tagged_t* qkv_tag = nullptr;
  std::vector<std::pair<uint32_t, float*>> rope_tables;  // theta -> [hd/2] inverse frequencies
  std::vector<std::pair<uint32_t, float2*>> rope_cs;     // theta -> [ctx][hd/2] (cos, sin)
  // per-phase kernels of one step (qkv, attn, oproj, gateup, down per layer; lm_head, select)
  std::vector<Launch> kernels_logits, kernels_plain;
  // what a step replays (captured as one graph each)
  std::vector<Launch> step_logits, step_plain;
  hipGraph_t graph_logits = nullptr, graph_plain = nullptr;
  hipGraphExec_t exec_logits = nullptr, exec_plain = nullptr;
  // the same steps with the q|k|v matvec and the attention as separate launches:
  // what the engine replays while another engine lives on its device (fuse_qkv)
  std::vector<Launch> step_logits_sep, step_plain_sep;
  hipGraph_t graph_logits_sep = nullptr, graph_plain_sep = nullptr;
  hipGraphExec_t exec_logits_sep = nullptr, exec_plain_sep = nullptr;
  // kMultiSteps logits steps in one graph: what runs of consecutive steps with
  // no host work between them replay (one launch gap per kMultiSteps tokens)
  hipGraph_t graph_multi = nullptr;
  hipGraphExec_t exec_multi = nullptr;
  bool registered = false;  // counted in device_engines()
  // pinned host staging
  DevState* h_state = nullptr;
  int32_t* h_tok = nullptr;
  DevSampling* h_samp = nullptr;
  DevSampling last_samp{};
  bool samp_valid = false;
  // host mirror of the conversation
  int pos = 0;
  int known_token_pos = -1;  // position whose history slot the device already holds
  int32_t known_token = 0;
  bool logits_valid = false;
  std::vector<int32_t> cached_ids;
  bool has_cached_next = false;
  int32_t cached_next = 0;
  uint64_t weight_bytes_per_token = 0;
  // batched prompt processing: row buffers allocated on first use
  bool batched_prefill = true;
  uint8_t* scratch = nullptr;  // device address of this GPU's no-allocation prompt-pass scratch
  int noalloc_rows = 0;        // rows one chonk_engine_prefill_noalloc call may take (0: none)
  void* pf_mem = nullptr;
  float *pf_x = nullptr, *pf_qkv = nullptr, *pf_att = nullptr, *pf_g = nullptr, *pf_u = nullptr, *pf_act = nullptr,
        *pf_d = nullptr, *pf_xscale = nullptr, *pf_part = nullptr;
  _Float16 *pf_h = nullptr, *pf_l = nullptr;
  int32_t* pf_tok = nullptr;
  // status
  std::atomic<bool> busy{false};
  bool lost = false;
  bool fail_next_launch = false;  // test hook: the next launch reports a HIP error
  void* flush = nullptr;          // benchmark: buffer written between cold launches
  size_t flush_bytes = 0;
  std::string err;
};

namespace chonk {
namespace {

struct Guard {
  chonk_engine* e;
  explicit Guard(chonk_engine* eng) : e(eng) {
    bool expected = false;
    if (!e->busy.compare_exchange_strong(expected, true))
      throw Error(CHONK_EBUSY, "engine call already in progress");
    if (e->lost) {
      e->busy = false;
      throw Error(CHONK_ELOST, "engine lost after an earlier device error: " + e->err);
    }
    (void)hipSetDevice(e->device);
  }
  ~Guard() { e->busy = false; }
};

template <typename F>
int api(chonk_engine* e, F&& f) {
  try {
    if (!e) throw Error(CHONK_EINVAL, "null engine");
    Guard g(e);
    try {
      f();
    } catch (const Error& x) {
      if (x.code == CHONK_EHIP) e->lost = true;
      throw;
    }
    return CHONK_OK;
  } catch (const Error& x) {
    g_last_error = x.what();
    if (e && x.code != CHONK_EBUSY) e->err = x.what();
    return x.code;
  } catch (const std::exception& x) {
    g_last_error = x.what();
    if (e) e->err = x.what();
    return CHONK_EINVAL;
  }
}

template <typename F>
int api_free(F&& f) {
  try {
    f();
    return CHONK_OK;
  } catch (const Error& x) {
    g_last_error = x.what();
    return x.code;
  } catch (const std::exception& x) {
    g_last_error = x.what();
    return CHONK_EIO;
  }
}

const GgufTensorInfo& tensor(const GgufFile& g, const std::string& name) {
  const GgufTensorInfo* t = g.find(name);
  if (!t) throw Error(CHONK_EINVAL, "Llama WGSL manifest missing tensor " + name);
  return *t;
}

std::vector<uint8_t> read_tensor(const ByteSource& src, const GgufFile& g, const GgufTensorInfo& t) {
  std::vector<uint8_t> raw((size_t)t.n_bytes);
  try {
    src.read(g.data_offset + t.offset, t.n_bytes, raw.data());
  } catch (const std::exception& e) {
    throw Error(CHONK_EIO, e.what());
  }
  return raw;
}

// Size of the stripes of an N x K matrix of `type`.
size_t stripes_bytes(uint32_t type, int64_t N, int64_t K) {
  TypeTraits t;
  type_traits(type, &t);
  const size_t nb = (size_t)(N * (K / t.block_elems));
  switch (type) {
    case GGML_Q4_K: return align256(nb * 128) + align256(nb * 16);
    case GGML_Q5_K: return align256(nb * 128) + align256(nb * 16) + align256(nb * 32);
    case GGML_Q6_K: return align256(nb * 128) + align256(nb * 64) + align256(nb * 16) + align256(nb * 2);
    case GGML_Q8_0: return align256(nb * 32) + align256(nb * 2);
    case GGML_Q5_0: return align256(nb * 16) + align256(nb * 4) + align256(nb * 2);
    case GGML_Q5_1: return align256(nb * 16) + align256(nb * 4) + align256(nb * 2) + align256(nb * 2);
  }
  return 0;
}

void check_matrix(const GgufTensorInfo& t, int64_t K, int64_t N) {
  TypeTraits tt;
  if (!type_traits(t.type, &tt) || !tt.quantized)
    throw Error(CHONK_EINVAL, "Llama WGSL tensor " + t.name + " is not a supported GGUF quantized tensor");
  if (K % tt.block_elems != 0 || K % 32 != 0)
    throw Error(CHONK_EINVAL, "tensor " + t.name + " row length " + std::to_string(K) + " is not a multiple of its " +
                                  std::to_string(tt.block_elems) + "-element block");
  if (t.shape.empty() || (int64_t)t.shape[0] != K)
    throw Error(CHONK_EINVAL, "tensor " + t.name + " row length does not match the model (" + std::to_string(K) + ")");
  if ((int64_t)(t.n_elements / t.shape[0]) < N)
    throw Error(CHONK_EINVAL, "tensor " + t.name + " has fewer than " + std::to_string(N) + " rows");
  if (K > 32768) throw Error(CHONK_EINVAL, "tensor " + t.name + " row length above 32768 is not supported");
}

// Power of two that brings every dequantized weight of the tensor below 2^14
// (bound from the blocks' fp16 scales), so that the GEMM's fp16 hi/lo split of
// W * 2^ws neither overflows nor loses the low half to subnormals.
int weight_exponent(uint32_t type, const uint8_t* raw, size_t n_blocks, size_t block_bytes) {
  auto h = [&](size_t b, size_t off) {
    uint16_t v;
    std::memcpy(&v, raw + b * block_bytes + off, 2);
    return std::fabs(f16_to_f32(v));
  };
  double bound = 0;
  for (size_t b = 0; b < n_blocks; ++b) {
    double v = 0;
    switch (type) {
      case GGML_Q4_K: v = 63.0 * 15 * h(b, 0) + 63.0 * h(b, 2); break;
      case GGML_Q5_K: v = 63.0 * 31 * h(b, 0) + 63.0 * h(b, 2); break;
      case GGML_Q6_K: v = 128.0 * 32 * h(b, 208); break;
      case GGML_Q8_0: v = 128.0 * h(b, 0); break;
      case GGML_Q5_0: v = 16.0 * h(b, 0); break;
      case GGML_Q5_1: v = 31.0 * h(b, 0) + h(b, 2); break;
      default: break;
    }
    if (std::isfinite(v)) bound = std::max(bound, v);
  }
  if (!(bound > 0)) return 0;
  return std::max(-30, std::min(30, (int)std::floor(std::log2(16384.0 / bound))));
}

DevMat upload_matrix(Arena& arena, const ByteSource& src, const GgufFile& g, const GgufTensorInfo& t, int64_t K,
                     int64_t N) {
  check_matrix(t, K, N);
  std::vector<uint8_t> raw = read_tensor(src, g, t);
  TypeTraits tt;
  type_traits(t.type, &tt);
  const Stripes st = repack(t.type, raw.data(), N, K);
  DevMat m;
  m.q.type = (int32_t)t.type;
  m.q.n = (int32_t)N;
  m.q.k = (int32_t)K;
  const uint8_t** dst[4] = {&m.q.s0, &m.q.s1, &m.q.s2, &m.q.s3};
  for (int i = 0; i < 4; ++i) {
    if (st.s[i].empty()) continue;
    void* p = arena.take(st.s[i].size());
    HIP_OK(hipMemcpy(p, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
    *dst[i] = (const uint8_t*)p;
  }
  m.gguf_bytes = (uint64_t)(N * (K / tt.block_elems)) * tt.block_bytes;
  m.ws = weight_exponent(t.type, raw.data(), (size_t)(N * (K / tt.block_elems)), tt.block_bytes);
  return m;
}

float* upload_floats(Arena& arena, const ByteSource& src, const GgufFile& g, const std::string& name, int64_t n) {
  const GgufTensorInfo& t = tensor(g, name);
  if (t.type != GGML_F32 && t.type != GGML_F16)
    throw Error(CHONK_EINVAL, "Llama WGSL tensor " + name + " is " + type_name(t.type) + ", expected float32/float16");
  if ((int64_t)t.n_elements < n) throw Error(CHONK_EINVAL, "tensor " + name + " is shorter than " + std::to_string(n));
  std::vector<uint8_t> raw = read_tensor(src, g, t);
  std::vector<float> f((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    if (t.type == GGML_F32) {
      std::memcpy(&f[i], raw.data() + 4 * i, 4);
    } else {
      uint16_t h;
      std::memcpy(&h, raw.data() + 2 * i, 2);
      f[i] = f16_to_f32(h);
    }
  }
  float* p = (float*)arena.take((size_t)n * 4);
  HIP_OK(hipMemcpy(p, f.data(), (size_t)n * 4, hipMemcpyHostToDevice));
  return p;
}

// The LFM loader's checks (lfm-wgsl-runtime.ts:313-431): a missing tensor, a
// linear tensor that is not Q8_0 / Q4_K / Q6_K, a float tensor that is not
// F32 / F16, each with the reference's wording.
const GgufTensorInfo& lfm_tensor(const GgufFile& g, const std::string& name) {
  const GgufTensorInfo* t = g.find(name);
  if (!t) throw Error(CHONK_EINVAL, "LFM GGUF missing tensor " + name);
  return *t;
}

const GgufTensorInfo& lfm_linear(const GgufFile& g, const std::string& name) {
  const GgufTensorInfo& t = lfm_tensor(g, name);
  if (t.type != GGML_Q8_0 && t.type != GGML_Q4_K && t.type != GGML_Q6_K)
    throw Error(CHONK_EINVAL, "unsupported LFM GGUF linear tensor " + name + ": " + type_name(t.type));
  return t;
}

float* lfm_floats(Arena& arena, const ByteSource& src, const GgufFile& g, const std::string& name, int64_t n) {
  const GgufTensorInfo& t = lfm_tensor(g, name);
  if (t.type != GGML_F32 && t.type != GGML_F16)
    throw Error(CHONK_EINVAL, "LFM GGUF tensor " + name + " is " + type_name(t.type) + ", expected F32/F16");
  return upload_floats(arena, src, g, name, n);
}

// The Granite loader's checks (granite-wgsl-runtime.ts:397-491) with its
// wording: a missing tensor, a linear tensor that is not a quantized matrix of
// shape [k, n], a float tensor that is not F32 / F16.
const GgufTensorInfo& granite_tensor(const GgufFile& g, const std::string& name) {
  const GgufTensorInfo* t = g.find(name);
  if (!t) throw Error(CHONK_EINVAL, "Granite WGSL manifest missing tensor " + name);
  return *t;
}
const GgufTensorInfo& granite_linear(const GgufFile& g, const std::string& name, int64_t K, int64_t N) {
  const GgufTensorInfo& t = granite_tensor(g, name);
  if (t.type != GGML_Q8_0 && t.type != GGML_Q4_K && t.type != GGML_Q6_K)
    throw Error(CHONK_EINVAL, "Granite WGSL tensor " + name + " is " + type_name(t.type) +
                                  ", expected a GGUF quantized matrix");
  if (t.shape.size() != 2 || (int64_t)t.shape[0] != K || (int64_t)t.shape[1] != N) {
    std::string got;
    for (size_t i = 0; i < t.shape.size(); ++i) got += (i ? ", " : "") + std::to_string(t.shape[i]);
    throw Error(CHONK_EINVAL, "Granite WGSL tensor " + name + " shape [" + got + "], expected [" + std::to_string(K) +
                                  ", " + std::to_string(N) + "]");
  }
  return t;
}
float* granite_floats(Arena& arena, const ByteSource& src, const GgufFile& g, const std::string& name, int64_t n) {
  const GgufTensorInfo& t = granite_tensor(g, name);
  if (t.type != GGML_F32 && t.type != GGML_F16)
    throw Error(CHONK_EINVAL, "Granite WGSL tensor " + name + " is " + type_name(t.type) + ", expected float32/float16");
  return upload_floats(arena, src, g, name, n);
}

// Rows of the class-major lm_head copy: 256 classes (id mod 256) of
// ceil(V / 256) rows each.
int64_t class_rows(int64_t V) { return 256 * ((V + 255) / 256); }

// The vocab x K matrix `t` stored class-major for the lm_head: physical row
// c * R + j holds id j * 256 + c (R = ceil(V / 256); rows past V are zero
// blocks, which decode to 0), so that one workgroup of R rows sees one
// residue class in id order (TOPK256_WGSL's slot, lfm-wgsl-runtime.ts:1925-1947).
DevMat upload_class_major(Arena& arena, const ByteSource& src, const GgufFile& g, const GgufTensorInfo& t,
                          int64_t K, int64_t V) {
  check_matrix(t, K, V);
  std::vector<uint8_t> raw = read_tensor(src, g, t);
  TypeTraits tt;
  type_traits(t.type, &tt);
  const size_t row_bytes = (size_t)(K / tt.block_elems) * tt.block_bytes;
  const int64_t R = (V + 255) / 256, N = 256 * R;
  std::vector<uint8_t> perm((size_t)N * row_bytes, 0);
  for (int64_t c = 0; c < 256; ++c)
    for (int64_t j = 0; j < R; ++j) {
      const int64_t id = j * 256 + c;
      if (id < V) std::memcpy(perm.data() + (size_t)(c * R + j) * row_bytes, raw.data() + (size_t)id * row_bytes, row_bytes);
    }
  const Stripes st = repack(t.type, perm.data(), N, K);
  DevMat m;
  m.q.type = (int32_t)t.type;
  m.q.n = (int32_t)N;
  m.q.k = (int32_t)K;
  const uint8_t** dst[4] = {&m.q.s0, &m.q.s1, &m.q.s2, &m.q.s3};
  for (int i = 0; i < 4; ++i) {
    if (st.s[i].empty()) continue;
    void* p = arena.take(st.s[i].size());
    HIP_OK(hipMemcpy(p, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
    *dst[i] = (const uint8_t*)p;
  }
  m.gguf_bytes = (uint64_t)V * row_bytes;
  return m;
}

// The lm_head's lane-interleaved copy (qdot.h, load_lane_unit): rows in blocks of
// 64, the fragments of one unit of the block's 64 rows side by side in each
// stream, so that k_lm_lanes (one row per lane) reads every unit of a wave as
// one contiguous run. Rows past N (up to a multiple of 256, the rows of a
// k_lm_lanes workgroup) are zero blocks (they decode to 0). The bytes
// per stream are those of the striped layout of the padded matrix.
bool lane_layout_type(uint32_t type) { return type == GGML_Q4_K || type == GGML_Q6_K || type == GGML_Q8_0; }
int64_t lane_rows(int64_t N) { return 256 * ((N + 255) / 256); }  // whole k_lm_lanes workgroups

DevMat upload_lanes(Arena& arena, const ByteSource& src, const GgufFile& g, const GgufTensorInfo& t, int64_t K,
                    int64_t N) {
  check_matrix(t, K, N);
  if (!lane_layout_type(t.type)) throw Error(CHONK_EINVAL, "no lane-interleaved layout for " + type_name(t.type));
  std::vector<uint8_t> raw = read_tensor(src, g, t);
  TypeTraits tt;
  type_traits(t.type, &tt);
  const size_t row_bytes = (size_t)(K / tt.block_elems) * tt.block_bytes;
  const int64_t NP = lane_rows(N), U = K / 32, SB = K / 256;
  const size_t nb = (size_t)(NP * (K / tt.block_elems));
  Stripes st;
  switch (t.type) {
    case GGML_Q6_K: st.s[0].assign(nb * 128, 0); st.s[1].assign(nb * 64, 0); st.s[2].assign(nb * 16, 0); st.s[3].assign(nb * 2, 0); break;
    case GGML_Q8_0: st.s[0].assign(nb * 32, 0); st.s[1].assign(nb * 2, 0); break;
    default: st.s[0].assign(nb * 128, 0); st.s[1].assign(nb * 16, 0); break;  // Q4_K
  }
  for (int64_t r = 0; r < N; ++r) {
    const uint8_t* row = raw.data() + (size_t)r * row_bytes;
    const int64_t blk = r >> 6, lane = r & 63;
    auto ui = [&](int64_t u) { return (size_t)((blk * U + u) * 64 + lane); };
    auto sj = [&](int64_t sb) { return (size_t)((blk * SB + sb) * 64 + lane); };
    if (t.type == GGML_Q8_0) {
      for (int64_t u = 0; u < U; ++u) {
        const uint8_t* p = row + 34 * u;
        std::memcpy(st.s[0].data() + 32 * ui(u), p + 2, 32);
        std::memcpy(st.s[1].data() + 2 * ui(u), p, 2);
      }
      continue;
    }
    for (int64_t sb = 0; sb < SB; ++sb) {
      const uint8_t* p = row + (size_t)sb * tt.block_bytes;
      if (t.type == GGML_Q6_K) {
        // unit c of the super-block: half h = c / 4, run b = c % 4 (load_unit<Q6_K>)
        for (int c = 0; c < 8; ++c) {
          const int h = c >> 2, b = c & 3;
          const size_t i = ui(8 * sb + c);
          std::memcpy(st.s[0].data() + 16 * i, p + 64 * h + 8 * b, 8);
          std::memcpy(st.s[0].data() + 16 * i + 8, p + 64 * h + 32 + 8 * b, 8);
          std::memcpy(st.s[1].data() + 8 * i, p + 128 + 32 * h + 8 * b, 8);
        }
        std::memcpy(st.s[2].data() + 16 * sj(sb), p + 192, 16);
        std::memcpy(st.s[3].data() + 2 * sj(sb), p + 208, 2);
      } else {  // Q4_K: header (d, dmin, scales) then 128 bytes of nibbles, 16 per unit
        for (int c = 0; c < 8; ++c) std::memcpy(st.s[0].data() + 16 * ui(8 * sb + c), p + 16 + 16 * c, 16);
        std::memcpy(st.s[1].data() + 16 * sj(sb), p, 16);
      }
    }
  }
  DevMat m;
  m.q.type = (int32_t)t.type;
  m.q.n = (int32_t)NP;
  m.q.k = (int32_t)K;
  const uint8_t** dst[4] = {&m.q.s0, &m.q.s1, &m.q.s2, &m.q.s3};
  for (int i = 0; i < 4; ++i) {
    if (st.s[i].empty()) continue;
    void* ptr = arena.take(st.s[i].size());
    HIP_OK(hipMemcpy(ptr, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
    *dst[i] = (const uint8_t*)ptr;
  }
  m.gguf_bytes = (uint64_t)N * row_bytes;
  return m;
}

// Device address of `scratch` on `device`, looked up once per device with
// that device current (the caller has made it current).
uint8_t* scratch_address(int device) {
  static std::mutex* mu = new std::mutex();
  static std::map<int, uint8_t*>* addr = new std::map<int, uint8_t*>();
  std::lock_guard<std::mutex> l(*mu);
  auto it = addr->find(device);
  if (it != addr->end()) return it->second;
  void* p = nullptr;
  HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  if (!p) throw Error(CHONK_EHIP, "hipGetSymbolAddress returned no address for the prompt-pass scratch");
  (*addr)[device] = (uint8_t*)p;
  return (uint8_t*)p;
}

// Serializes the no-allocation prompt passes on one GPU: every engine on the
// device shares that device's scratch array.
std::mutex& scratch_lock(int device) {
  static std::mutex* mu = new std::mutex();
  static std::map<int, std::unique_ptr<std::mutex>>* locks = new std::map<int, std::unique_ptr<std::mutex>>();
  std::lock_guard<std::mutex> l(*mu);
  std::unique_ptr<std::mutex>& m = (*locks)[device];
  if (!m) m.reset(new std::mutex());
  return *m;
}

// Rows of one no-allocation prompt pass for this model (defined with the row buffers).
int noalloc_rows_for(const ModelCfg& c);

int target_wgs() { return 512; }

// Fills seg geometry for n_out output rows of matrix w (glu: gate/up pairs).
void plan_seg(MvSeg& sg, const QMat& w, int n_out, bool glu, int wg_begin) {
  sg.w = w;
  sg.n_out = n_out;
  sg.lpr = pick_lpr(w.k / 32);
  const int ng = kWg / sg.lpr;
  const int per_pass = glu ? ng / 2 : ng;
  const int passes = std::max(1, (n_out + per_pass * target_wgs() - 1) / (per_pass * target_wgs()));
  sg.tile = per_pass * passes;
  sg.wg_begin = wg_begin;
}

int seg_wgs(const MvSeg& sg) { return (sg.n_out + sg.tile - 1) / sg.tile; }

// Geometry of the one-row-per-lane-group matvec (k_mvr_*): the smallest lane
// count that keeps a lane at <= `units` units, widened (up to a wave) while the
// segment has fewer than `min_wgs` workgroups.
void plan_seg_row(MvSeg& sg, int wg_begin, int units, int min_wgs) {
  const int U = sg.w.k / 32;
  int lpr = 4;
  while (lpr < 64 && (U + lpr - 1) / lpr > units) lpr *= 2;
  while (lpr < 64 && (sg.n_out + kWg / lpr - 1) / (kWg / lpr) < min_wgs) lpr *= 2;
  sg.lpr = lpr;
  sg.tile = kWg / lpr;
  sg.wg_begin = wg_begin;
}

// Moves a decode-step matvec onto the row kernels when its shape allows
// (CHONK_MV=generic keeps every launch on the generic kernels).
void use_row_kernel(MvArgs& a) {
  static const bool off = [] {
    const char* v = std::getenv("CHONK_MV");
    return v && std::string(v) == "generic";
  }();
  // GPT-2's prologues and epilogues (LayerNorm, biases, GELU, clamped residual)
  // exist only in the row kernels
  bool needs_row = a.epi == EPI_GELU || a.pro == PRO_LN || a.pro == PRO_EMBED_LN || a.sanitize;
  // (so are the lfm2 convolution prologue and state shift)
  needs_row = needs_row || a.pro == PRO_CONV || a.conv_commit;
  for (int i = 0; i < a.nseg; ++i) needs_row = needs_row || a.seg[i].bias;
  if ((off && !needs_row) || a.epi == EPI_LOGITS) return;
  // the register-resident plain / norm prologues hold at most 4 float4 per thread;
  // wider rows of the plain prologue with the residual add (ffn_down) take the
  // LDS-staged variant of the row kernel
  const bool wide_ok = a.pro == PRO_PLAIN && a.epi == EPI_ADD;
  if ((a.pro == PRO_PLAIN || a.pro == PRO_NORM) && a.k > 4 * 4 * kWg && !wide_ok) {
    if (needs_row) throw Error(CHONK_EINVAL, "row-kernel prologues hold at most 4096 elements (the plain one excepted)");
    return;
  }
  for (int i = 0; i < a.nseg; ++i)
    if (a.seg[i].w.k / 32 > kRowUnits * 64) {
      if (needs_row) throw Error(CHONK_EINVAL, "the row kernels take rows of at most 8192 weights");
      return;
    }
  // one unit per lane and >= 192 workgroups per segment; the three-segment
  // q|k|v launch runs faster with two units per lane and half the workgroups
  // (measured on the Qwen3-0.6B shapes)
  const bool multi = a.nseg > 1;
  int wg = 0;
  for (int i = 0; i < a.nseg; ++i) {
    plan_seg_row(a.seg[i], wg, multi ? 2 : 1, multi ? 96 : 192);
    wg += seg_wgs(a.seg[i]);
  }
  a.row_kernel = 1;
}

// Rotary inverse frequencies theta^(-2d/hd) in f32, evaluated once on the host
// with the reference's operation order (rope_angle, llama-wgsl-runtime.ts:2884-2887).
const float* rope_table(chonk_engine* e, uint32_t theta, int hd) {
  for (const auto& t : e->rope_tables)
    if (t.first == theta) return t.second;
  std::vector<float> inv((size_t)hd / 2);
  // theta 0: no rotary embedding (GPT-2): every angle is 0
  for (int d = 0; d < hd / 2; ++d) inv[d] = theta == 0 ? 0.0f : std::pow((float)theta, (-2.0f * (float)d) / (float)hd);
  float* p = (float*)e->weights.take(inv.size() * 4);
  HIP_OK(hipMemcpy(p, inv.data(), inv.size() * 4, hipMemcpyHostToDevice));
  e->rope_tables.emplace_back(theta, p);
  return p;
}

// (cos, sin) of every position's rotary angles for one theta, computed on the
// device with the kernels' own expression (so the values are those the
// kernels would compute inline).
const float2* rope_cs_table(chonk_engine* e, uint32_t theta, int hd) {
  for (const auto& t : e->rope_cs)
    if (t.first == theta) return t.second;
  const float* inv = rope_table(e, theta, hd);
  float2* p = nullptr;
  HIP_OK(hipMalloc(&p, (size_t)e->cfg.ctx * (hd / 2) * sizeof(float2)));
  e->rope_cs.emplace_back(theta, p);
  HIP_OK(launch_rope_cs(inv, hd / 2, e->cfg.ctx, p, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  return p;
}

// fuse: join each qualifying layer's q|k|v matvec and attention (fuse_qkv engines)
void build_steps(chonk_engine* e, bool fuse) {
  const ModelCfg& c = e->cfg;
  const int H = c.hidden;
  auto mv_base = [&]() {
    MvArgs a{};
    a.st = e->st;
    a.eps = c.eps;
    a.vocab = c.vocab;
    a.hist = e->hist;
    a.embed = e->embed.q;
    a.embed_scale = c.embed_scale;
    a.samp = e->samp;
    a.pen_bits = e->pen_bits;
    a.cand = e->cand;
    return a;
  };
  auto finish = [&](Launch& L, MvArgs& a, int max_rows) {
    use_row_kernel(a);
    L.kind = Launch::MV;
    L.mv = a;
    L.grid = 0;
    for (int i = 0; i < a.nseg; ++i) L.grid += seg_wgs(a.seg[i]);
    L.shmem = mv_shared_bytes(a.k, max_rows);
  };
  std::vector<Launch> steps;
  for (int i = 0; i < c.layers; ++i) {
    LayerDev& Ld = e->layers[i];
    const std::string li = "L" + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    const int qdim = lc.heads * c.hd, kvdim = lc.kv_heads * c.hd, G = lc.heads / lc.kv_heads;
    if (lc.conv) {
      // LfmWgslEngine.runToken's convolution branch (lfm-wgsl-runtime.ts:740-744):
      // in_proj with the operator norm as prologue, then out_proj whose
      // prologue is CONV_BLOCK over this token's B | C | x and the layer's state
      // (shifted afterwards by the gate|up launch) and whose epilogue adds the
      // residual (opAddNorm's add)
      {
        Launch L;
        MvArgs a = mv_base();
        a.k = H;
        a.nseg = 1;
        plan_seg(a.seg[0], Ld.conv_in.q, 3 * H, false, 0);
        a.seg[0].out = e->conv_proj;
        a.epi = EPI_STORE;
        a.w_norm = Ld.in_norm;
        if (i == 0) {
          a.pro = PRO_EMBED_NORM;
          a.res_out = e->resA;
        } else {
          a.pro = PRO_NORM;
          a.in = e->resA;
        }
        finish(L, a, a.seg[0].tile);
        L.name = li + "inproj";
        L.weight_bytes = Ld.conv_in.gguf_bytes + (i == 0 ? e->embed.gguf_bytes / c.vocab : 0);
        L.layer = i;
        steps.push_back(L);
      }
      {
        Launch L;
        MvArgs a = mv_base();
        a.k = H;
        a.nseg = 1;
        plan_seg(a.seg[0], Ld.conv_out.q, H, false, 0);
        a.pro = PRO_CONV;
        a.conv_proj = e->conv_proj;
        a.conv_w = Ld.conv_w;
        a.conv_s1 = Ld.conv_s1;
        a.conv_s2 = Ld.conv_s2;
        a.conv_n = H;
        a.epi = EPI_ADD;
        a.seg[0].out = e->resB;
        a.seg[0].add = e->resA;
        finish(L, a, a.seg[0].tile);
        L.name = li + "outproj";
        L.weight_bytes = Ld.conv_out.gguf_bytes;
        L.layer = i;
        steps.push_back(L);
      }
    }
    if (lc.mamba) {
      // GraniteWgslEngine.runToken's Mamba branch (granite-wgsl-runtime.ts:786-791):
      // in_proj with the input norm as prologue; the convolution and selective
      // scan; out_proj whose prologue is MAMBA_GATE_NORM and whose epilogue is
      // the scaled residual add (the reference's addScaledRmsNorm add)
      {
        Launch L;
        MvArgs a = mv_base();
        a.k = H;
        a.nseg = 1;
        plan_seg(a.seg[0], Ld.ssm_in.q, c.ssm_inner + c.ssm_conv + c.ssm_heads, false, 0);
        a.seg[0].out = e->mproj;
        a.epi = EPI_STORE;
        a.w_norm = Ld.in_norm;
        if (i == 0) {
          a.pro = PRO_EMBED_NORM;
          a.res_out = e->resA;
        } else {
          a.pro = PRO_NORM;
          a.in = e->resA;
        }
        finish(L, a, a.seg[0].tile);
        L.name = li + "inproj";
        L.weight_bytes = Ld.ssm_in.gguf_bytes + (i == 0 ? e->embed.gguf_bytes / c.vocab : 0);
        L.layer = i;
        steps.push_back(L);
      }
      {
        Launch L;
        L.kind = Launch::SSM;
        SsmArgs& m = L.ssm;
        m.proj = e->mproj;
        m.conv_w = Ld.c1d_w;
        m.conv_b = Ld.c1d_b;
        m.conv_state = Ld.mconv_state;
        m.dt_bias = Ld.dt_b;
        m.a_neg = Ld.a_neg;
        m.d = Ld.d_w;
        m.ssm_state = Ld.ssm_state;
        m.y = e->my;
        m.st = e->st;
        m.inner = c.ssm_inner;
        m.conv = c.ssm_conv;
        m.heads = c.ssm_heads;
        L.grid = c.ssm_heads * 4;
        L.name = li + "ssm";
        L.layer = i;
        steps.push_back(L);
      }
      {
        Launch L;
        MvArgs a = mv_base();
        a.k = c.ssm_inner;
        a.nseg = 1;
        plan_seg(a.seg[0], Ld.ssm_out.q, H, false, 0);
        a.pro = PRO_GATE;
        a.in = e->my;
        a.gate_z = e->mproj;
        a.w_norm = Ld.ssm_norm;
        a.epi = EPI_ADD;
        a.seg[0].out = e->resB;
        a.seg[0].add = e->resA;
        a.add_scale = c.res_scale;
        finish(L, a, a.seg[0].tile);
        L.name = li + "outproj";
        L.weight_bytes = Ld.ssm_out.gguf_bytes;
        L.layer = i;
        steps.push_back(L);
      }
    }
    // qkv (gpt2: one fused matrix with bias, LayerNorm prologue; embedding +
    // position on layer 0)
    if (lc.conv || lc.mamba) {
      // (no attention in a convolution or Mamba2 layer)
    } else if (c.gpt) {
      Launch L;
      MvArgs a = mv_base();
      a.k = H;
      a.nseg = 1;
      plan_seg(a.seg[0], Ld.qkv.q, 3 * H, false, 0);
      a.seg[0].out = e->qkv;
      a.seg[0].bias = Ld.qkv_b;
      a.epi = EPI_STORE;
      a.w_norm = Ld.in_norm;
      a.norm_b = Ld.in_norm_b;
      if (i == 0) {
        a.pro = PRO_EMBED_LN;
        a.pos_embd = e->pos_embd;
        a.res_out = e->resA;
      } else {
        a.pro = PRO_LN;
        a.in = e->resA;
      }
      finish(L, a, a.seg[0].tile);
      L.name = li + "qkv";
      L.weight_bytes = Ld.qkv.gguf_bytes + (i == 0 ? e->embed.gguf_bytes / c.vocab : 0);
      L.layer = i;
      steps.push_back(L);
    } else {
      Launch L;
      MvArgs a = mv_base();
      a.k = H;
      if (c.openelm) {
        // one fused matrix whose rows are q | k | v (attn.qkv_proj, :359, :1071-1074)
        a.nseg = 1;
        plan_seg(a.seg[0], Ld.qkv.q, qdim + 2 * kvdim, false, 0);
        a.seg[0].out = e->qkv;
      } else {
        a.nseg = 3;
        plan_seg(a.seg[0], Ld.q.q, qdim, false, 0);
        a.seg[0].out = e->qkv;
        plan_seg(a.seg[1], Ld.k.q, kvdim, false, seg_wgs(a.seg[0]));
        a.seg[1].out = e->qkv + qdim;
        plan_seg(a.seg[2], Ld.v.q, kvdim, false, a.seg[1].wg_begin + seg_wgs(a.seg[1]));
        a.seg[2].out = e->qkv + qdim + kvdim;
      }
      a.epi = EPI_STORE;
      a.w_norm = Ld.in_norm;
      if (i == 0) {
        a.pro = PRO_EMBED_NORM;
        a.res_out = e->resA;
      } else if (c.gemma) {
        a.pro = PRO_RES_NORM;
        a.in = e->resB;
        a.delta = e->delta;
        a.w_delta = e->layers[i - 1].post_ffn_norm;
        a.res_out = e->resA;
      } else {
        a.pro = PRO_NORM;
        a.in = e->resA;
      }
      int max_tile = 0;
      for (int si = 0; si < a.nseg; ++si) max_tile = std::max(max_tile, a.seg[si].tile);
      finish(L, a, max_tile);
      L.name = li + "qkv";
      L.weight_bytes = Ld.q.gguf_bytes + Ld.k.gguf_bytes + Ld.v.gguf_bytes + Ld.qkv.gguf_bytes +
                       (i == 0 ? e->embed.gguf_bytes / c.vocab : 0);
      L.layer = i;
      steps.push_back(L);
    }
    // attention
    if (!lc.conv && !lc.mamba) {
      Launch L;
      L.kind = Launch::ATTN;
      AttnArgs& t = L.at;
      t.qkv = e->qkv;
      t.qn_w = c.qk_norm ? Ld.q_norm : nullptr;
      t.kn_w = c.qk_norm ? Ld.k_norm : nullptr;
      t.kc = Ld.kc;
      t.vc = Ld.vc;
      t.part = e->part;
      t.cnt = e->cnt;
      t.out = e->attn;
      t.st = e->st;
      t.heads = lc.heads;
      t.kv_heads = lc.kv_heads;
      t.hd = c.hd;
      t.ctx = c.ctx;
      t.window = c.layer[i].window;
      t.chunk = e->chunk;
      t.nchunk = e->nchunk;
      t.theta = c.layer[i].theta;
      t.interleaved = c.interleaved ? 1 : 0;
      t.kv_f16 = e->kv_elem == 2 ? 1 : 0;
      t.eps = c.qk_eps;
      t.scale = c.scale;
      t.merge_floats = attn_merge_floats(G, c.hd, e->nchunk);
      t.rope_inv = rope_table(e, c.layer[i].theta, c.hd);
      // full-context layers fetch K/V before the position is known; that reads
      // the whole cache span of every chunk, so only for short contexts
      t.spec_kv = (t.window == 0 && c.ctx <= 4096) ? 1 : 0;
      t.tpp = attn_threads_per_position(c.hd, e->chunk, (int)e->kv_elem);
      L.shmem = attn_shared_bytes(G, c.hd, e->chunk, e->nchunk, e->kv_elem);
      L.grid = lc.kv_heads * e->nchunk;
      if (e->dec_attn) {
        t.variant = 1;
        t.tpart = e->dpart;
        t.rope_cs = rope_cs_table(e, c.layer[i].theta, c.hd);
        t.chunk = attn_dec_chunk();
        t.nchunk = e->dnchunk;
        t.sub = e->dsub;
        t.merge_floats = attn_merge_floats(G, c.hd, e->dnchunk);
        L.shmem = attn_dec_shared_bytes(G, c.hd, e->dnchunk);
        L.grid = lc.kv_heads * e->dnchunk;
      }
      L.name = li + "attn";
      L.layer = i;
      // the layer's q|k|v matvec (the launch before) joins this one when it is
      // the three-matrix row kernel with the RMSNorm prologue, an instance
      // exists and the joint grid fits on the device at once
      Launch* Q = steps.empty() ? nullptr : &steps.back();
      if (fuse && e->fuse_qkv && Q && Q->kind == Launch::MV && Q->layer == i && Q->name == li + "qkv" &&
          Q->mv.pro == PRO_NORM && Q->mv.nseg == 3 && Q->mv.row_kernel && L.at.variant == 1 && L.at.sub == 1) {
        Launch F;
        F.kind = Launch::QKVATTN;
        F.mv = Q->mv;
        F.mv.epi = EPI_TAG;
        F.mv.tag_epoch = e->cnt;
        F.mv.seg[0].out = (float*)e->qkv_tag;  // (EPI_TAG stores 8-byte tagged words)
        F.mv.seg[1].out = (float*)(e->qkv_tag + qdim);
        F.mv.seg[2].out = (float*)(e->qkv_tag + qdim + kvdim);
        F.mv.seg[0].tag_div = G * c.hd;
        F.mv.seg[1].tag_div = c.hd;
        F.mv.seg[2].tag_div = c.hd;
        F.at = L.at;
        F.at.qkv_tag = e->qkv_tag;
        // the attention's K/V requests wait 0.9 us, behind the matvec's loads (measured at the
        // Qwen3-0.6B shape at 2K context: 1223 -> 1240 tokens/s; 0.6 and 1.2 us gained less);
        // CHONK_KV_DELAY overrides (ticks of 10 ns)
        F.at.kv_delay = 90;
        if (const char* kd = std::getenv("CHONK_KV_DELAY")) F.at.kv_delay = std::max(0, std::min(1000, std::atoi(kd)));
        F.nq = Q->grid;
        F.grid = Q->grid + L.grid;
        F.shmem = std::max(Q->shmem, L.shmem);
        F.name = li + "qkv_attn";
        F.weight_bytes = Q->weight_bytes;
        F.layer = i;
        if (qkv_attn_resident(e->device, G, c.hd, F.shmem) >= F.grid) {
          steps.back() = F;
        } else {
          steps.push_back(L);
        }
      } else {
        steps.push_back(L);
      }
    }
    // o projection
    if (!lc.conv && !lc.mamba) {
      Launch L;
      MvArgs a = mv_base();
      a.k = qdim;
      a.nseg = 1;
      plan_seg(a.seg[0], Ld.o.q, H, false, 0);
      a.pro = PRO_PLAIN;
      a.in = e->attn;
      a.add_scale = c.res_scale;  // (granitehybrid: residual + out * 0.246)
      if (c.gemma) {
        a.epi = EPI_STORE;
        a.seg[0].out = e->delta;
      } else {
        a.epi = EPI_ADD;
        a.seg[0].out = e->resB;
        a.seg[0].add = e->resA;
      }
      if (c.gpt) {
        a.seg[0].bias = Ld.o_b;
        a.sanitize = 1;
      }
      finish(L, a, a.seg[0].tile);
      L.name = li + "oproj";
      L.weight_bytes = Ld.o.gguf_bytes;
      L.layer = i;
      steps.push_back(L);
    }
    // gate|up (gpt2: up with bias, GELU-tanh, LayerNorm prologue)
    if (c.gpt) {
      Launch L;
      MvArgs a = mv_base();
      a.k = H;
      a.nseg = 1;
      plan_seg(a.seg[0], Ld.up.q, lc.ffn, false, 0);
      a.seg[0].out = e->ff;
      a.seg[0].bias = Ld.up_b;
      a.epi = EPI_GELU;
      a.pro = PRO_LN;
      a.in = e->resB;
      a.w_norm = Ld.post_norm;
      a.norm_b = Ld.post_norm_b;
      finish(L, a, a.seg[0].tile);
      L.name = li + "gateup";
      L.weight_bytes = Ld.up.gguf_bytes;
      L.layer = i;
      steps.push_back(L);
    } else {
      Launch L;
      MvArgs a = mv_base();
      a.k = H;
      a.nseg = 1;
      plan_seg(a.seg[0], Ld.gate.q, lc.ffn, true, 0);
      a.seg[0].w2 = Ld.up.q;
      a.seg[0].out = e->ff;
      a.epi = c.gemma ? EPI_GLU_GELU : EPI_GLU_SILU;
      if (c.gemma) {
        a.pro = PRO_RES_NORM;
        a.in = e->resA;
        a.delta = e->delta;
        a.w_delta = Ld.post_norm;
        a.res_out = e->resB;
        a.w_norm = Ld.pre_ffn_norm;
      } else {
        a.pro = PRO_NORM;
        a.in = e->resB;
        a.w_norm = Ld.post_norm;
      }
      if (lc.conv) {
        // every reader of the old state (out_proj) has finished: shift it
        a.conv_commit = 1;
        a.conv_proj = e->conv_proj;
        a.conv_s1 = Ld.conv_s1;
        a.conv_s2 = Ld.conv_s2;
        a.conv_n = H;
      }
      finish(L, a, 2 * a.seg[0].tile);
      L.name = li + "gateup";
      L.weight_bytes = Ld.gate.gguf_bytes + Ld.up.gguf_bytes;
      L.layer = i;
      steps.push_back(L);
    }
    // down
    {
      Launch L;
      MvArgs a = mv_base();
      a.k = lc.ffn;
      a.nseg = 1;
      plan_seg(a.seg[0], Ld.down.q, H, false, 0);
      a.pro = PRO_PLAIN;
      a.in = e->ff;
      a.add_scale = c.res_scale;  // (granitehybrid: ADD_SCALED_WGSL's residual + out * 0.246)
      if (c.gemma) {
        a.epi = EPI_STORE;
        a.seg[0].out = e->delta;
      } else {
        a.epi = EPI_ADD;
        a.seg[0].out = e->resA;
        a.seg[0].add = e->resB;
      }
      if (c.gpt) {
        a.seg[0].bias = Ld.down_b;
        a.sanitize = 1;
      }
      finish(L, a, a.seg[0].tile);
      L.name = li + "down";
      L.weight_bytes = Ld.down.gguf_bytes;
      L.layer = i;
      steps.push_back(L);
    }
  }
  e->kernels_plain = steps;
  e->kernels_plain.back().mv.advance_pos = 1;
  // lm_head + group argmax
  {
    Launch L;
    MvArgs a = mv_base();
    a.k = H;
    a.nseg = 1;
    MvSeg& sg = a.seg[0];
    sg.w = e->lm_head.q;
    sg.n_out = c.vocab;
    sg.lpr = pick_lpr(H / 32);
    sg.tile = 256;
    sg.wg_begin = 0;
    sg.out = e->logits;
    if (c.lfm || c.granite) {
      // class-major rows: workgroup c computes ids c, c + 256, ... (TOPK256's slot c)
      sg.n_out = (int)class_rows(c.vocab);
      sg.tile = sg.n_out / 256;
      a.lfm_classes = 1;
    }
    a.logit_scale = c.logit_scale;  // (granitehybrid: SCALE_LOGITS_WGSL's x 1/3)
    if (e->lm_lanes.q.s0) {
      sg.w = e->lm_lanes.q;
      a.lm_lanes = 1;
    }
    a.epi = EPI_LOGITS;
    a.w_norm = e->final_norm;
    a.gpt_argmax = c.gpt ? 1 : 0;
    if (c.gpt) {
      a.pro = PRO_LN;
      a.in = e->resA;
      a.norm_b = e->final_norm_b;
    } else if (c.gemma) {
      a.pro = PRO_RES_NORM;
      a.in = e->resB;
      a.delta = e->delta;
      a.w_delta = e->layers[c.layers - 1].post_ffn_norm;
      a.res_out = e->resA;
    } else {
      a.pro = PRO_NORM;
      a.in = e->resA;
    }
    finish(L, a, std::max(256, sg.tile));
    L.name = "lmhead";
    L.weight_bytes = e->lm_head.gguf_bytes;
    steps.push_back(L);
  }
  {
    Launch L;
    L.kind = Launch::SEL;
    SelArgs& s = L.sel;
    s.cand = e->cand;
    // (ARGMAX_WGSL's stage over the 256 slots is the same strict-greater tree, lfm-wgsl-runtime.ts:1903-1922)
    s.gpt_argmax = c.gpt || c.lfm || c.granite ? 1 : 0;
    s.groups = e->groups;
    s.vocab = c.vocab;
    s.ctx = c.ctx;
    s.samp = e->samp;
    s.pen_bits = e->pen_bits;
    s.seen_bits = e->seen_bits;
    s.hist = e->hist;
    s.gen = e->gen;
    s.st = e->st;
    L.grid = 1;
    L.name = "select";
    steps.push_back(L);
  }
  e->kernels_logits = steps;
}

void enqueue(const Launch& L, hipStream_t s) {
  switch (L.kind) {
    case Launch::MV: HIP_OK(launch_matvec(L.mv, L.grid, L.shmem, s)); break;
    case Launch::ATTN: HIP_OK(launch_attention(L.at, L.shmem, s)); break;
    case Launch::SSM: HIP_OK(launch_ssm(L.ssm, s)); break;
    case Launch::SEL: HIP_OK(launch_select(L.sel, s)); break;
    case Launch::QKVATTN: HIP_OK(launch_qkv_attn(L.mv, L.nq, L.at, L.shmem, s)); break;
  }
}

void capture(chonk_engine* e, const std::vector<Launch>& steps, hipGraph_t* g, hipGraphExec_t* x, int repeat = 1) {
  HIP_OK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
  try {
    for (int r = 0; r < repeat; ++r)
      for (const Launch& L : steps) enqueue(L, e->stream);
  } catch (...) {
    hipGraph_t tmp;
    (void)hipStreamEndCapture(e->stream, &tmp);
    throw;
  }
  HIP_OK(hipStreamEndCapture(e->stream, g));
  HIP_OK(hipGraphInstantiate(x, *g, nullptr, nullptr, 0));
}

// At most one engine per GPU runs the spin-merging decode attention
// (k_attn_dec): its chunks wait for each other's rows, so its whole grid must
// be resident at once, and the grids of two engines decoding on different
// threads could together exceed the device and wait until the time bound.
// The first engine on a device that qualifies claims the device; engines
// created while the claim is held use the arrival-counter k_attention (no
// waiting). The claim ends with the engine.
struct SpinClaims {
  std::mutex mu;
  std::map<int, const chonk_engine*> owner;
};
SpinClaims& spin_claims() {
  static SpinClaims* c = new SpinClaims();
  return *c;
}
bool claim_spin(int device, const chonk_engine* e) {
  SpinClaims& c = spin_claims();
  std::lock_guard<std::mutex> l(c.mu);
  auto it = c.owner.find(device);
  if (it != c.owner.end() && it->second != e) return false;
  c.owner[device] = e;
  return true;
}
void release_spin(int device, const chonk_engine* e) {
  SpinClaims& c = spin_claims();
  std::lock_guard<std::mutex> l(c.mu);
  auto it = c.owner.find(device);
  if (it != c.owner.end() && it->second == e) c.owner.erase(it);
}

// The engines alive on each device. The fused q|k|v + attention launch needs
// its whole grid resident at once (the attention's chunks wait for each
// other's rows). A launch of another engine's stream that the dispatcher
// interleaves with a partly dispatched fused grid can wait for the resources
// its resident workgroups hold while the rest of the grid waits behind it, so
// an engine replays its fused steps only while it is the only engine on its
// device (under this lock, which also orders a new engine's registration after
// the fused steps already queued: registration waits for them to finish).
struct DeviceEngines {
  std::mutex mu;
  std::map<int, std::vector<chonk_engine*>> live;
};
DeviceEngines& device_engines() {
  static DeviceEngines* d = new DeviceEngines();
  return *d;
}
void register_engine(chonk_engine* e) {
  DeviceEngines& d = device_engines();
  std::lock_guard<std::mutex> l(d.mu);
  for (chonk_engine* o : d.live[e->device]) HIP_OK(hipStreamSynchronize(o->stream));
  d.live[e->device].push_back(e);
  e->registered = true;
}
void unregister_engine(chonk_engine* e) {
  if (!e->registered) return;
  DeviceEngines& d = device_engines();
  std::lock_guard<std::mutex> l(d.mu);
  auto& v = d.live[e->device];
  v.erase(std::remove(v.begin(), v.end(), e), v.end());
  e->registered = false;
}

void engine_free(chonk_engine* e) {
  if (!e) return;
  unregister_engine(e);
  release_spin(e->device, e);
  (void)hipSetDevice(e->device);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  if (e->exec_logits) (void)hipGraphExecDestroy(e->exec_logits);
  if (e->exec_plain) (void)hipGraphExecDestroy(e->exec_plain);
  if (e->graph_logits) (void)hipGraphDestroy(e->graph_logits);
  if (e->graph_plain) (void)hipGraphDestroy(e->graph_plain);
  if (e->exec_logits_sep) (void)hipGraphExecDestroy(e->exec_logits_sep);
  if (e->exec_plain_sep) (void)hipGraphExecDestroy(e->exec_plain_sep);
  if (e->graph_logits_sep) (void)hipGraphDestroy(e->graph_logits_sep);
  if (e->graph_plain_sep) (void)hipGraphDestroy(e->graph_plain_sep);
  if (e->exec_multi) (void)hipGraphExecDestroy(e->exec_multi);
  if (e->graph_multi) (void)hipGraphDestroy(e->graph_multi);
  e->weights.release();
  e->state.release();
  uncached_pool().give_back(e->device, e->uncached);
  if (e->pf_mem) (void)hipFree(e->pf_mem);
  if (e->flush) (void)hipFree(e->flush);
  for (auto& t : e->rope_cs) (void)hipFree(t.second);
  if (e->h_state) (void)hipHostFree(e->h_state);
  if (e->h_tok) (void)hipHostFree(e->h_tok);
  if (e->h_samp) (void)hipHostFree(e->h_samp);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  delete e;
}

void create_engine(const chonk_model_def* def, std::unique_ptr<ByteSource> src, const std::string& label,
                   chonk_engine** out) {
  if (!def || !out) throw Error(CHONK_EINVAL, "null argument");
  if (def->vocab <= 0 || def->max_context <= 0) throw Error(CHONK_EINVAL, "ModelDef vocab and maxContext must be positive");
  if (def->n_eos < 0 || def->n_eos > 16) throw Error(CHONK_EINVAL, "at most 16 EOS ids are supported");
  GgufFile g;
  try {
    g = read_gguf_header(*src, label);
  } catch (const Error&) {
    throw;
  } catch (const std::exception& x) {
    throw Error(CHONK_EINVAL, x.what());
  }
  std::unique_ptr<chonk_engine, void (*)(chonk_engine*)> e(new chonk_engine(), engine_free);
  e->def = *def;
  e->model_id = def->id ? def->id : "";
  e->eos.assign(def->eos_ids, def->eos_ids + def->n_eos);
  e->device = def->device;
  e->cfg = build_config(g, *def);
  const ModelCfg& c = e->cfg;
  HIP_OK(hipSetDevice(e->device));
  HIP_OK(hipStreamCreate(&e->stream));
  register_engine(e.get());
  e->kv_elem = def->kv_dtype == CHONK_KV_F32 ? 4 : 2;

  const int H = c.hidden, qdim = c.heads * c.hd, kvdim = c.kv_heads * c.hd;
  const std::string lm_name = g.find("output.weight") ? "output.weight" : "token_embd.weight";
  const bool tied = lm_name == "token_embd.weight";
  // the lm_head's lane-interleaved copy for k_lm_lanes (CHONK_LM=rows keeps k_mv_logits_t)
  const char* lmv = std::getenv("CHONK_LM");
  // (k_lm_lanes keeps 2 or 4 units in flight per lane: an even number of 32-element units per row)
  const bool lm_lanes = !c.lfm && !c.granite && lane_layout_type(tensor(g, lm_name).type) && (H / 32) % 2 == 0 &&
                        !(lmv && std::strcmp(lmv, "rows") == 0);
  // size the weight arena
  size_t wbytes = 0;
  auto mat_bytes = [&](const std::string& name, int64_t K, int64_t N) {
    const GgufTensorInfo& t = tensor(g, name);
    check_matrix(t, K, N);
    wbytes += stripes_bytes(t.type, N, K);
  };
  auto vec_bytes = [&](int64_t n) { wbytes += align256((size_t)n * 4); };
  if (c.lfm || c.granite) {
    // the embedding, its class-major copy as lm_head, the final norm
    const GgufTensorInfo& te = c.granite ? granite_linear(g, "token_embd.weight", H, c.vocab)
                                         : lfm_linear(g, "token_embd.weight");
    check_matrix(te, H, c.vocab);
    wbytes += stripes_bytes(te.type, c.vocab, H) + stripes_bytes(te.type, class_rows(c.vocab), H);
  } else {
    mat_bytes("token_embd.weight", H, c.vocab);
    if (!tied) mat_bytes(lm_name, H, c.vocab);
    if (lm_lanes) wbytes += stripes_bytes(tensor(g, lm_name).type, lane_rows(c.vocab), H);
  }
  vec_bytes(H);
  if (c.gpt) {
    if (tied) throw Error(CHONK_EINVAL, "GPT WGSL GGUF missing tensor output.weight");
    vec_bytes(H);                                // final LayerNorm bias
    vec_bytes((int64_t)c.pos_rows * H);          // position table
    vec_bytes(c.hd / 2);                         // (zero) rotary table
    for (int i = 0; i < c.layers; ++i) {
      const std::string p = "blk." + std::to_string(i) + ".";
      mat_bytes(p + "attn_qkv.weight", H, 3 * (int64_t)H);
      mat_bytes(p + "attn_output.weight", H, H);
      mat_bytes(p + "ffn_up.weight", H, c.ffn);
      mat_bytes(p + "ffn_down.weight", c.ffn, H);
      for (int v = 0; v < 4; ++v) vec_bytes(H);  // LayerNorm weights and biases
      vec_bytes(3 * (int64_t)H);
      vec_bytes(H);
      vec_bytes(c.ffn);
      vec_bytes(H);
    }
  }
  for (int i = 0; i < (c.lfm ? c.layers : 0); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    auto lin = [&](const std::string& name, int64_t K, int64_t N) {
      const GgufTensorInfo& t = lfm_linear(g, p + name);
      check_matrix(t, K, N);
      wbytes += stripes_bytes(t.type, N, K);
    };
    if (lc.conv) {
      const GgufTensorInfo& cw = lfm_tensor(g, p + "shortconv.conv.weight");
      if (cw.shape.size() != 2 || cw.shape[0] != 3 || (int64_t)cw.shape[1] != H)
        throw Error(CHONK_EINVAL, "LFM GGUF tensor " + cw.name + " must be [3, " + std::to_string(H) + "]");
      lin("shortconv.in_proj.weight", H, 3 * (int64_t)H);
      lin("shortconv.out_proj.weight", H, H);
      vec_bytes(3 * (int64_t)H);
    } else {
      lin("attn_q.weight", H, lc.heads * c.hd);
      lin("attn_k.weight", H, lc.kv_heads * c.hd);
      lin("attn_v.weight", H, lc.kv_heads * c.hd);
      lin("attn_output.weight", lc.heads * c.hd, H);
      vec_bytes(c.hd);
      vec_bytes(c.hd);
      vec_bytes(c.hd / 2);
    }
    lin("ffn_gate.weight", H, lc.ffn);
    lin("ffn_up.weight", H, lc.ffn);
    lin("ffn_down.weight", lc.ffn, H);
    vec_bytes(H);
    vec_bytes(H);
  }
  const int64_t ssm_proj = (int64_t)c.ssm_inner + c.ssm_conv + c.ssm_heads;  // granitehybrid in_proj rows
  for (int i = 0; i < (c.granite ? c.layers : 0); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    auto lin = [&](const std::string& name, int64_t K, int64_t N) {
      wbytes += stripes_bytes(granite_linear(g, p + name, K, N).type, N, K);
    };
    if (lc.mamba) {
      lin("ssm_in.weight", H, ssm_proj);
      lin("ssm_out.weight", c.ssm_inner, H);
      vec_bytes(4 * (int64_t)c.ssm_conv);
      vec_bytes(c.ssm_conv);
      for (int v = 0; v < 3; ++v) vec_bytes(c.ssm_heads);
      vec_bytes(c.ssm_inner);
    } else {
      lin("attn_q.weight", H, lc.heads * c.hd);
      lin("attn_k.weight", H, lc.kv_heads * c.hd);
      lin("attn_v.weight", H, lc.kv_heads * c.hd);
      lin("attn_output.weight", lc.heads * c.hd, H);
      vec_bytes(c.hd / 2);  // (zero) rotary table
    }
    lin("ffn_gate.weight", H, lc.ffn);
    lin("ffn_up.weight", H, lc.ffn);
    lin("ffn_down.weight", lc.ffn, H);
    vec_bytes(H);
    vec_bytes(H);
  }
  for (int i = 0; i < (c.gpt || c.lfm || c.granite ? 0 : c.layers); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    const int lq = lc.heads * c.hd, lkv = lc.kv_heads * c.hd;
    if (c.openelm) {
      mat_bytes(p + "attn_qkv.weight", H, lq + 2 * lkv);
    } else {
      mat_bytes(p + "attn_q.weight", H, lq);
      mat_bytes(p + "attn_k.weight", H, lkv);
      mat_bytes(p + "attn_v.weight", H, lkv);
    }
    mat_bytes(p + "attn_output.weight", lq, H);
    mat_bytes(p + "ffn_gate.weight", H, lc.ffn);
    mat_bytes(p + "ffn_up.weight", H, lc.ffn);
    mat_bytes(p + "ffn_down.weight", lc.ffn, H);
    vec_bytes(H);
    vec_bytes(H);
    if (c.gemma) {
      vec_bytes(H);
      vec_bytes(H);
    }
    if (c.qk_norm) {
      vec_bytes(c.hd);
      vec_bytes(c.hd);
    }
    vec_bytes(c.hd / 2);  // rotary table (one per distinct theta at most)
  }
  e->weights.reserve(wbytes);

  // state arena: K/V cache + activations + bookkeeping
  // (lfm2: one argmax slot per residue class, TOPK256_WGSL)
  e->groups = c.lfm || c.granite ? 256 : (c.vocab + 255) / 256;
  int kv_layers = 0, conv_layers = 0, mamba_layers = 0;  // layers holding a K/V cache / a conv state / an SSM state
  for (const LayerCfg& lc : c.layer) (lc.conv ? conv_layers : lc.mamba ? mamba_layers : kv_layers) += 1;
  // attention chunk: the smallest power of two >= 16 giving at most ~512
  // workgroups and at most 32 chunks over the whole context (the last chunk to
  // finish merges all chunks), capped by the kernel's limit for hd
  e->chunk = 16;
  while (e->chunk < attn_max_chunk(c.hd) &&
         ((int64_t)c.kv_heads * ((c.ctx + e->chunk - 1) / e->chunk) > 512 || (c.ctx + e->chunk - 1) / e->chunk > 32))
    e->chunk <<= 1;
  if (const char* ov = std::getenv("CHONK_ATTN_CHUNK")) {  // tuning override: a power of two in [16, limit]
    const int v = std::atoi(ov);
    if (v >= 16 && v <= attn_max_chunk(c.hd) && (v & (v - 1)) == 0) e->chunk = v;
  }
  e->nchunk = (c.ctx + e->chunk - 1) / e->chunk;
  const int G = c.gmax;  // partial rows are sized for the largest group
  // the register-resident decode attention where it applies (every layer's
  // group); CHONK_ATTN=chunked keeps k_attention
  {
    const char* av = std::getenv("CHONK_ATTN");
    e->dec_attn = !(av && std::strcmp(av, "chunked") == 0);
    e->dsub = attn_dec_sub(c.ctx, 128);
    if (e->dsub > 1) {
      // long contexts: each workgroup walks several 64-position chunks, as many
      // workgroups per kv head as stay resident together with the walking kernel
      int per_head = 128;
      for (const LayerCfg& lc : c.layer) {
        if (lc.conv || lc.mamba) continue;
        const int lg = lc.heads / lc.kv_heads;
        per_head = std::min(per_head, attn_dec_resident(e->device, lg, c.hd, attn_dec_shared_bytes(lg, c.hd, 128), true) /
                                          std::max(1, lc.kv_heads));
      }
      e->dsub = attn_dec_sub(c.ctx, per_head);
    }
    e->dnchunk = ((c.ctx + attn_dec_chunk() - 1) / attn_dec_chunk() + e->dsub - 1) / e->dsub;
    for (const LayerCfg& lc : c.layer) {
      const int lg = lc.heads / lc.kv_heads;
      if (lc.conv || lc.mamba) continue;
      if (e->dec_attn && (!attn_dec_supported(lg, c.hd, c.ctx, e->kv_elem == 2 ? 1 : 0) ||
                          attn_dec_resident(e->device, lg, c.hd, attn_dec_shared_bytes(lg, c.hd, e->dnchunk), e->dsub > 1) <
                              lc.kv_heads * e->dnchunk))
        e->dec_attn = false;
    }
    // (another engine on this GPU holds the spin-merging attention: k_attention)
    if (e->dec_attn && !claim_spin(e->device, e.get())) e->dec_attn = false;
    // the q|k|v matvec joins the attention launch where the layer allows it
    // (build_steps checks the instance and the grid's residency per layer);
    // CHONK_FUSE=0 keeps them apart
    const char* fv = std::getenv("CHONK_FUSE");
    e->fuse_qkv = e->dec_attn && e->dsub == 1 && !(fv && std::strcmp(fv, "0") == 0);
  }
  const size_t kv_bytes = (size_t)kvdim * c.ctx * e->kv_elem;
  const size_t bits_words = (size_t)(c.vocab + 31) / 32;
  size_t sbytes = 2 * align256(kv_bytes) * kv_layers;
  sbytes += c.lfm ? align256((size_t)3 * H * 4) + 2 * align256((size_t)H * 4) * conv_layers : 0;
  const size_t ssm_state_bytes = (size_t)c.ssm_heads * 32 * 128 * 4, mconv_bytes = (size_t)2 * c.ssm_conv * 3 * 4;
  sbytes += c.granite ? align256((size_t)ssm_proj * 4) + align256((size_t)c.ssm_inner * 4) +
                            (align256(ssm_state_bytes) + align256(mconv_bytes)) * mamba_layers
                      : 0;
  sbytes += 3 * align256((size_t)H * 4) + align256((size_t)(qdim + 2 * kvdim) * 4) + align256((size_t)qdim * 4) +
            align256((size_t)c.ffn * 4) + align256((size_t)c.vocab * 4) +
            align256((size_t)e->groups * 8) + align256(sizeof(DevState)) + align256(sizeof(DevSampling)) +
            2 * align256((size_t)(c.ctx + 1) * 4) + 2 * align256(bits_words * 4);
  const size_t dpart_bytes =
      e->dec_attn ? (size_t)c.kv_heads * e->dnchunk * attn_rowf(G, c.hd) * sizeof(tagged_t) : 0;
  sbytes += align256(dpart_bytes);
  const size_t qkv_tag_bytes = e->fuse_qkv ? (size_t)(qdim + 2 * kvdim) * sizeof(tagged_t) : 0;
  sbytes += align256(qkv_tag_bytes);
  e->state.reserve(sbytes);

  // weights
  e->embed = upload_matrix(e->weights, *src, g, tensor(g, "token_embd.weight"), H, c.vocab);
  if (c.lfm) {
    // LfmWgslEngine.create (:501-580): the embedding doubles as the lm_head
    e->lm_head = upload_class_major(e->weights, *src, g, tensor(g, "token_embd.weight"), H, c.vocab);
    e->final_norm = lfm_floats(e->weights, *src, g, "token_embd_norm.weight", H);
  } else if (c.granite) {
    // GraniteWgslEngine.create (:544-555): the embedding doubles as the lm_head
    e->lm_head = upload_class_major(e->weights, *src, g, tensor(g, "token_embd.weight"), H, c.vocab);
    e->final_norm = granite_floats(e->weights, *src, g, "output_norm.weight", H);
  } else {
    e->lm_head = tied ? e->embed : upload_matrix(e->weights, *src, g, tensor(g, lm_name), H, c.vocab);
    if (lm_lanes) e->lm_lanes = upload_lanes(e->weights, *src, g, tensor(g, lm_name), H, c.vocab);
    e->final_norm = upload_floats(e->weights, *src, g, "output_norm.weight", H);
  }
  for (int i = 0; i < (c.lfm ? c.layers : 0); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    LayerDev L;
    auto lin = [&](const std::string& name, int64_t K, int64_t N) {
      return upload_matrix(e->weights, *src, g, lfm_linear(g, p + name), K, N);
    };
    L.in_norm = lfm_floats(e->weights, *src, g, p + "attn_norm.weight", H);
    L.post_norm = lfm_floats(e->weights, *src, g, p + "ffn_norm.weight", H);
    if (lc.conv) {
      L.conv_w = lfm_floats(e->weights, *src, g, p + "shortconv.conv.weight", 3 * (int64_t)H);
      L.conv_in = lin("shortconv.in_proj.weight", H, 3 * (int64_t)H);
      L.conv_out = lin("shortconv.out_proj.weight", H, H);
    } else {
      L.q_norm = lfm_floats(e->weights, *src, g, p + "attn_q_norm.weight", c.hd);
      L.k_norm = lfm_floats(e->weights, *src, g, p + "attn_k_norm.weight", c.hd);
      L.q = lin("attn_q.weight", H, lc.heads * c.hd);
      L.k = lin("attn_k.weight", H, lc.kv_heads * c.hd);
      L.v = lin("attn_v.weight", H, lc.kv_heads * c.hd);
      L.o = lin("attn_output.weight", lc.heads * c.hd, H);
      L.kc = e->state.take(kv_bytes);
      L.vc = e->state.take(kv_bytes);
    }
    L.gate = lin("ffn_gate.weight", H, lc.ffn);
    L.up = lin("ffn_up.weight", H, lc.ffn);
    L.down = lin("ffn_down.weight", lc.ffn, H);
    if (L.gate.q.type != L.up.q.type)
      throw Error(CHONK_EINVAL, "ffn_gate and ffn_up of layer " + std::to_string(i) + " have different types");
    e->layers.push_back(L);
  }
  for (int i = 0; i < (c.granite ? c.layers : 0); ++i) {
    // GraniteWgslEngine.create's loadLayer (:571-624)
    const std::string p = "blk." + std::to_string(i) + ".";
    const LayerCfg& lc = c.layer[i];
    LayerDev L;
    auto lin = [&](const std::string& name, int64_t K, int64_t N) {
      return upload_matrix(e->weights, *src, g, granite_linear(g, p + name, K, N), K, N);
    };
    auto vec = [&](const std::string& name, int64_t n) { return granite_floats(e->weights, *src, g, p + name, n); };
    L.in_norm = vec("attn_norm.weight", H);
    L.post_norm = vec("ffn_norm.weight", H);
    if (lc.mamba) {
      L.ssm_in = lin("ssm_in.weight", H, ssm_proj);
      L.ssm_out = lin("ssm_out.weight", c.ssm_inner, H);
      const GgufTensorInfo& cw = granite_tensor(g, p + "ssm_conv1d.weight");
      if (cw.shape.size() != 2 || cw.shape[0] != 4 || (int64_t)cw.shape[1] != c.ssm_conv)
        throw Error(CHONK_EINVAL, "Granite WGSL tensor " + cw.name + " must be [4, " + std::to_string(c.ssm_conv) + "]");
      L.c1d_w = vec("ssm_conv1d.weight", 4 * (int64_t)c.ssm_conv);
      L.c1d_b = vec("ssm_conv1d.bias", c.ssm_conv);
      L.dt_b = vec("ssm_dt.bias", c.ssm_heads);
      L.a_neg = vec("ssm_a", c.ssm_heads);
      L.d_w = vec("ssm_d", c.ssm_heads);
      L.ssm_norm = vec("ssm_norm.weight", c.ssm_inner);
    } else {
      L.q = lin("attn_q.weight", H, lc.heads * c.hd);
      L.k = lin("attn_k.weight", H, lc.kv_heads * c.hd);
      L.v = lin("attn_v.weight", H, lc.kv_heads * c.hd);
      L.o = lin("attn_output.weight", lc.heads * c.hd, H);
      L.kc = e->state.take(kv_bytes);
      L.vc = e->state.take(kv_bytes);
    }
    L.gate = lin("ffn_gate.weight", H, lc.ffn);
    L.up = lin("ffn_up.weight", H, lc.ffn);
    L.down = lin("ffn_down.weight", lc.ffn, H);
    if (L.gate.q.type != L.up.q.type)
      throw Error(CHONK_EINVAL, "ffn_gate and ffn_up of layer " + std::to_string(i) + " have different types");
    e->layers.push_back(L);
  }
  if (c.gpt) {
    // GptWgslEngine buffers (gpt-wgsl-runtime.ts:540-640)
    e->final_norm_b = upload_floats(e->weights, *src, g, "output_norm.bias", H);
    e->pos_embd = upload_floats(e->weights, *src, g, "position_embd.weight", (int64_t)c.pos_rows * H);
    for (int i = 0; i < c.layers; ++i) {
      const std::string p = "blk." + std::to_string(i) + ".";
      LayerDev L;
      L.in_norm = upload_floats(e->weights, *src, g, p + "attn_norm.weight", H);
      L.in_norm_b = upload_floats(e->weights, *src, g, p + "attn_norm.bias", H);
      L.post_norm = upload_floats(e->weights, *src, g, p + "ffn_norm.weight", H);
      L.post_norm_b = upload_floats(e->weights, *src, g, p + "ffn_norm.bias", H);
      L.qkv = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_qkv.weight"), H, 3 * (int64_t)H);
      L.qkv_b = upload_floats(e->weights, *src, g, p + "attn_qkv.bias", 3 * (int64_t)H);
      L.o = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_output.weight"), H, H);
      L.o_b = upload_floats(e->weights, *src, g, p + "attn_output.bias", H);
      L.up = upload_matrix(e->weights, *src, g, tensor(g, p + "ffn_up.weight"), H, c.ffn);
      L.up_b = upload_floats(e->weights, *src, g, p + "ffn_up.bias", c.ffn);
      L.down = upload_matrix(e->weights, *src, g, tensor(g, p + "ffn_down.weight"), c.ffn, H);
      L.down_b = upload_floats(e->weights, *src, g, p + "ffn_down.bias", H);
      L.kc = e->state.take(kv_bytes);
      L.vc = e->state.take(kv_bytes);
      e->layers.push_back(L);
    }
  }
  for (int i = 0; i < (c.gpt || c.lfm || c.granite ? 0 : c.layers); ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    LayerDev L;
    L.in_norm = upload_floats(e->weights, *src, g, p + "attn_norm.weight", H);
    L.post_norm = upload_floats(e->weights, *src, g, p + (c.gemma ? "post_attention_norm.weight" : "ffn_norm.weight"), H);
    if (c.gemma) {
      L.pre_ffn_norm = upload_floats(e->weights, *src, g, p + "ffn_norm.weight", H);
      L.post_ffn_norm = upload_floats(e->weights, *src, g, p + "post_ffw_norm.weight", H);
    }
    if (c.qk_norm) {
      L.q_norm = upload_floats(e->weights, *src, g, p + "attn_q_norm.weight", c.hd);
      L.k_norm = upload_floats(e->weights, *src, g, p + "attn_k_norm.weight", c.hd);
    }
    const LayerCfg& lc = c.layer[i];
    const int lq = lc.heads * c.hd, lkv = lc.kv_heads * c.hd;
    if (c.openelm) {
      L.qkv = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_qkv.weight"), H, lq + 2 * lkv);
    } else {
      L.q = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_q.weight"), H, lq);
      L.k = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_k.weight"), H, lkv);
      L.v = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_v.weight"), H, lkv);
    }
    L.o = upload_matrix(e->weights, *src, g, tensor(g, p + "attn_output.weight"), lq, H);
    L.gate = upload_matrix(e->weights, *src, g, tensor(g, p + "ffn_gate.weight"), H, lc.ffn);
    L.up = upload_matrix(e->weights, *src, g, tensor(g, p + "ffn_up.weight"), H, lc.ffn);
    L.down = upload_matrix(e->weights, *src, g, tensor(g, p + "ffn_down.weight"), lc.ffn, H);
    if (L.gate.q.type != L.up.q.type)
      throw Error(CHONK_EINVAL, "ffn_gate and ffn_up of layer " + std::to_string(i) + " have different types");
    L.kc = e->state.take(kv_bytes);
    L.vc = e->state.take(kv_bytes);
    e->layers.push_back(L);
  }
  uint64_t wpt = e->lm_head.gguf_bytes + e->embed.gguf_bytes / c.vocab + (uint64_t)H * 4;
  for (const LayerDev& L : e->layers)
    wpt += L.q.gguf_bytes + L.k.gguf_bytes + L.v.gguf_bytes + L.qkv.gguf_bytes + L.o.gguf_bytes + L.gate.gguf_bytes +
           L.up.gguf_bytes + L.down.gguf_bytes + (uint64_t)H * 4 * (c.gemma || c.gpt ? 4 : 2) +
           (c.qk_norm && !L.conv_w ? 2ull * c.hd * 4 : 0) + (c.gpt ? 4ull * (5 * (uint64_t)H + c.ffn) : 0) +
           L.conv_in.gguf_bytes + L.conv_out.gguf_bytes + (L.conv_w ? 12ull * H : 0) + L.ssm_in.gguf_bytes +
           L.ssm_out.gguf_bytes + (L.c1d_w ? 4ull * (5ull * c.ssm_conv + 3ull * c.ssm_heads + c.ssm_inner) : 0);
  if (c.gpt) wpt += 8ull * H;  // final LayerNorm bias, the position row
  e->weight_bytes_per_token = wpt;

  e->resA = (float*)e->state.take((size_t)H * 4);
  e->resB = (float*)e->state.take((size_t)H * 4);
  e->delta = (float*)e->state.take((size_t)H * 4);
  e->qkv = (float*)e->state.take((size_t)(qdim + 2 * kvdim) * 4);
  e->attn = (float*)e->state.take((size_t)qdim * 4);
  e->ff = (float*)e->state.take((size_t)c.ffn * 4);
  e->logits = (float*)e->state.take((size_t)c.vocab * 4);
  e->cand = (Candidate*)e->state.take((size_t)e->groups * 8);
  if (c.lfm) {
    // the convolution states start at zero with the rest of this region
    e->conv_proj = (float*)e->state.take((size_t)3 * H * 4);
    for (size_t i = 0; i < e->layers.size(); ++i) {
      if (!c.layer[i].conv) continue;
      e->layers[i].conv_s1 = (float*)e->state.take((size_t)H * 4);
      e->layers[i].conv_s2 = (float*)e->state.take((size_t)H * 4);
    }
  }
  if (c.granite) {
    e->mproj = (float*)e->state.take((size_t)ssm_proj * 4);
    e->my = (float*)e->state.take((size_t)c.ssm_inner * 4);
    for (size_t i = 0; i < e->layers.size(); ++i) {
      if (!c.layer[i].mamba) continue;
      e->layers[i].ssm_state = (float*)e->state.take(ssm_state_bytes);
      e->layers[i].mconv_state = (float*)e->state.take(mconv_bytes);
    }
  }
  {
    const size_t rowf = ((size_t)G * (c.hd + 2) + 3) & ~(size_t)3;
    const size_t part_bytes = align256((size_t)c.kv_heads * std::max(e->nchunk, e->dnchunk) * rowf * 4);
    e->uncached = uncached_pool().take(e->device, part_bytes + align256((size_t)c.kv_heads * 4));
    e->part = (float*)e->uncached;
    e->cnt = (uint32_t*)((uint8_t*)e->uncached + part_bytes);
    HIP_OK(hipMemset(e->cnt, 0, (size_t)c.kv_heads * 4));
  }
  if (e->dec_attn) e->dpart = (tagged_t*)e->state.take(dpart_bytes);
  if (e->fuse_qkv) e->qkv_tag = (tagged_t*)e->state.take(qkv_tag_bytes);
  e->st = (DevState*)e->state.take(sizeof(DevState));
  e->samp = (DevSampling*)e->state.take(sizeof(DevSampling));
  e->hist = (int32_t*)e->state.take((size_t)(c.ctx + 1) * 4);
  e->gen = (int32_t*)e->state.take((size_t)(c.ctx + 1) * 4);
  e->pen_bits = (uint32_t*)e->state.take(bits_words * 4);
  e->seen_bits = (uint32_t*)e->state.take(bits_words * 4);
  HIP_OK(hipMemset((void*)e->resA, 0, e->state.capacity() - 2 * align256(kv_bytes) * kv_layers));
  // chunk rows start with tag 0xffffffff, which no launch uses (epochs start at 0)
  if (e->dpart) HIP_OK(hipMemset(e->dpart, 0xff, dpart_bytes));
  if (e->qkv_tag) HIP_OK(hipMemset(e->qkv_tag, 0xff, qkv_tag_bytes));
  for (const LayerDev& L : e->layers) {
    if (!L.kc) continue;
    HIP_OK(hipMemset(L.kc, 0, kv_bytes));
    HIP_OK(hipMemset(L.vc, 0, kv_bytes));
  }
  HIP_OK(hipHostMalloc((void**)&e->h_state, sizeof(DevState), hipHostMallocDefault));
  HIP_OK(hipHostMalloc((void**)&e->h_tok, 64, hipHostMallocDefault));
  HIP_OK(hipHostMalloc((void**)&e->h_samp, sizeof(DevSampling), hipHostMallocDefault));
  std::memset(e->h_samp, 0, sizeof(DevSampling));
  HIP_OK(hipDeviceSynchronize());

  HIP_OK(init_kernel_attributes());
  HIP_OK(init_gemm_attributes());
  build_steps(e.get(), false);
  if (e->fuse_qkv) {
    e->step_logits_sep = e->kernels_logits;
    e->step_plain_sep = e->kernels_plain;
    build_steps(e.get(), true);
    bool any = false;
    for (const Launch& L : e->kernels_logits) any = any || L.kind == Launch::QKVATTN;
    e->fuse_qkv = any;  // (no layer qualified: one set of steps)
  }
  e->step_logits = e->kernels_logits;
  e->step_plain = e->kernels_plain;
  // CHONK_PREFILL=token keeps the reference's token-by-token prompt pass
  const char* pv = std::getenv("CHONK_PREFILL");
  // (the row-batch glue kernels hold a row of at most 4096 elements in registers)
  e->batched_prefill = !(pv && std::strcmp(pv, "token") == 0) && !c.gpt && !c.lfm && !c.granite &&
                       std::max(c.hidden, std::max(c.heads * c.hd, c.ffn)) <= 4096;
  // the no-allocation prompt pass: as many rows (a multiple of 16, at most one
  // full pass) as fit the scratch with this model's row buffers
  e->scratch = scratch_address(e->device);
  e->noalloc_rows = e->batched_prefill ? noalloc_rows_for(c) : 0;
  const char* ng = std::getenv("CHONK_NO_GRAPH");
  e->use_graph = !(ng && ng[0] == '1');
  for (const Launch& L : e->kernels_logits)
    if (L.shmem > lds_limit())
      throw Error(CHONK_EINVAL, "kernel " + L.name + " needs " + std::to_string(L.shmem) + " bytes of LDS, above the " +
                                    std::to_string(lds_limit()) + "-byte limit of this device");
  capture(e.get(), e->step_plain, &e->graph_plain, &e->exec_plain);
  capture(e.get(), e->step_logits, &e->graph_logits, &e->exec_logits);
  if (e->use_graph) capture(e.get(), e->step_logits, &e->graph_multi, &e->exec_multi, kMultiSteps);
  if (e->fuse_qkv) {
    capture(e.get(), e->step_plain_sep, &e->graph_plain_sep, &e->exec_plain_sep);
    capture(e.get(), e->step_logits_sep, &e->graph_logits_sep, &e->exec_logits_sep);
  }
  *out = e.release();
}

// The test hook's stand-in for a failed launch: the same error path as a HIP
// error returned by the runtime (the caller marks the engine lost).
void check_injected_failure(chonk_engine* e, const char* where) {
  if (!e->fail_next_launch) return;
  e->fail_next_launch = false;
  throw Error(CHONK_EHIP, std::string("HIP error hipErrorLaunchFailure (injected by "
                                      "chonk_engine_debug_fail_next_launch) at ") + where);
}

// n consecutive decode steps with no host work between them: graph replays,
// or (CHONK_NO_GRAPH=1, for profilers that cannot trace graph launches) the
// same launches issued one by one. Runs of kMultiSteps logits steps replay the
// multi-step graph. An engine with fused steps replays them (and the
// multi-step graph) only while it is alone on its device.
void replay(chonk_engine* e, bool logits, int64_t n = 1) {
  while (n > 0) {
    check_injected_failure(e, "hipGraphLaunch");
    std::unique_lock<std::mutex> l;
    bool sep = false;
    if (e->fuse_qkv) {
      DeviceEngines& d = device_engines();
      l = std::unique_lock<std::mutex>(d.mu);
      sep = d.live[e->device].size() > 1;
    }
    if (e->use_graph) {
      if (logits && !sep && e->exec_multi && n >= kMultiSteps && !multi_off()) {
        HIP_OK(hipGraphLaunch(e->exec_multi, e->stream));
        n -= kMultiSteps;
        continue;
      }
      hipGraphExec_t x = logits ? (sep ? e->exec_logits_sep : e->exec_logits) : (sep ? e->exec_plain_sep : e->exec_plain);
      HIP_OK(hipGraphLaunch(x, e->stream));
    } else {
      for (const Launch& L : logits ? (sep ? e->step_logits_sep : e->step_logits) : (sep ? e->step_plain_sep : e->step_plain))
        enqueue(L, e->stream);
    }
    --n;
  }
}

void upload_state_fields(chonk_engine* e, const DevState& s) {
  *e->h_state = s;
  HIP_OK(hipMemcpyAsync(e->st, e->h_state, sizeof(DevState), hipMemcpyHostToDevice, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
}

DevState read_state(chonk_engine* e) {
  HIP_OK(hipMemcpyAsync(e->h_state, e->st, sizeof(DevState), hipMemcpyDeviceToHost, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  return *e->h_state;
}

// JS Math.round for the penalty milli value (round half up).
double js_round(double x) { return std::floor(x + 0.5); }

DevSampling make_sampling(chonk_engine* e, const chonk_sampling* s, bool stage1, bool seen) {
  DevSampling d{};
  const double temperature = s ? s->temperature : 0.0;
  const double top_p = s ? s->top_p : 1.0;
  int top_k = s ? s->top_k : 0;
  const double rp = s ? s->repetition_penalty : 1.0;
  if (top_k < 0) top_k = 0;
  d.temperature = temperature;
  d.top_p = std::min(std::max(top_p, 0.0), 1.0);
  d.top_k = top_k;
  d.seed = s ? s->seed : 0;
  d.sample_mode = (temperature > 0 || top_p < 1 || top_k > 0) ? 1 : 0;  // needsSamplingReadback
  // the LFM runtime also takes the candidate path for any penalty other than 1
  // (needsCandidateReadback, sampling.ts:18-21; lfm-wgsl-runtime.ts:787-806)
  if ((e->cfg.lfm || e->cfg.granite) && rp != 1.0) d.sample_mode = 1;
  // the caller decides: llama applies the list when rp > 1 (:1649-1661), the
  // GPT-2 runtime whenever rp != 1 (gpt-wgsl-runtime.ts:789-798)
  d.stage1_penalty = stage1 ? 1 : 0;
  d.stage1_pen = (float)js_round(rp * 1000) / 1000.0f;
  d.repetition_penalty = std::max(rp, 1e-6);
  d.seen_penalty = seen && d.repetition_penalty != 1 ? 1 : 0;
  d.n_eos = (int32_t)e->eos.size();
  for (int i = 0; i < d.n_eos && i < 16; ++i) d.eos[i] = e->eos[i];
  return d;
}

void upload_sampling(chonk_engine* e, const DevSampling& d) {
  if (e->samp_valid && std::memcmp(&e->last_samp, &d, sizeof d) == 0) return;
  *e->h_samp = d;
  HIP_OK(hipMemcpyAsync(e->samp, e->h_samp, sizeof d, hipMemcpyHostToDevice, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  e->last_samp = d;
  e->samp_valid = true;
}

void upload_bits(chonk_engine* e, uint32_t* dst, const int32_t* ids, size_t n) {
  std::vector<uint32_t> bits((size_t)(e->cfg.vocab + 31) / 32, 0u);
  for (size_t i = 0; i < n; ++i) {
    const int32_t id = ids[i];
    if (id >= 0 && id < e->cfg.vocab) bits[(size_t)id >> 5] |= 1u << (id & 31);
  }
  HIP_OK(hipMemcpy(dst, bits.data(), bits.size() * 4, hipMemcpyHostToDevice));
}

void put_token(chonk_engine* e, int position, int32_t token) {
  if (e->known_token_pos == position && e->known_token == token) return;
  *e->h_tok = token;
  HIP_OK(hipMemcpyAsync(e->hist + position, e->h_tok, 4, hipMemcpyHostToDevice, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  e->known_token_pos = position;
  e->known_token = token;
}

// The context error in the wording of the engine's runtime
// (llama-wgsl-runtime.ts:1032, gpt-wgsl-runtime.ts:751-753, lfm-wgsl-runtime.ts:732-734).
Error context_exhausted(const chonk_engine* e) {
  const char* name = e->cfg.gpt ? "GPT" : e->cfg.lfm ? "LFM" : e->cfg.granite ? "Granite" : "Llama";
  return Error(CHONK_ECONTEXT, std::string(name) + " WGSL context exhausted at " + std::to_string(e->cfg.ctx) + " tokens");
}

void check_token(const chonk_engine* e, int32_t token) {
  if (token < 0 || token >= e->cfg.vocab)
    throw Error(CHONK_EINVAL, "token id " + std::to_string(token) + " outside embedding table");
}

void engine_reset(chonk_engine* e) {
  HIP_OK(hipStreamSynchronize(e->stream));
  const size_t kv_bytes = (size_t)e->cfg.kv_heads * e->cfg.hd * e->cfg.ctx * e->kv_elem;
  for (const LayerDev& L : e->layers) {
    if (L.kc) {
      HIP_OK(hipMemsetAsync(L.kc, 0, kv_bytes, e->stream));
      HIP_OK(hipMemsetAsync(L.vc, 0, kv_bytes, e->stream));
    }
    if (L.conv_s1) {  // LfmWgslEngine.reset clears each convolution state (:711-724)
      HIP_OK(hipMemsetAsync(L.conv_s1, 0, (size_t)e->cfg.hidden * 4, e->stream));
      HIP_OK(hipMemsetAsync(L.conv_s2, 0, (size_t)e->cfg.hidden * 4, e->stream));
    }
    if (L.ssm_state) {  // GraniteWgslEngine.reset clears each conv and SSM state (:750-763)
      HIP_OK(hipMemsetAsync(L.ssm_state, 0, (size_t)e->cfg.ssm_heads * 32 * 128 * 4, e->stream));
      HIP_OK(hipMemsetAsync(L.mconv_state, 0, (size_t)2 * e->cfg.ssm_conv * 3 * 4, e->stream));
    }
  }
  DevState s{};
  upload_state_fields(e, s);
  e->pos = 0;
  e->known_token_pos = -1;
  e->logits_valid = false;
}

// The error a step reported.
Error device_error(chonk_engine* e, const DevState& st) {
  (void)e;
  return Error(CHONK_EHIP, "device reported error code " + std::to_string(st.error));
}

// ---- row batches: prompt pass and batched decode ---------------------------------------

constexpr int kPrefillRows = 2048;  // prompt rows per pass (longer prompts take several)
constexpr int64_t kPartFloats = (int64_t)4 << 20;  // K-split partial sums

// Device buffers of a row batch (rows <= cap).
struct RowBufs {
  float *x = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr, *u = nullptr, *act = nullptr, *d = nullptr,
        *xscale = nullptr, *part = nullptr;
  _Float16 *h = nullptr, *l = nullptr;
  int32_t* tok = nullptr;
  int cap = 0;
  int64_t part_cap = 0;  // floats in part
};

// Floats of the partial-sum buffer for `rows` rows: room for every deferred
// GEMM result of a layer without a K split, and at least kPartFloats.
int64_t row_part_floats(const ModelCfg& c, int rows) {
  const int64_t R = rows;
  const int64_t qkv = (int64_t)(c.heads + 2 * c.kv_heads) * c.hd;
  return std::max<int64_t>({kPartFloats, R * qkv, 2 * R * c.ffn, R * c.hidden});
}

// Sizes the buffers of `rows` rows for the engine's model; returns the bytes
// needed and, with base != null, carves them from base.
size_t row_bufs_layout(const ModelCfg& c, int rows, uint8_t* base, RowBufs* out) {
  const size_t R = rows;
  const size_t H = c.hidden, qdim = (size_t)c.heads * c.hd, kvdim = (size_t)c.kv_heads * c.hd, F = c.ffn;
  const size_t kmax = gemm_kpad((int)std::max(H, std::max(qdim, F)));
  const size_t sizes[12] = {R * H * 4, R * (qdim + 2 * kvdim) * 4, R * qdim * 4, R * F * 4, R * F * 4, R * F * 4,
                            R * H * 4, R * 4, (size_t)row_part_floats(c, rows) * 4, R * kmax * 2, R * kmax * 2, R * 4};
  size_t off = 0;
  void* ptr[12];
  for (int i = 0; i < 12; ++i) {
    ptr[i] = base ? base + off : nullptr;
    off += align256(sizes[i]);
  }
  if (out) {
    out->x = (float*)ptr[0];
    out->qkv = (float*)ptr[1];
    out->att = (float*)ptr[2];
    out->g = (float*)ptr[3];
    out->u = (float*)ptr[4];
    out->act = (float*)ptr[5];
    out->d = (float*)ptr[6];
    out->xscale = (float*)ptr[7];
    out->part = (float*)ptr[8];
    out->h = (_Float16*)ptr[9];
    out->l = (_Float16*)ptr[10];
    out->tok = (int32_t*)ptr[11];
    out->cap = rows;
    out->part_cap = row_part_floats(c, rows);
  }
  return off;
}

// K/V placement of a row batch: per-layer caches, optionally paged.
struct RowKv {
  std::vector<void*> kc, vc;
  int ctx = 0;
  const int32_t* pages = nullptr;
  int max_pages = 0;
};

// Where the rows sit: positions p0 + row of sequence seq0, or per-row arrays.
struct RowPlace {
  int p0 = 0, seq0 = 0;
  const int32_t* row_seq = nullptr;  // device [rows]
  const int32_t* row_pos = nullptr;  // device [rows]
};

// The layers for rows 0..T-1 whose token ids are in b.tok: every layer's K/V
// of the rows into the cache; with logits != null also the last layer's
// attention and MLP and the final norm and lm_head of rows [lr0, lr0 + nlr)
// into logits ([nlr][vocab]). Launches on s; does not synchronize.
void run_rows(chonk_engine* e, const RowBufs& b, const RowKv& kvs, const RowPlace& pl, int T, float* logits, int lr0,
              int nlr, hipStream_t s) {
  const ModelCfg& c = e->cfg;
  const int H = c.hidden;
  // split of x into the GEMM operand planes, after the pending residual update
  // (x += add, or the Gemma-3 sandwich with add_w) when add.p is set
  auto split = [&](const float* x, int ld, int k, const float* w, int rows, PartSum add, const float* add_w) {
    PfSplitArgs a{};
    a.x = x;
    a.ldx = ld;
    a.k = k;
    a.kpad = gemm_kpad(k);
    a.w = w;
    a.eps = c.eps;
    a.xh = b.h;
    a.xl = b.l;
    a.xscale = b.xscale;
    a.add = add;
    a.add_w = add_w;
    HIP_OK(launch_pf_split(a, rows, s));
  };
  // GEMM of the operand planes with the result left as partial sums in
  // part[off, off + cap) (the consumer kernel adds them)
  auto gemm = [&](const DevMat& m, int rows, int64_t off, int64_t cap) {
    GemmArgs g{};
    g.w = m.q;
    g.xh = b.h;
    g.xl = b.l;
    g.xscale = b.xscale;
    g.t = rows;
    g.kpad = gemm_kpad(m.q.k);
    g.ws = m.ws;
    PartSum ps{};
    HIP_OK(launch_gemm_deferred(g, b.part + off, cap, &ps, s));
    return ps;
  };
  // one launch over two or three matrices of one type and K whose results are
  // column ranges of one partial-sum row (segments start on 64-row tiles);
  // returns false (nothing launched) when the matrices do not qualify
  auto gemm_fused = [&](std::initializer_list<const DevMat*> ms, int rows, PartSum* out) {
    std::vector<const DevMat*> m(ms);
    for (size_t i = 1; i < m.size(); ++i)
      if (m[i]->q.type != m[0]->q.type || m[i]->q.k != m[0]->q.k || m[i - 1]->q.n % 64 != 0) return false;
    GemmArgs g{};
    g.w = m[0]->q;
    g.w2 = m[1]->q;
    g.w3 = m.size() > 2 ? m[2]->q : m[1]->q;
    g.n1 = m[0]->q.n;
    g.n2 = g.n1 + m[1]->q.n;
    g.n_all = g.n2 + (m.size() > 2 ? m[2]->q.n : 0);
    g.xh = b.h;
    g.xl = b.l;
    g.xscale = b.xscale;
    g.t = rows;
    g.kpad = gemm_kpad(m[0]->q.k);
    g.ws = m[0]->ws;
    for (const DevMat* d : m) g.ws = std::min(g.ws, d->ws);  // every matrix stays below 2^14
    HIP_OK(launch_gemm_deferred(g, b.part, b.part_cap, out, s));
    return true;
  };
  // column range [c0, c0 + n) of a fused result
  auto columns = [](PartSum p, int c0, int n) {
    p.p += c0;
    p.n = n;
    return p;
  };
  auto kv_addr = [&](int i) {
    KvAddr k{};
    k.kc = kvs.kc[i];
    k.vc = kvs.vc[i];
    k.ctx = kvs.ctx;
    k.pages = kvs.pages;
    k.max_pages = kvs.max_pages;
    k.seq0 = pl.seq0;
    k.row_seq = pl.row_seq;
    k.row_pos = pl.row_pos;
    k.p0 = pl.p0;
    return k;
  };
  const int64_t P = b.part_cap;
  HIP_OK(launch_pf_embed(e->embed.q, b.tok, c.embed_scale, H, b.x, T, s));
  PartSum pending{};                // the previous layer's ffn_down, not yet added to x
  const float* pending_w = nullptr; // its Gemma-3 post-ffn norm
  for (int i = 0; i < c.layers; ++i) {
    const LayerDev& L = e->layers[i];
    const LayerCfg& lc = c.layer[i];
    const int qdim = lc.heads * c.hd, kvdim = lc.kv_heads * c.hd, F = lc.ffn;
    const int ldqkv = qdim + 2 * kvdim;
    split(b.x, H, H, L.in_norm, T, pending, pending_w);
    pending = PartSum{};
    PfRopeArgs r{};
    PartSum fused{};
    if (c.openelm) {
      // one fused q|k|v result; k and v are column ranges of it
      const PartSum f = gemm(L.qkv, T, 0, P);
      r.pq = columns(f, 0, qdim);
      r.pk = columns(f, qdim, kvdim);
      r.pv = columns(f, qdim + kvdim, kvdim);
    } else if (gemm_fused({&L.q, &L.k, &L.v}, T, &fused)) {
      r.pq = columns(fused, 0, qdim);
      r.pk = columns(fused, qdim, kvdim);
      r.pv = columns(fused, qdim + kvdim, kvdim);
    } else {
      // the partial-sum buffer shared out in proportion to each result's size
      const int64_t pq = P * qdim / ldqkv, pk = P * kvdim / ldqkv;
      r.pq = gemm(L.q, T, 0, pq);
      r.pk = gemm(L.k, T, pq, pk);
      r.pv = gemm(L.v, T, pq + pk, P - pq - pk);
    }
    r.qkv = b.qkv;
    r.ld = ldqkv;
    r.hd = c.hd;
    r.heads = lc.heads;
    r.kv_heads = lc.kv_heads;
    r.interleaved = c.interleaved ? 1 : 0;
    r.kv16 = e->kv_elem == 2 ? 1 : 0;
    r.qn_w = c.qk_norm ? L.q_norm : nullptr;
    r.kn_w = c.qk_norm ? L.k_norm : nullptr;
    r.eps = c.qk_eps;
    r.rope_inv = rope_table(e, c.layer[i].theta, c.hd);
    r.kv = kv_addr(i);
    const bool last_kv = i == c.layers - 1 && !logits;  // only the last layer's K/V are needed from it
    // decode batches: the page-walking attention (one workgroup per (kv head,
    // row) walking all of its pages also does the rotary/K-V write)
    const bool walk = pl.row_seq && c.hd >= 64 && lc.heads / lc.kv_heads <= 8 && kvs.max_pages <= 64;
    const bool fuse_rope = walk && !last_kv && bd_attn_segments(T, lc.kv_heads, kvs.max_pages) == 1;
    if (!fuse_rope) HIP_OK(launch_pf_rope_kv(r, T, s));
    if (last_kv) break;
    PfAttnArgs at{};
    at.qkv = b.qkv;
    at.ld = ldqkv;
    at.out = b.att;
    at.ldo = qdim;
    at.heads = lc.heads;
    at.kv_heads = lc.kv_heads;
    at.hd = c.hd;
    at.window = c.layer[i].window;
    at.kv16 = r.kv16;
    at.scale = c.scale;
    at.kv = r.kv;
    bool planes = false;  // the attention wrote the o-projection's operand planes
    if (walk) {
      at.oh = b.h;
      at.ol = b.l;
      at.oscale = b.xscale;
      at.okpad = gemm_kpad(qdim);
      HIP_OK(launch_bd_attn(at, T, b.part, P, s, &planes, fuse_rope ? &r : nullptr));
    } else {
      HIP_OK(launch_pf_attn(at, T, s));
    }
    if (!planes) split(b.att, qdim, qdim, nullptr, T, PartSum{}, nullptr);
    const PartSum po = gemm(L.o, T, 0, P);
    // x += o (Gemma-3: x = clamp(x + RMSNorm(o) * post_norm)), then the ffn norm
    split(b.x, H, H, c.gemma ? L.pre_ffn_norm : L.post_norm, T, po, c.gemma ? L.post_norm : nullptr);
    PfGluArgs gl{};
    PartSum gu{};
    if (gemm_fused({&L.gate, &L.up}, T, &gu)) {
      gl.pg = columns(gu, 0, F);
      gl.pu = columns(gu, F, F);
    } else {
      gl.pg = gemm(L.gate, T, 0, P / 2);
      gl.pu = gemm(L.up, T, P / 2, P - P / 2);
    }
    gl.act = b.act;
    gl.k = F;
    gl.kpad = gemm_kpad(F);
    gl.gelu = c.gemma ? 1 : 0;
    gl.xh = b.h;
    gl.xl = b.l;
    gl.xscale = b.xscale;
    HIP_OK(launch_pf_glu_split(gl, T, s));
    pending = gemm(L.down, T, 0, P);
    pending_w = c.gemma ? L.post_ffn_norm : nullptr;
  }
  if (logits) {
    PartSum add = pending;
    if (add.p) add.p += (int64_t)lr0 * add.ld;  // rows [lr0, lr0 + nlr) of the result
    split(b.x + (size_t)lr0 * H, H, H, e->final_norm, nlr, add, pending_w);
    GemmArgs g{};
    g.w = e->lm_head.q;
    g.xh = b.h;
    g.xl = b.l;
    g.xscale = b.xscale;
    g.y = logits;
    g.ldy = c.vocab;
    g.t = nlr;
    g.kpad = gemm_kpad(e->lm_head.q.k);
    g.epi = GEMM_STORE;
    g.ws = e->lm_head.ws;
    g.part = b.part;
    g.part_cap = P;
    HIP_OK(launch_gemm(g, s));
  }
}

// The largest multiple of 16 rows, at most one full pass, whose row buffers fit
// the no-allocation scratch (0 when not even 16 rows fit).
int noalloc_rows_for(const ModelCfg& c) {
  for (int r = kPrefillRows; r >= 16; r -= 16)
    if (row_bufs_layout(c, r, nullptr, nullptr) <= kNoAllocScratchBytes) return r;
  return 0;
}

void prefill_alloc(chonk_engine* e) {
  if (e->pf_mem) return;
  RowBufs b;
  const size_t bytes = row_bufs_layout(e->cfg, kPrefillRows, nullptr, nullptr);
  HIP_OK(hipMalloc(&e->pf_mem, bytes));
  row_bufs_layout(e->cfg, kPrefillRows, (uint8_t*)e->pf_mem, &b);
  e->pf_x = b.x;
  e->pf_qkv = b.qkv;
  e->pf_att = b.att;
  e->pf_g = b.g;
  e->pf_u = b.u;
  e->pf_act = b.act;
  e->pf_d = b.d;
  e->pf_xscale = b.xscale;
  e->pf_part = b.part;
  e->pf_h = b.h;
  e->pf_l = b.l;
  e->pf_tok = b.tok;
}

RowBufs engine_row_bufs(const chonk_engine* e) {
  RowBufs b;
  b.x = e->pf_x;
  b.qkv = e->pf_qkv;
  b.att = e->pf_att;
  b.g = e->pf_g;
  b.u = e->pf_u;
  b.act = e->pf_act;
  b.d = e->pf_d;
  b.xscale = e->pf_xscale;
  b.part = e->pf_part;
  b.h = e->pf_h;
  b.l = e->pf_l;
  b.tok = e->pf_tok;
  b.cap = kPrefillRows;
  b.part_cap = row_part_floats(e->cfg, kPrefillRows);
  return b;
}

// K/V of every layer for tokens[0, n) at positions e->pos .. e->pos + n - 1,
// computed as row batches (dequant-fused MFMA GEMMs, causal attention over the
// cache). The host position and the device state are left to the caller; no
// logits are produced (the reference's runToken(id, false) for each token).
void prefill_rows_in(chonk_engine* e, const RowBufs& b, const int32_t* tokens, int n);

void prefill_rows(chonk_engine* e, const int32_t* tokens, int n) {
  if (n <= 0) return;
  prefill_alloc(e);
  prefill_rows_in(e, engine_row_bufs(e), tokens, n);
}

// The same pass with row buffers b (passes of at most b.cap rows).
void prefill_rows_in(chonk_engine* e, const RowBufs& b, const int32_t* tokens, int n) {
  check_injected_failure(e, "the prompt pass");
  const ModelCfg& c = e->cfg;
  if (n <= 0) return;
  if ((int64_t)e->pos + n > c.ctx)
    throw context_exhausted(e);
  RowKv kvs;
  for (const LayerDev& L : e->layers) {
    kvs.kc.push_back(L.kc);
    kvs.vc.push_back(L.vc);
  }
  kvs.ctx = c.ctx;
  for (int off = 0; off < n; off += b.cap) {
    const int T = std::min(b.cap, n - off);
    HIP_OK(hipMemcpyAsync(b.tok, tokens + off, (size_t)T * 4, hipMemcpyHostToDevice, e->stream));
    RowPlace pl;
    pl.p0 = e->pos + off;
    run_rows(e, b, kvs, pl, T, nullptr, 0, 0, e->stream);
  }
  HIP_OK(hipStreamSynchronize(e->stream));
}

int32_t run_token(chonk_engine* e, int32_t token, bool need_logits, const chonk_sampling* s, const int32_t* pen,
                  size_t n_pen, const int32_t* seen, size_t n_seen) {
  if (e->pos >= e->cfg.ctx)
    throw context_exhausted(e);
  check_token(e, token);
  put_token(e, e->pos, token);
  if (need_logits) {
    // argmax(): the penalty list is the last `context` ids (:1649-1653)
    const double rp = s ? s->repetition_penalty : 1.0;
    // (the GPT-2 runtime applies the list whenever the penalty is not 1, :785-796)
    // (the LFM runtime has no penalty list: its penalty acts on the candidates)
    const bool stage1 = !e->cfg.lfm && !e->cfg.granite && (e->cfg.gpt ? rp != 1.0 : rp > 1) && n_pen > 0;
    const size_t keep = std::min(n_pen, (size_t)e->cfg.ctx);
    if (stage1) upload_bits(e, e->pen_bits, pen + (n_pen - keep), keep);
    const DevSampling d = make_sampling(e, s, stage1, n_seen > 0);
    if (d.sample_mode && d.seen_penalty) upload_bits(e, e->seen_bits, seen, n_seen);
    upload_sampling(e, d);
    replay(e, true);
    HIP_OK(hipMemcpyAsync(e->h_state, e->st, sizeof(DevState), hipMemcpyDeviceToHost, e->stream));
    HIP_OK(hipStreamSynchronize(e->stream));
    const DevState st = *e->h_state;
    if (st.error) throw device_error(e, st);
    e->pos += 1;
    e->known_token_pos = e->pos;
    e->known_token = st.last_token;
    e->logits_valid = true;
    return st.last_token;
  }
  replay(e, false);
  e->pos += 1;
  return 0;
}

int64_t common_prefix(const std::vector<int32_t>& a, const int32_t* b, size_t nb) {
  const size_t n = std::min(a.size(), nb);
  size_t i = 0;
  while (i < n && a[i] == b[i]) ++i;
  return (int64_t)i;
}

double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// generateLlamaWgsl's option defaults (:255-262): temperature 0, topP 1,
// topK 0, repetitionPenalty = opts ?? def.defaultRepetitionPenalty ?? 1
// (a non-positive or non-finite value means "not given"). generateGptWgsl and
// generateLfmWgsl take opts.repetitionPenalty ?? 1 and ignore the definition's
// default (gpt-wgsl-runtime.ts:198-203, lfm-wgsl-runtime.ts:236-241).
chonk_sampling effective_sampling(const chonk_engine* e, const chonk_sampling* s_in) {
  chonk_sampling s{};
  s.temperature = 0;
  s.top_p = 1;
  s.top_k = 0;
  s.repetition_penalty =
      (!e->cfg.gpt && !e->cfg.lfm && !e->cfg.granite && e->def.default_repetition_penalty > 0)
          ? e->def.default_repetition_penalty
          : 1.0;
  if (s_in) {
    s.temperature = s_in->temperature;
    s.top_p = s_in->top_p;
    s.top_k = s_in->top_k;
    s.seed = s_in->seed;
    if (s_in->repetition_penalty > 0 && std::isfinite(s_in->repetition_penalty)) s.repetition_penalty = s_in->repetition_penalty;
  }
  return s;
}

void generate(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new, const chonk_sampling* s_in,
              std::vector<int32_t>* out, chonk_gen_stats* stats) {
  const ModelCfg& c = e->cfg;
  // maxNewTokens ?? 128 (:255): a negative value stands for "not given"
  const int64_t max = std::min<int64_t>(max_new >= 0 ? max_new : 128, (int64_t)e->def.max_context - (int64_t)n_prompt);
  const chonk_sampling s = effective_sampling(e, s_in);
  for (size_t i = 0; i < n_prompt; ++i) check_token(e, prompt[i]);
  const double t0 = now_ms();
  int64_t prefix = common_prefix(e->cached_ids, prompt, n_prompt);
  if (prefix != (int64_t)e->cached_ids.size()) {
    engine_reset(e);
    e->cached_ids.clear();
    e->has_cached_next = false;
    prefix = 0;
  }
  const size_t n_suffix = n_prompt - (size_t)prefix;
  if ((int64_t)e->pos + (int64_t)n_suffix > c.ctx)
    throw context_exhausted(e);
  auto is_eos = [&](int32_t id) { return std::find(e->eos.begin(), e->eos.end(), id) != e->eos.end(); };

  // penalty list = prompt (+ generated ids, appended on the device)
  const bool stage1 = !c.lfm && !c.granite && s.repetition_penalty > 1;
  DevSampling d = make_sampling(e, &s, stage1, true);
  if (stage1 || d.seen_penalty) {
    upload_bits(e, e->pen_bits, prompt, n_prompt);
    upload_bits(e, e->seen_bits, prompt, n_prompt);
  }
  upload_sampling(e, d);

  DevState st{};
  st.pos = e->pos;
  st.generating = max > 0 ? 1 : 0;
  st.max_generated = (int32_t)std::max<int64_t>(max, 0);
  int32_t next = 0;
  bool need_decode_seed = false;
  double t_prefill_end = t0;
  if (n_suffix == 0) {
    next = e->has_cached_next ? e->cached_next : 0;
    need_decode_seed = true;
  } else {
    std::vector<int32_t> suf(prompt + prefix, prompt + n_prompt);
    HIP_OK(hipMemcpy(e->hist + e->pos, suf.data(), suf.size() * 4, hipMemcpyHostToDevice));
    if (e->batched_prefill && n_suffix > 1) {
      // all but the last prompt token as row batches, the last one as a step
      prefill_rows(e, suf.data(), (int)n_suffix - 1);
      st.pos = e->pos + (int)n_suffix - 1;
      upload_state_fields(e, st);
    } else {
      upload_state_fields(e, st);
      for (size_t i = 0; i + 1 < n_suffix; ++i) replay(e, false);
    }
    replay(e, true);
    st = read_state(e);
    if (st.error) throw device_error(e, st);
    e->pos = st.pos;
    next = st.last_token;
    e->logits_valid = true;
    t_prefill_end = now_ms();
  }
  std::vector<int32_t> generated;
  if (max > 0) {
    if (need_decode_seed) {
      // first generated id comes from the cache (or is 0); seed the device loop with it
      *e->h_tok = next;
      HIP_OK(hipMemcpy(e->hist + e->pos, e->h_tok, 4, hipMemcpyHostToDevice));
      HIP_OK(hipMemcpy(e->gen, e->h_tok, 4, hipMemcpyHostToDevice));
      if (stage1 || d.seen_penalty) {
        std::vector<int32_t> ids(prompt, prompt + n_prompt);
        ids.push_back(next);
        upload_bits(e, e->pen_bits, ids.data(), ids.size());
        upload_bits(e, e->seen_bits, ids.data(), ids.size());
      }
      st.pos = e->pos;
      st.generating = 1;
      st.n_generated = 1;
      st.stopped = (is_eos(next) || max <= 1) ? 1 : 0;
      upload_state_fields(e, st);
    }
    // decode: up to max-1 further steps, in batches between host checks
    int64_t remaining = max - 1;
    while (remaining > 0 && !st.stopped) {
      const int64_t batch = std::min<int64_t>(remaining, 32);
      replay(e, true, batch);
      remaining -= batch;
      st = read_state(e);
      if (st.error) throw device_error(e, st);
    }
    st = read_state(e);
    generated.resize((size_t)st.n_generated);
    if (!generated.empty())
      HIP_OK(hipMemcpy(generated.data(), e->gen, generated.size() * 4, hipMemcpyDeviceToHost));
    e->pos = st.pos;
    next = generated.empty() ? next : generated.back();
    if ((c.lfm || c.granite) && !generated.empty() && !is_eos(generated.back())) {
      // generateLfmWgsl / generateGraniteWgsl also run the last generated id
      // (lfm-wgsl-runtime.ts:288-300, granite-wgsl-runtime.ts:270-284):
      // its pick is the cached next id; the device holds that id at hist[pos]
      st.generating = 0;
      st.stopped = 0;
      upload_state_fields(e, st);
      replay(e, true);
      st = read_state(e);
      if (st.error) throw device_error(e, st);
      e->pos = st.pos;
      next = st.last_token;
    }
  }
  // leave the device in API mode
  st.generating = 0;
  st.stopped = 0;
  upload_state_fields(e, st);
  e->known_token_pos = -1;
  const double t_end = now_ms();
  e->cached_ids.assign(prompt, prompt + n_prompt);
  e->cached_ids.insert(e->cached_ids.end(), generated.begin(), generated.end());
  const bool last_eos = !generated.empty() && is_eos(generated.back());
  e->has_cached_next = !last_eos;
  e->cached_next = next;
  *out = generated;
  if (stats) {
    stats->prefill_ms = t_prefill_end - t0;
    stats->decode_ms = t_end - t_prefill_end;
    stats->prompt_tokens = (int32_t)n_prompt;
    stats->generated_tokens = (int32_t)generated.size();
    stats->tokens_per_sec = (double)generated.size() / std::max((t_end - t0) / 1000.0, 1e-3);
  }
}

// The reference loop (:266-313) stepped from the host through run_token.
void generate_stepped(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new,
                      const chonk_sampling* s_in, chonk_token_callback cb, void* user, std::vector<int32_t>* out,
                      chonk_gen_stats* stats) {
  // maxNewTokens ?? 128 (:255): a negative value stands for "not given"
  const int64_t max = std::min<int64_t>(max_new >= 0 ? max_new : 128, (int64_t)e->def.max_context - (int64_t)n_prompt);
  const chonk_sampling s = effective_sampling(e, s_in);
  for (size_t i = 0; i < n_prompt; ++i) check_token(e, prompt[i]);
  auto is_eos = [&](int32_t id) { return std::find(e->eos.begin(), e->eos.end(), id) != e->eos.end(); };
  const double t0 = now_ms();
  int64_t prefix = common_prefix(e->cached_ids, prompt, n_prompt);
  if (prefix != (int64_t)e->cached_ids.size()) {
    engine_reset(e);
    e->cached_ids.clear();
    e->has_cached_next = false;
    prefix = 0;
  }
  int32_t next = 0;
  const size_t n_suffix = n_prompt - (size_t)prefix;
  const bool gpt = e->cfg.gpt, lfm = e->cfg.lfm || e->cfg.granite;  // (granitehybrid: the LFM loop, :223-292)
  if (n_suffix == 0 && gpt && !e->has_cached_next)
    throw Error(CHONK_EINVAL, "GPT WGSL has no cached next token for an empty prompt");
  if (n_suffix == 0 && e->has_cached_next) {
    next = e->cached_next;
  } else {
    for (size_t i = 0; i < n_suffix; ++i) {
      const bool need = i + 1 == n_suffix;
      const size_t n_pen = (size_t)prefix + i + 1;
      next = run_token(e, prompt[prefix + i], need, &s, prompt, need ? n_pen : 0, prompt, need ? n_pen : 0);
    }
  }
  HIP_OK(hipStreamSynchronize(e->stream));
  const double t_prefill_end = now_ms();
  std::vector<int32_t> generated;
  std::vector<int32_t> ids(prompt, prompt + n_prompt);
  for (int64_t step = 0; step < max; ++step) {
    if (cb && cb(user, 0, 0)) break;
    generated.push_back(next);
    ids.push_back(next);
    if (cb) cb(user, 1, next);
    if (is_eos(next)) break;
    // (generateGptWgsl, gpt-wgsl-runtime.ts:228-245, and generateLfmWgsl,
    // lfm-wgsl-runtime.ts:288-300, also run the token after the last generated
    // one: its result is the cached next id)
    if (step + 1 >= max && !gpt && !lfm) break;
    next = run_token(e, next, true, &s, ids.data(), ids.size(), ids.data(), ids.size());
  }
  const double t_end = now_ms();
  e->cached_ids = ids;
  e->has_cached_next = !(!generated.empty() && is_eos(generated.back()));
  e->cached_next = next;
  *out = generated;
  if (stats) {
    stats->prefill_ms = t_prefill_end - t0;
    stats->decode_ms = t_end - t_prefill_end;
    stats->prompt_tokens = (int32_t)n_prompt;
    stats->generated_tokens = (int32_t)generated.size();
    stats->tokens_per_sec = (double)generated.size() / std::max((t_end - t0) / 1000.0, 1e-3);
  }
}

}  // namespace
}  // namespace chonk

// ---- C ABI ------------------------------------------------------------------------

extern "C" {

const char* chonk_last_error(void) { return g_last_error.c_str(); }

const char* chonk_engine_last_error(const chonk_engine* e) { return e ? e->err.c_str() : g_last_error.c_str(); }

int chonk_engine_create(const chonk_model_def* def, const char* path, chonk_engine** out) {
  return api_free([&] {
    if (!path) throw Error(CHONK_EINVAL, "null path");
    std::unique_ptr<ByteSource> src;
    try {
      src = open_byte_source(path);
    } catch (const std::exception& x) {
      throw Error(CHONK_EIO, x.what());
    }
    create_engine(def, std::move(src), path, out);
  });
}

int chonk_engine_create_from_memory(const chonk_model_def* def, const void* bytes, size_t n, chonk_engine** out) {
  return api_free([&] {
    if (!bytes) throw Error(CHONK_EINVAL, "null buffer");
    create_engine(def, memory_byte_source(bytes, n), "<memory>", out);
  });
}

int chonk_engine_destroy(chonk_engine* e) {
  if (!e) return CHONK_OK;
  bool expected = false;
  if (!e->busy.compare_exchange_strong(expected, true)) {
    g_last_error = "engine call already in progress";
    return CHONK_EBUSY;
  }
  engine_free(e);
  return CHONK_OK;
}

int chonk_engine_info_get(const chonk_engine* e, chonk_engine_info* out) {
  if (!e || !out) {
    g_last_error = "null argument";
    return CHONK_EINVAL;
  }
  const ModelCfg& c = e->cfg;
  out->hidden = c.hidden;
  out->ffn = c.ffn;
  out->vocab = c.vocab;
  out->layers = c.layers;
  out->heads = c.heads;
  out->kv_heads = c.kv_heads;
  out->head_dim = c.hd;
  out->context = c.ctx;
  out->architecture = c.arch == "llama" ? 0 : c.arch == "qwen3" ? 1 : c.arch == "gemma3" ? 2 : c.arch == "gpt2" ? 3
                      : c.arch == "openelm" ? 4 : c.arch == "lfm2" ? 5 : 6;
  out->qk_norm = c.qk_norm;
  out->interleaved_rope = c.interleaved;
  out->kv_dtype = e->kv_elem == 2 ? CHONK_KV_F16 : CHONK_KV_F32;
  out->weight_bytes_per_token = e->weight_bytes_per_token;
  out->device_bytes = e->weights.capacity() + e->state.capacity();
  out->kernels_per_step = (int32_t)e->kernels_logits.size();
  out->persistent_step = 0;  // (the one-launch-per-token step was retired: the graph ran twice as fast)
  out->noalloc_prefill_rows = e->noalloc_rows;
  out->spin_attention = e->dec_attn ? 1 : 0;
  out->fused_attention = 0;
  for (const Launch& L : e->kernels_logits) out->fused_attention += L.kind == Launch::QKVATTN ? 1 : 0;
  return CHONK_OK;
}

int chonk_engine_run_token(chonk_engine* e, int32_t token, int32_t need_logits, const chonk_sampling* s,
                           const int32_t* penalized, size_t n_penalized, const int32_t* seen, size_t n_seen,
                           int32_t* out_token) {
  return api(e, [&] {
    const int32_t t = run_token(e, token, need_logits != 0, s, penalized, penalized ? n_penalized : 0, seen,
                                seen ? n_seen : 0);
    if (out_token) *out_token = t;
  });
}

int chonk_engine_prefill(chonk_engine* e, const int32_t* tokens, size_t n) {
  return api(e, [&] {
    if (n == 0) return;
    if (!tokens) throw Error(CHONK_EINVAL, "tokens is null");
    for (size_t i = 0; i < n; ++i) check_token(e, tokens[i]);
    if ((int64_t)e->pos + (int64_t)n > e->cfg.ctx)
      throw context_exhausted(e);
    if (!e->batched_prefill) {
      // token by token through the decode step (gpt2, or CHONK_PREFILL=token)
      for (size_t i = 0; i < n; ++i) run_token(e, tokens[i], false, nullptr, nullptr, 0, nullptr, 0);
      e->known_token_pos = -1;
      e->logits_valid = false;
      return;
    }
    HIP_OK(hipMemcpy(e->hist + e->pos, tokens, n * 4, hipMemcpyHostToDevice));
    prefill_rows(e, tokens, (int)n);
    e->pos += (int)n;
    DevState st = read_state(e);
    st.pos = e->pos;
    upload_state_fields(e, st);
    e->known_token_pos = -1;
    e->logits_valid = false;
  });
}

int chonk_engine_prefill_noalloc(chonk_engine* e, const int32_t* tokens, size_t n) {
  return api(e, [&] {
    if (n == 0) return;
    if (!tokens) throw Error(CHONK_EINVAL, "tokens is null");
    if (e->noalloc_rows <= 0)
      throw Error(CHONK_EINVAL, std::string("chonk_engine_prefill_noalloc: this model has no row-batch prompt pass ") +
                                    "that fits the " + std::to_string(kNoAllocScratchBytes >> 20) +
                                    " MiB scratch (gpt2, lfm2, granitehybrid, rows wider than 4096, or "
                                    "CHONK_PREFILL=token)");
    if (n > (size_t)e->noalloc_rows)
      throw Error(CHONK_EINVAL, "chonk_engine_prefill_noalloc takes at most " + std::to_string(e->noalloc_rows) +
                                    " tokens per call for this model (its " +
                                    std::to_string(kNoAllocScratchBytes >> 20) + " MiB scratch), got " +
                                    std::to_string(n));
    for (size_t i = 0; i < n; ++i) check_token(e, tokens[i]);
    if ((int64_t)e->pos + (int64_t)n > e->cfg.ctx)
      throw context_exhausted(e);
    // every row buffer is written before it is read (the operand split writes
    // its own zero padding), so the previous call's contents need no clearing;
    // calls of engines on the same GPU take turns (the call returns once its
    // pass has finished on the device)
    std::lock_guard<std::mutex> scratch_turn(scratch_lock(e->device));
    RowBufs b;
    row_bufs_layout(e->cfg, e->noalloc_rows, e->scratch, &b);
    HIP_OK(hipMemcpy(e->hist + e->pos, tokens, n * 4, hipMemcpyHostToDevice));
    prefill_rows_in(e, b, tokens, (int)n);
    e->pos += (int)n;
    DevState st = read_state(e);
    st.pos = e->pos;
    upload_state_fields(e, st);
    e->known_token_pos = -1;
    e->logits_valid = false;
  });
}

int chonk_engine_generate(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new_tokens,
                          const chonk_sampling* s, int32_t* out_ids, size_t out_cap, size_t* n_out,
                          chonk_gen_stats* stats) {
  return api(e, [&] {
    if (!prompt && n_prompt) throw Error(CHONK_EINVAL, "null prompt");
    std::vector<int32_t> ids;
    // GPT-2 follows generateGptWgsl from the host (one more step at the end)
    if (e->cfg.gpt)
      generate_stepped(e, prompt, n_prompt, max_new_tokens, s, nullptr, nullptr, &ids, stats);
    else
      generate(e, prompt, n_prompt, max_new_tokens, s, &ids, stats);
    const size_t n = std::min(ids.size(), out_cap);
    if (out_ids && n) std::memcpy(out_ids, ids.data(), n * 4);
    if (n_out) *n_out = ids.size();
  });
}

int chonk_engine_generate_stepped(chonk_engine* e, const int32_t* prompt, size_t n_prompt, int32_t max_new_tokens,
                                  const chonk_sampling* s, chonk_token_callback callback, void* user,
                                  int32_t* out_ids, size_t out_cap, size_t* n_out, chonk_gen_stats* stats) {
  return api(e, [&] {
    if (!prompt && n_prompt) throw Error(CHONK_EINVAL, "null prompt");
    std::vector<int32_t> ids;
    generate_stepped(e, prompt, n_prompt, max_new_tokens, s, callback, user, &ids, stats);
    const size_t n = std::min(ids.size(), out_cap);
    if (out_ids && n) std::memcpy(out_ids, ids.data(), n * 4);
    if (n_out) *n_out = ids.size();
  });
}

int chonk_engine_conversation(chonk_engine* e, int32_t* ids, size_t cap, size_t* n_cached, int32_t* next_id) {
  return api(e, [&] {
    const size_t n = std::min(cap, e->cached_ids.size());
    if (ids && n) std::memcpy(ids, e->cached_ids.data(), n * 4);
    if (n_cached) *n_cached = e->cached_ids.size();
    if (next_id) *next_id = e->has_cached_next ? e->cached_next : -1;
  });
}

int chonk_engine_reset(chonk_engine* e) { return api(e, [&] { engine_reset(e); }); }

int chonk_engine_debug_fail_next_launch(chonk_engine* e) {
  return api(e, [&] { e->fail_next_launch = true; });
}

int chonk_engine_reset_conversation(chonk_engine* e) {
  return api(e, [&] {
    engine_reset(e);
    e->cached_ids.clear();
    e->has_cached_next = false;
  });
}

int chonk_engine_position(const chonk_engine* e, int32_t* out_pos) {
  if (!e || !out_pos) {
    g_last_error = "null argument";
    return CHONK_EINVAL;
  }
  *out_pos = e->pos;
  return CHONK_OK;
}

int chonk_engine_read_logits(chonk_engine* e, float* out, size_t n) {
  return api(e, [&] {
    if (!e->logits_valid) throw Error(CHONK_EINVAL, "no step has computed logits yet");
    if (!out || n < (size_t)e->cfg.vocab) throw Error(CHONK_EINVAL, "output buffer smaller than vocab");
    HIP_OK(hipStreamSynchronize(e->stream));
    HIP_OK(hipMemcpy(out, e->logits, (size_t)e->cfg.vocab * 4, hipMemcpyDeviceToHost));
  });
}

int chonk_engine_read_buffer(chonk_engine* e, int32_t which, void* out, size_t n_bytes) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    const void* src = nullptr;
    size_t bytes = 0;
    switch (which) {
      case 0: src = e->resA; bytes = (size_t)c.hidden * 4; break;
      case 1: src = e->attn; bytes = (size_t)c.heads * c.hd * 4; break;
      case 2: src = e->cand; bytes = (size_t)e->groups * 8; break;
      case 3: src = e->qkv; bytes = (size_t)(c.heads + 2 * c.kv_heads) * c.hd * 4; break;
      default: throw Error(CHONK_EINVAL, "unknown buffer id");
    }
    if (!out || n_bytes < bytes) throw Error(CHONK_EINVAL, "output buffer too small");
    HIP_OK(hipStreamSynchronize(e->stream));
    HIP_OK(hipMemcpy(out, src, bytes, hipMemcpyDeviceToHost));
  });
}

int chonk_engine_read_kv(chonk_engine* e, int32_t layer, int32_t is_value, int32_t pos, float* out) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (layer < 0 || layer >= c.layers || pos < 0 || pos >= c.ctx || !out) throw Error(CHONK_EINVAL, "bad layer/position");
    HIP_OK(hipStreamSynchronize(e->stream));
    const LayerDev& L = e->layers[layer];
    if (!L.kc)
      throw Error(CHONK_EINVAL, "layer " + std::to_string(layer) + " is a " +
                                    (e->cfg.granite ? "Mamba2" : "convolution") + " layer (no K/V cache)");
    const uint8_t* base = (const uint8_t*)(is_value ? L.vc : L.kc);
    std::vector<uint8_t> row((size_t)c.hd * e->kv_elem);
    for (int h = 0; h < c.kv_heads; ++h) {
      HIP_OK(hipMemcpy(row.data(), base + (((size_t)h * c.ctx + pos) * c.hd) * e->kv_elem, row.size(),
                       hipMemcpyDeviceToHost));
      for (int d = 0; d < c.hd; ++d) {
        if (e->kv_elem == 2) {
          uint16_t hv;
          std::memcpy(&hv, row.data() + 2 * d, 2);
          out[h * c.hd + d] = f16_to_f32(hv);
        } else {
          std::memcpy(&out[h * c.hd + d], row.data() + 4 * d, 4);
        }
      }
    }
  });
}

int chonk_engine_fake_context(chonk_engine* e, int32_t pos, uint64_t seed) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (pos < 0 || pos >= c.ctx) throw Error(CHONK_EINVAL, "position outside the context");
    for (int i = 0; i < c.layers; ++i)
      if (e->layers[i].kc)  // (lfm2 convolution layers keep only their zero state)
        HIP_OK(launch_fill_kv(e->layers[i].kc, e->layers[i].vc, c.layer[i].kv_heads, c.ctx, c.hd, pos, e->kv_elem == 2,
                            seed + 1000003ull * i, e->stream));
    DevState st{};
    st.pos = pos;
    upload_state_fields(e, st);
    e->pos = pos;
    e->known_token_pos = -1;
    e->cached_ids.clear();
    e->has_cached_next = false;
  });
}

int chonk_engine_bench_decode(chonk_engine* e, int32_t n_warmup, int32_t n_steps, double* ms_total) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (n_warmup < 0 || n_steps <= 0) throw Error(CHONK_EINVAL, "bad step counts");
    if ((int64_t)e->pos + n_warmup + n_steps > c.ctx)
      throw context_exhausted(e);
    DevSampling d = make_sampling(e, nullptr, false, false);
    upload_sampling(e, d);
    // the history slot at the current position must hold a token
    DevState st = read_state(e);
    int32_t tok = 0;
    HIP_OK(hipMemcpy(&tok, e->hist + e->pos, 4, hipMemcpyDeviceToHost));
    check_token(e, tok);
    replay(e, true, n_warmup);
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    HIP_OK(hipEventRecord(a, e->stream));
    replay(e, true, n_steps);
    HIP_OK(hipEventRecord(b, e->stream));
    HIP_OK(hipEventSynchronize(b));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    st = read_state(e);
    if (st.error) throw device_error(e, st);
    e->pos = st.pos;
    e->known_token_pos = -1;
    e->logits_valid = true;
    e->cached_ids.clear();
    e->has_cached_next = false;
    if (ms_total) *ms_total = ms;
  });
}

int chonk_engine_time_kernels(chonk_engine* e, const int32_t* ids, int32_t n_ids, int32_t rounds,
                              double* us_per_launch) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (!ids || n_ids <= 0 || rounds <= 0 || !us_per_launch) throw Error(CHONK_EINVAL, "bad kernel list or rounds");
    std::vector<Launch> run;
    for (int i = 0; i < n_ids; ++i) {
      if (ids[i] < 0 || ids[i] >= (int32_t)e->kernels_logits.size()) throw Error(CHONK_EINVAL, "bad kernel id");
      Launch L = e->kernels_logits[(size_t)ids[i]];
      if (L.kind == Launch::SEL) throw Error(CHONK_EINVAL, "the select kernel advances the position; not timed alone");
      if (L.kind == Launch::MV) L.mv.advance_pos = 0;
      run.push_back(L);
    }
    if (e->pos >= c.ctx) throw context_exhausted(e);
    const DevState saved = read_state(e);
    DevState st = saved;
    st.stopped = 0;
    st.generating = 0;
    upload_state_fields(e, st);
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    double total_ms = 0;
    for (int r = 0; r < rounds; ++r) {
      HIP_OK(hipEventRecord(a, e->stream));
      for (const Launch& L : run) enqueue(L, e->stream);
      HIP_OK(hipEventRecord(b, e->stream));
      HIP_OK(hipEventSynchronize(b));
      float ms = 0;
      HIP_OK(hipEventElapsedTime(&ms, a, b));
      total_ms += ms;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    upload_state_fields(e, saved);
    *us_per_launch = total_ms * 1000.0 / ((double)rounds * n_ids);
  });
}

int chonk_engine_bench_kernel(chonk_engine* e, int32_t kernel_id, int32_t reps, double* avg_us, char* name,
                              size_t name_len, uint64_t* bytes) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (kernel_id < 0 || kernel_id >= (int32_t)e->kernels_logits.size() || reps < 0)
      throw Error(CHONK_EINVAL, "bad kernel id or repetitions");
    const Launch& L = e->kernels_logits[(size_t)kernel_id];
    if (reps > 0 && L.kind == Launch::SEL)
      throw Error(CHONK_EINVAL, "the select kernel advances the position; not timed alone");
    if (e->pos >= c.ctx) throw context_exhausted(e);
    if (avg_us) *avg_us = 0.0;
    if (reps > 0) {
    const DevState saved = read_state(e);
    DevState st = saved;
    st.stopped = 0;
    st.generating = 0;
    upload_state_fields(e, st);
    Launch run = L;
    if (run.kind == Launch::MV) run.mv.advance_pos = 0;
    enqueue(run, e->stream);  // warm
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    HIP_OK(hipEventRecord(a, e->stream));
    for (int i = 0; i < reps; ++i) enqueue(run, e->stream);
    HIP_OK(hipEventRecord(b, e->stream));
    HIP_OK(hipEventSynchronize(b));
    float ms = 0;
    HIP_OK(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    upload_state_fields(e, saved);
    if (avg_us) *avg_us = (double)ms * 1000.0 / reps;
    }
    if (name && name_len) std::snprintf(name, name_len, "%s", L.name.c_str());
    if (bytes) {
      uint64_t by = L.weight_bytes;
      if (L.kind == Launch::MV || L.kind == Launch::QKVATTN) {
        by += (uint64_t)L.mv.k * 4;
        for (int i = 0; i < L.mv.nseg; ++i) by += (uint64_t)L.mv.seg[i].n_out * (L.kind == Launch::MV ? 4 : 8);
      }
      if (L.kind == Launch::ATTN || L.kind == Launch::QKVATTN) {
        const int pos = e->pos;
        const int w = L.at.window;
        const int start = (w != 0 && pos + 1 > w) ? pos + 1 - w : 0;
        const uint64_t nh = (uint64_t)L.at.heads, nkv = (uint64_t)L.at.kv_heads;
        by += 2ull * nkv * c.hd * (uint64_t)(pos + 1 - start) * e->kv_elem;
        by += (nh + 2 * nkv) * c.hd * 4 + nh * c.hd * 4;
      }
      *bytes = by;
    }
  });
}

int chonk_engine_bench_kernel_cold(chonk_engine* e, int32_t kernel_id, int32_t reps, uint64_t flush_bytes,
                                   double* cold_us, double* warm_us) {
  return api(e, [&] {
    const ModelCfg& c = e->cfg;
    if (kernel_id < 0 || kernel_id >= (int32_t)e->kernels_logits.size() || reps <= 0)
      throw Error(CHONK_EINVAL, "bad kernel id or repetitions");
    const Launch& L = e->kernels_logits[(size_t)kernel_id];
    if (L.kind == Launch::SEL) throw Error(CHONK_EINVAL, "the select kernel advances the position; not timed alone");
    if (e->pos >= c.ctx) throw context_exhausted(e);
    flush_bytes = std::max<uint64_t>(flush_bytes, (uint64_t)512 << 20);
    if (e->flush_bytes < flush_bytes) {
      if (e->flush) HIP_OK(hipFree(e->flush));
      e->flush = nullptr;
      e->flush_bytes = 0;
      HIP_OK(hipMalloc(&e->flush, flush_bytes));
      e->flush_bytes = flush_bytes;
    }
    const DevState saved = read_state(e);
    DevState st = saved;
    st.stopped = 0;
    st.generating = 0;
    upload_state_fields(e, st);
    Launch run = L;
    if (run.kind == Launch::MV) run.mv.advance_pos = 0;
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a));
    HIP_OK(hipEventCreate(&b));
    double sum[2] = {0, 0};
    enqueue(run, e->stream);
    for (int mode = 0; mode < 2; ++mode)  // 0 cold: caches flushed before the launch; 1 warm: launched twice, the second timed
      for (int i = 0; i < reps; ++i) {
        if (mode == 0)
          HIP_OK(hipMemsetAsync(e->flush, i & 0xff, e->flush_bytes, e->stream));
        else
          enqueue(run, e->stream);
        HIP_OK(hipEventRecord(a, e->stream));
        enqueue(run, e->stream);
        HIP_OK(hipEventRecord(b, e->stream));
        HIP_OK(hipEventSynchronize(b));
        float ms = 0;
        HIP_OK(hipEventElapsedTime(&ms, a, b));
        sum[mode] += ms;
      }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    upload_state_fields(e, saved);
    if (cold_us) *cold_us = sum[0] * 1000.0 / reps;
    if (warm_us) *warm_us = sum[1] * 1000.0 / reps;
  });
}

int chonk_dequant(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len, float* out) {
  return api_free([&] {
    TypeTraits t;
    if (!type_traits(ggml_type, &t) || !t.quantized) throw Error(CHONK_EINVAL, "unsupported GGUF tensor type " + type_name(ggml_type));
    if (n_rows <= 0 || row_len <= 0 || row_len % t.block_elems || row_len % 32 || !blocks || !out)
      throw Error(CHONK_EINVAL, "bad dequant shape");
    HIP_OK(hipSetDevice(device));
    const Stripes st = repack(ggml_type, (const uint8_t*)blocks, n_rows, row_len);
    QMat q{};
    q.type = (int32_t)ggml_type;
    q.n = (int32_t)n_rows;
    q.k = (int32_t)row_len;
    std::vector<void*> bufs;
    const uint8_t** dst[4] = {&q.s0, &q.s1, &q.s2, &q.s3};
    float* d_out = nullptr;
    try {
      for (int i = 0; i < 4; ++i) {
        if (st.s[i].empty()) continue;
        void* p;
        HIP_OK(hipMalloc(&p, st.s[i].size()));
        bufs.push_back(p);
        HIP_OK(hipMemcpy(p, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
        *dst[i] = (const uint8_t*)p;
      }
      HIP_OK(hipMalloc((void**)&d_out, (size_t)(n_rows * row_len) * 4));
      HIP_OK(launch_dequant(q, d_out, nullptr));
      HIP_OK(hipDeviceSynchronize());
      HIP_OK(hipMemcpy(out, d_out, (size_t)(n_rows * row_len) * 4, hipMemcpyDeviceToHost));
    } catch (...) {
      for (void* p : bufs) (void)hipFree(p);
      if (d_out) (void)hipFree(d_out);
      throw;
    }
    for (void* p : bufs) (void)hipFree(p);
    (void)hipFree(d_out);
  });
}

int chonk_matvec(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len,
                 const float* x, float* y, int32_t reps, double* avg_us) {
  return api_free([&] {
    TypeTraits t;
    if (!type_traits(ggml_type, &t) || !t.quantized) throw Error(CHONK_EINVAL, "unsupported GGUF tensor type " + type_name(ggml_type));
    if (n_rows <= 0 || row_len <= 0 || row_len % t.block_elems || row_len % 32 || row_len > 32768 || !blocks || !x || !y)
      throw Error(CHONK_EINVAL, "bad matvec shape");
    HIP_OK(hipSetDevice(device));
    const Stripes st = repack(ggml_type, (const uint8_t*)blocks, n_rows, row_len);
    QMat q{};
    q.type = (int32_t)ggml_type;
    q.n = (int32_t)n_rows;
    q.k = (int32_t)row_len;
    std::vector<void*> bufs;
    auto dev = [&](size_t n) {
      void* p;
      HIP_OK(hipMalloc(&p, n));
      bufs.push_back(p);
      return p;
    };
    hipStream_t s = nullptr;
    try {
      const uint8_t** dst[4] = {&q.s0, &q.s1, &q.s2, &q.s3};
      for (int i = 0; i < 4; ++i) {
        if (st.s[i].empty()) continue;
        void* p = dev(st.s[i].size());
        HIP_OK(hipMemcpy(p, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
        *dst[i] = (const uint8_t*)p;
      }
      float* d_x = (float*)dev((size_t)row_len * 4);
      float* d_y = (float*)dev((size_t)n_rows * 4);
      DevState* d_st = (DevState*)dev(sizeof(DevState));
      HIP_OK(hipMemset(d_st, 0, sizeof(DevState)));
      HIP_OK(hipMemcpy(d_x, x, (size_t)row_len * 4, hipMemcpyHostToDevice));
      MvArgs a{};
      a.nseg = 1;
      a.k = (int32_t)row_len;
      a.pro = PRO_PLAIN;
      a.epi = EPI_STORE;
      a.in = d_x;
      a.st = d_st;
      plan_seg(a.seg[0], q, (int)n_rows, false, 0);
      a.seg[0].out = d_y;
      const int grid = seg_wgs(a.seg[0]);
      const size_t shmem = mv_shared_bytes((int)row_len, a.seg[0].tile);
      HIP_OK(init_kernel_attributes());
      if (shmem > lds_limit()) throw Error(CHONK_EINVAL, "row length too large for the LDS limit");
      HIP_OK(hipStreamCreate(&s));
      HIP_OK(launch_matvec(a, grid, shmem, s));
      HIP_OK(hipStreamSynchronize(s));
      if (reps > 0) {
        hipEvent_t e0, e1;
        HIP_OK(hipEventCreate(&e0));
        HIP_OK(hipEventCreate(&e1));
        HIP_OK(hipEventRecord(e0, s));
        for (int i = 0; i < reps; ++i) HIP_OK(launch_matvec(a, grid, shmem, s));
        HIP_OK(hipEventRecord(e1, s));
        HIP_OK(hipEventSynchronize(e1));
        float ms = 0;
        HIP_OK(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        if (avg_us) *avg_us = (double)ms * 1000.0 / reps;
      }
      HIP_OK(hipMemcpy(y, d_y, (size_t)n_rows * 4, hipMemcpyDeviceToHost));
    } catch (...) {
      if (s) (void)hipStreamDestroy(s);
      for (void* p : bufs) (void)hipFree(p);
      throw;
    }
    (void)hipStreamDestroy(s);
    for (void* p : bufs) (void)hipFree(p);
  });
}

int chonk_gemm(int32_t device, uint32_t ggml_type, const void* blocks, int64_t n_rows, int64_t row_len,
               const float* x, int64_t n_tokens, float* y, int32_t reps, double* avg_us) {
  return api_free([&] {
    TypeTraits t;
    if (!type_traits(ggml_type, &t) || !t.quantized) throw Error(CHONK_EINVAL, "unsupported GGUF tensor type " + type_name(ggml_type));
    if (n_rows <= 0 || row_len <= 0 || row_len % t.block_elems || row_len % 32 || row_len > 4096 || n_tokens <= 0 ||
        n_tokens > 65536 || !blocks || !x || !y)
      throw Error(CHONK_EINVAL, "bad gemm shape");
    HIP_OK(hipSetDevice(device));
    const Stripes st = repack(ggml_type, (const uint8_t*)blocks, n_rows, row_len);
    QMat q{};
    q.type = (int32_t)ggml_type;
    q.n = (int32_t)n_rows;
    q.k = (int32_t)row_len;
    const int ws = weight_exponent(ggml_type, (const uint8_t*)blocks, (size_t)(n_rows * (row_len / t.block_elems)),
                                   t.block_bytes);
    const int kpad = gemm_kpad((int)row_len);
    std::vector<void*> bufs;
    auto dev = [&](size_t n) {
      void* p;
      HIP_OK(hipMalloc(&p, n));
      bufs.push_back(p);
      return p;
    };
    hipStream_t s = nullptr;
    try {
      const uint8_t** dst[4] = {&q.s0, &q.s1, &q.s2, &q.s3};
      for (int i = 0; i < 4; ++i) {
        if (st.s[i].empty()) continue;
        void* p = dev(st.s[i].size());
        HIP_OK(hipMemcpy(p, st.s[i].data(), st.s[i].size(), hipMemcpyHostToDevice));
        *dst[i] = (const uint8_t*)p;
      }
      float* d_x = (float*)dev((size_t)n_tokens * row_len * 4);
      float* d_y = (float*)dev((size_t)n_tokens * n_rows * 4);
      _Float16* d_h = (_Float16*)dev((size_t)n_tokens * kpad * 2);
      _Float16* d_l = (_Float16*)dev((size_t)n_tokens * kpad * 2);
      float* d_s = (float*)dev((size_t)n_tokens * 4);
      float* d_part = (float*)dev((size_t)kPartFloats * 4);
      HIP_OK(hipMemcpy(d_x, x, (size_t)n_tokens * row_len * 4, hipMemcpyHostToDevice));
      PfSplitArgs sa{};
      sa.x = d_x;
      sa.ldx = (int)row_len;
      sa.k = (int)row_len;
      sa.kpad = kpad;
      sa.xh = d_h;
      sa.xl = d_l;
      sa.xscale = d_s;
      GemmArgs g{};
      g.w = q;
      g.xh = d_h;
      g.xl = d_l;
      g.xscale = d_s;
      g.y = d_y;
      g.ldy = (int)n_rows;
      g.t = (int)n_tokens;
      g.kpad = kpad;
      g.epi = GEMM_STORE;
      g.ws = ws;
      g.part = d_part;
      g.part_cap = kPartFloats;
      HIP_OK(init_kernel_attributes());
      HIP_OK(init_gemm_attributes());
      HIP_OK(hipStreamCreate(&s));
      auto run = [&] {
        HIP_OK(launch_pf_split(sa, (int)n_tokens, s));
        HIP_OK(launch_gemm(g, s));
      };
      run();
      HIP_OK(hipStreamSynchronize(s));
      if (reps > 0) {
        hipEvent_t e0, e1;
        HIP_OK(hipEventCreate(&e0));
        HIP_OK(hipEventCreate(&e1));
        HIP_OK(hipEventRecord(e0, s));
        for (int i = 0; i < reps; ++i) run();
        HIP_OK(hipEventRecord(e1, s));
        HIP_OK(hipEventSynchronize(e1));
        float ms = 0;
        HIP_OK(hipEventElapsedTime(&ms, e0, e1));
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        if (avg_us) *avg_us = (double)ms * 1000.0 / reps;
      }
      HIP_OK(hipMemcpy(y, d_y, (size_t)n_tokens * n_rows * 4, hipMemcpyDeviceToHost));
    } catch (...) {
      if (s) (void)hipStreamDestroy(s);
      for (void* p : bufs) (void)hipFree(p);
      throw;
    }
    (void)hipStreamDestroy(s);
    for (void* p : bufs) (void)hipFree(p);
  });
}

int chonk_write_synthetic_gguf(const chonk_synth_config* c, const char* path, int32_t n_threads) {
  return api_free([&] {
    if (!c || !path || !c->arch || !c->recipe) throw Error(CHONK_EINVAL, "null argument");
    SynthConfig s;
    s.arch = c->arch;
    s.recipe = c->recipe;
    s.hidden = c->hidden;
    s.layers = c->layers;
    s.heads = c->heads;
    s.kv_heads = c->kv_heads;
    s.head_dim = c->head_dim;
    s.ffn = c->ffn;
    s.vocab = c->vocab;
    s.context_length = c->context_length;
    s.rope_theta = c->rope_theta;
    s.norm_eps = c->norm_eps;
    s.sliding_window = c->sliding_window;
    s.seed = c->seed;
    s.weight_std = c->weight_std > 0 ? c->weight_std : 0.02f;
    s.norm_std = c->norm_std > 0 ? c->norm_std : 0.02f;
    if (c->layers > 0) {
      if (c->layer_heads) s.layer_heads.assign(c->layer_heads, c->layer_heads + c->layers);
      if (c->layer_kv_heads) s.layer_kv_heads.assign(c->layer_kv_heads, c->layer_kv_heads + c->layers);
      if (c->layer_ffn) s.layer_ffn.assign(c->layer_ffn, c->layer_ffn + c->layers);
    }
    try {
      write_synthetic_gguf(s, path, n_threads);
    } catch (const std::exception& x) {
      throw Error(CHONK_EIO, x.what());
    }
  });
}

int chonk_write_shards(const char* gguf_path, const char* out_dir, uint64_t shard_size, const char* quant) {
  return api_free([&] {
    if (!gguf_path || !out_dir) throw Error(CHONK_EINVAL, "null argument");
    try {
      write_shards(gguf_path, out_dir, shard_size, quant ? quant : "");
    } catch (const std::exception& x) {
      throw Error(CHONK_EIO, x.what());
    }
  });
}

}  // extern "C"

// ---- batched decoding: independent sequences over one engine's weights ---------------

struct chonk_batch {
  chonk_engine* e = nullptr;
  int max_seqs = 0, max_tokens = 0, max_pages = 0, rows_cap = 0;
  void* kv_mem = nullptr;   // per layer: K pages | V pages, [page][kv_heads][64][hd] fp16
  void* row_mem = nullptr;  // row buffers, page table, row arrays, logits
  int32_t *pages = nullptr, *rseq = nullptr, *rpos = nullptr, *next = nullptr;
  float* logits = nullptr;  // [max(max_seqs, 1)][vocab], rows of the last call
  int last_rows = 0;
  RowBufs b;
  RowKv kvs;
  std::vector<int> len;     // positions held by each sequence's pages
  std::map<int, hipGraphExec_t> step_graphs;  // one captured step per row count
};

namespace chonk {
namespace {

void batch_free(chonk_batch* b) {
  if (!b) return;
  if (b->e) (void)hipSetDevice(b->e->device);
  if (b->e && b->e->stream) (void)hipStreamSynchronize(b->e->stream);
  for (auto& g : b->step_graphs) (void)hipGraphExecDestroy(g.second);
  if (b->kv_mem) (void)hipFree(b->kv_mem);
  if (b->row_mem) (void)hipFree(b->row_mem);
  delete b;
}

void batch_create(chonk_engine* e, int max_seqs, int max_tokens, chonk_batch** out) {
  const ModelCfg& c = e->cfg;
  if (max_seqs <= 0 || max_seqs > 1024 || max_tokens <= 0 || max_tokens > c.ctx)
    throw Error(CHONK_EINVAL, "batch needs 1..1024 sequences of 1.." + std::to_string(c.ctx) + " tokens");
  if (std::max(c.hidden, std::max(c.heads * c.hd, c.ffn)) > 4096)
    throw Error(CHONK_EINVAL, "batched decoding needs hidden, q and ffn widths of at most 4096");
  if (c.gpt) throw Error(CHONK_EINVAL, "batched decoding covers the llama-family runtime, not gpt2");
  if (c.lfm || c.granite)
    throw Error(CHONK_EINVAL, "batched decoding covers the llama-family runtime, not lfm2 or granitehybrid");
  if (e->kv_elem != 2) throw Error(CHONK_EINVAL, "batched decoding needs the fp16 K/V cache");
  if (c.heads / c.kv_heads > 16) throw Error(CHONK_EINVAL, "batched decoding supports GQA groups up to 16");
  if (c.openelm) throw Error(CHONK_EINVAL, "batched decoding needs one head geometry for every layer (not openelm)");
  std::unique_ptr<chonk_batch, void (*)(chonk_batch*)> b(new chonk_batch(), batch_free);
  b->e = e;
  b->max_seqs = max_seqs;
  b->max_tokens = max_tokens;
  b->max_pages = (max_tokens + kKvPage - 1) / kKvPage;
  b->rows_cap = std::max(kPrefillRows, max_seqs);
  b->len.assign((size_t)max_seqs, 0);
  const size_t n_pages = (size_t)max_seqs * b->max_pages;
  const size_t pool = align256(n_pages * c.kv_heads * kKvPage * c.hd * 2);
  HIP_OK(hipMalloc(&b->kv_mem, pool * 2 * c.layers));
  HIP_OK(hipMemset(b->kv_mem, 0, pool * 2 * c.layers));  // finite values in slots not yet written
  b->kvs.ctx = max_tokens;
  b->kvs.max_pages = b->max_pages;
  for (int i = 0; i < c.layers; ++i) {
    b->kvs.kc.push_back((uint8_t*)b->kv_mem + pool * 2 * i);
    b->kvs.vc.push_back((uint8_t*)b->kv_mem + pool * (2 * i + 1));
  }
  const size_t rb = row_bufs_layout(c, b->rows_cap, nullptr, nullptr);
  const size_t tab = align256(n_pages * 4), arr = align256((size_t)b->rows_cap * 4);
  const size_t lg = align256((size_t)max_seqs * c.vocab * 4);
  HIP_OK(hipMalloc(&b->row_mem, rb + tab + 3 * arr + lg));
  uint8_t* p = (uint8_t*)b->row_mem;
  row_bufs_layout(c, b->rows_cap, p, &b->b);
  p += rb;
  b->pages = (int32_t*)p;
  p += tab;
  b->rseq = (int32_t*)p;
  b->rpos = (int32_t*)(p + arr);
  b->next = (int32_t*)(p + 2 * arr);
  b->logits = (float*)(p + 3 * arr);
  // sequence s owns physical pages [s * max_pages, (s + 1) * max_pages)
  std::vector<int32_t> table(n_pages);
  for (size_t i = 0; i < n_pages; ++i) table[i] = (int32_t)i;
  HIP_OK(hipMemcpy(b->pages, table.data(), n_pages * 4, hipMemcpyHostToDevice));
  b->kvs.pages = b->pages;
  *out = b.release();
}

void batch_prefill(chonk_batch* b, int seq, const int32_t* tokens, size_t n, int32_t* next) {
  chonk_engine* e = b->e;
  if (seq < 0 || seq >= b->max_seqs) throw Error(CHONK_EINVAL, "sequence index out of range");
  if (n == 0 || !tokens) throw Error(CHONK_EINVAL, "empty prompt");
  if ((int64_t)n > b->max_tokens)
    throw Error(CHONK_ECONTEXT, "batch sequence context exhausted at " + std::to_string(b->max_tokens) + " tokens");
  for (size_t i = 0; i < n; ++i) check_token(e, tokens[i]);
  for (size_t off = 0; off < n; off += kPrefillRows) {
    const int T = (int)std::min<size_t>(kPrefillRows, n - off);
    const bool last = off + T == n;
    HIP_OK(hipMemcpyAsync(b->b.tok, tokens + off, (size_t)T * 4, hipMemcpyHostToDevice, e->stream));
    RowPlace pl;
    pl.p0 = (int)off;
    pl.seq0 = seq;
    run_rows(e, b->b, b->kvs, pl, T, last ? b->logits : nullptr, T - 1, 1, e->stream);
  }
  HIP_OK(launch_row_argmax(b->logits, e->cfg.vocab, 1, b->b.part, b->next, e->stream));
  HIP_OK(hipMemcpyAsync(e->h_tok, b->next, 4, hipMemcpyDeviceToHost, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  b->len[(size_t)seq] = (int)n;
  b->last_rows = 1;
  if (next) *next = *e->h_tok;
}

void batch_step(chonk_batch* b, const int32_t* seqs, const int32_t* tokens, size_t n, int32_t* next) {
  chonk_engine* e = b->e;
  if (n == 0 || !seqs || !tokens) throw Error(CHONK_EINVAL, "empty step");
  if ((int64_t)n > b->max_seqs) throw Error(CHONK_EINVAL, "more rows than sequences");
  std::vector<int32_t> pos(n);
  std::vector<bool> used((size_t)b->max_seqs, false);
  for (size_t i = 0; i < n; ++i) {
    if (seqs[i] < 0 || seqs[i] >= b->max_seqs) throw Error(CHONK_EINVAL, "sequence index out of range");
    if (used[(size_t)seqs[i]]) throw Error(CHONK_EINVAL, "a sequence appears twice in one step");
    used[(size_t)seqs[i]] = true;
    check_token(e, tokens[i]);
    pos[i] = b->len[(size_t)seqs[i]];
    if (pos[i] >= b->max_tokens)
      throw Error(CHONK_ECONTEXT, "batch sequence context exhausted at " + std::to_string(b->max_tokens) + " tokens");
  }
  HIP_OK(hipMemcpyAsync(b->b.tok, tokens, n * 4, hipMemcpyHostToDevice, e->stream));
  HIP_OK(hipMemcpyAsync(b->rseq, seqs, n * 4, hipMemcpyHostToDevice, e->stream));
  HIP_OK(hipMemcpyAsync(b->rpos, pos.data(), n * 4, hipMemcpyHostToDevice, e->stream));
  // the step for n rows is captured once (inputs live in fixed device buffers);
  // CHONK_NO_GRAPH=1 launches it directly (for profilers)
  if (!e->use_graph) {
    RowPlace pl;
    pl.row_seq = b->rseq;
    pl.row_pos = b->rpos;
    run_rows(e, b->b, b->kvs, pl, (int)n, b->logits, 0, (int)n, e->stream);
    HIP_OK(launch_row_argmax(b->logits, e->cfg.vocab, (int)n, b->b.part, b->next, e->stream));
  }
  auto it = b->step_graphs.find((int)n);
  if (!e->use_graph) {
  } else if (it == b->step_graphs.end()) {
    RowPlace pl;
    pl.row_seq = b->rseq;
    pl.row_pos = b->rpos;
    hipGraph_t g = nullptr;
    HIP_OK(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    try {
      run_rows(e, b->b, b->kvs, pl, (int)n, b->logits, 0, (int)n, e->stream);
      HIP_OK(launch_row_argmax(b->logits, e->cfg.vocab, (int)n, b->b.part, b->next, e->stream));
    } catch (...) {
      (void)hipStreamEndCapture(e->stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    HIP_OK(hipStreamEndCapture(e->stream, &g));
    hipGraphExec_t x = nullptr;
    const hipError_t ie = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_OK(ie);
    it = b->step_graphs.emplace((int)n, x).first;
  }
  if (e->use_graph) HIP_OK(hipGraphLaunch(it->second, e->stream));
  std::vector<int32_t> out(n);
  HIP_OK(hipMemcpyAsync(out.data(), b->next, n * 4, hipMemcpyDeviceToHost, e->stream));
  HIP_OK(hipStreamSynchronize(e->stream));
  for (size_t i = 0; i < n; ++i) b->len[(size_t)seqs[i]] += 1;
  b->last_rows = (int)n;
  if (next) std::copy(out.begin(), out.end(), next);
}

}  // namespace
}  // namespace chonk

int chonk_batch_create(chonk_engine* e, int32_t max_seqs, int32_t max_tokens, chonk_batch** out) {
  if (!out) return CHONK_EINVAL;
  *out = nullptr;
  return api(e, [&] { batch_create(e, max_seqs, max_tokens, out); });
}

int chonk_batch_destroy(chonk_batch* b) {
  if (!b) return CHONK_OK;
  return api(b->e, [&] { batch_free(b); });
}

int chonk_batch_prefill(chonk_batch* b, int32_t seq, const int32_t* tokens, size_t n, int32_t* next_id) {
  if (!b) return CHONK_EINVAL;
  return api(b->e, [&] { batch_prefill(b, seq, tokens, n, next_id); });
}

int chonk_batch_step(chonk_batch* b, const int32_t* seqs, const int32_t* tokens, size_t n, int32_t* next_ids) {
  if (!b) return CHONK_EINVAL;
  return api(b->e, [&] { batch_step(b, seqs, tokens, n, next_ids); });
}

int chonk_batch_position(const chonk_batch* b, int32_t seq, int32_t* out_pos) {
  if (!b || !out_pos || seq < 0 || seq >= b->max_seqs) return CHONK_EINVAL;
  *out_pos = b->len[(size_t)seq];
  return CHONK_OK;
}

int chonk_batch_read_logits(chonk_batch* b, int32_t row, float* out, size_t n) {
  if (!b) return CHONK_EINVAL;
  return api(b->e, [&] {
    const size_t V = (size_t)b->e->cfg.vocab;
    if (row < 0 || row >= b->last_rows || !out || n < V) throw Error(CHONK_EINVAL, "bad logits row or buffer");
    HIP_OK(hipMemcpy(out, b->logits + (size_t)row * V, V * 4, hipMemcpyDeviceToHost));
  });
}
