// ORACLE — TEST INFRASTRUCTURE ONLY (see oracle.h).
//
// CPU restatement of the reference's llama-webgpu decode path. Each function
// cites the reference file:line whose arithmetic it follows. Compiled with
// -ffp-contract=off: every a*b+c below is two roundings, as written in WGSL.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// binary16 decode (unpack2x16float is exact): an independent restatement.
float half_to_float(uint16_t h) {
  const int s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 1024), e - 25);
  return s ? -v : v;
}

uint16_t float_to_half(float f) {  // round to nearest even
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  int exp = (int)((x >> 23) & 0xff);
  uint32_t man = x & 0x7fffffu;
  if (exp == 255) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0));
  int e = exp - 112;  // rebias 127 -> 15
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t r = man >> shift, rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = sign | ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) ++r;
  return (uint16_t)r;
}

inline uint32_t byte_at(const uint8_t* d, uint64_t i) { return d[i]; }
inline float f16_at(const uint8_t* d, uint64_t i) { return half_to_float((uint16_t)(d[i] | (d[i + 1] << 8))); }
inline uint32_t u32_at(const uint8_t* d, uint64_t i) {
  return (uint32_t)d[i] | ((uint32_t)d[i + 1] << 8) | ((uint32_t)d[i + 2] << 16) | ((uint32_t)d[i + 3] << 24);
}
inline int32_t i8_at(const uint8_t* d, uint64_t i) { return (int32_t)(int8_t)d[i]; }

struct BlockGeom {
  int elems;
  int bytes;
};
bool geom(uint32_t type, BlockGeom* g) {
  switch (type) {
    case 0: *g = {1, 4}; return true;
    case 1: *g = {1, 2}; return true;
    case 6: *g = {32, 22}; return true;
    case 7: *g = {32, 24}; return true;
    case 8: *g = {32, 34}; return true;
    case 12: *g = {256, 144}; return true;
    case 13: *g = {256, 176}; return true;
    case 14: *g = {256, 210}; return true;
    default: return false;
  }
}

// scale_min_k4 (llama-wgsl-runtime.ts:2382-2389)
inline void scale_min(uint32_t j, const uint8_t* d, uint64_t base, uint32_t* sc, uint32_t* m) {
  if (j < 4) {
    *sc = byte_at(d, base + j) & 63u;
    *m = byte_at(d, base + j + 4) & 63u;
  } else {
    *sc = (byte_at(d, base + j + 4) & 15u) | ((byte_at(d, base + j - 4) >> 6) << 4);
    *m = (byte_at(d, base + j + 4) >> 4) | ((byte_at(d, base + j) >> 6) << 4);
  }
}

// Weight element (row, col) of a row-major GGUF matrix with `row_len`
// columns, evaluated exactly as the *_weight WGSL helpers do:
//   q5_0 :2230-2246, q5_1 :2280-2289, q8_0 :2321-2327, q4_k :2391-2410,
//   q5_k :2479-2495, q6_k :2560-2580; F32/F16 are plain loads.
float weight_at(uint32_t type, const uint8_t* d, uint64_t row, uint64_t col, uint64_t row_len) {
  switch (type) {
    case 0: {
      float v;
      std::memcpy(&v, d + 4 * (row * row_len + col), 4);
      return v;
    }
    case 1: return f16_at(d, 2 * (row * row_len + col));
    case 6: {
      const uint64_t blocks = row_len / 32, block = col >> 5, within = col & 31;
      const uint64_t base = row * blocks * 22 + block * 22;
      const uint32_t qh = u32_at(d, base + 2);
      const uint32_t qb = byte_at(d, base + 6 + (within & 15));
      const uint32_t low4 = within >= 16 ? qb >> 4 : qb & 15u;
      const uint32_t high = (qh >> within) & 1u;
      const uint32_t qv = low4 | (high << 4);
      return f16_at(d, base) * (float)((int32_t)qv - 16);
    }
    case 7: {
      const uint64_t blocks = row_len / 32, block = col >> 5, within = col & 31;
      const uint64_t base = row * blocks * 24 + block * 24;
      const uint32_t qh = u32_at(d, base + 4);
      const uint32_t qb = byte_at(d, base + 8 + (within & 15));
      const uint32_t low4 = within >= 16 ? qb >> 4 : qb & 15u;
      const uint32_t high = (qh >> within) & 1u;
      const uint32_t qv = low4 | (high << 4);
      const float prod = f16_at(d, base) * (float)qv;
      return prod + f16_at(d, base + 2);
    }
    case 8: {
      const uint64_t blocks = row_len / 32, block = col >> 5, within = col & 31;
      const uint64_t base = row * blocks * 34 + block * 34;
      return (float)i8_at(d, base + 2 + within) * f16_at(d, base);
    }
    case 12:
    case 13: {
      const uint64_t blocks = row_len / 256, sb = col >> 8, within = col & 255;
      const uint32_t group64 = (uint32_t)(within >> 6), lane = (uint32_t)(within & 31);
      const bool high = (within & 32) != 0;
      const uint64_t bb = type == 12 ? 144 : 176;
      const uint64_t base = row * blocks * bb + sb * bb;
      const float dd = f16_at(d, base), dmin = f16_at(d, base + 2);
      uint32_t sc, m;
      scale_min(group64 * 2 + (high ? 1 : 0), d, base + 4, &sc, &m);
      uint32_t q;
      if (type == 12) {
        const uint32_t qb = byte_at(d, base + 16 + group64 * 32 + lane);
        q = high ? qb >> 4 : qb & 15u;
      } else {
        const uint32_t qb = byte_at(d, base + 48 + group64 * 32 + lane);
        const uint32_t low4 = high ? qb >> 4 : qb & 15u;
        const uint32_t mask = (high ? 2u : 1u) << (group64 * 2);
        q = low4 + ((byte_at(d, base + 16 + lane) & mask) != 0 ? 16u : 0u);
      }
      const float a = dd * (float)sc;
      const float b = a * (float)q;
      const float c = dmin * (float)m;
      return b - c;
    }
    case 14: {
      const uint64_t blocks = row_len / 256, sb = col >> 8, within = col & 255;
      const uint32_t half = (uint32_t)(within >> 7), local = (uint32_t)(within & 127);
      const uint32_t lane = local & 31, quarter = local >> 5;
      const uint64_t base = row * blocks * 210 + sb * 210;
      const uint64_t ql_base = base + half * 64, qh_base = base + 128 + half * 32, sc_base = base + 192 + half * 8;
      const uint32_t ql = byte_at(d, ql_base + lane + ((quarter & 1) ? 32 : 0));
      const uint32_t lo = quarter < 2 ? ql & 15u : ql >> 4;
      const uint32_t qh = (byte_at(d, qh_base + lane) >> (quarter * 2)) & 3u;
      const int32_t q = (int32_t)(lo | (qh << 4)) - 32;
      const int32_t scale = i8_at(d, sc_base + (lane >> 4) + quarter * 2);
      const float a = f16_at(d, base + 208) * (float)scale;
      return a * (float)q;
    }
  }
  return NAN;
}

// ---------------------------------------------------------------------------
// persistent worker pool for row-parallel loops
class Pool {
 public:
  explicit Pool(int n) : n_(std::max(1, n)) {
    for (int i = 1; i < n_; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  // fn(begin, end) over [0, n) split into n_ contiguous ranges.
  void run(int64_t n, const std::function<void(int64_t, int64_t)>& fn) {
    if (n_ == 1 || n < 64) {
      fn(0, n);
      return;
    }
    {
      std::lock_guard<std::mutex> l(mu_);
      fn_ = &fn;
      total_ = n;
      pending_ = n_ - 1;
      ++gen_;
    }
    cv_.notify_all();
    fn(0, n / n_);
    std::unique_lock<std::mutex> l(mu_);
    done_cv_.wait(l, [this] { return pending_ == 0; });
    fn_ = nullptr;
  }
  int size() const { return n_; }

 private:
  void loop(int idx) {
    uint64_t seen = 0;
    while (true) {
      const std::function<void(int64_t, int64_t)>* fn;
      int64_t total;
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
        fn = fn_;
        total = total_;
      }
      (*fn)(total * idx / n_, total * (idx + 1) / n_);
      std::lock_guard<std::mutex> l(mu_);
      if (--pending_ == 0) done_cv_.notify_one();
    }
  }
  int n_;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int64_t, int64_t)>* fn_ = nullptr;
  int64_t total_ = 0;
  int pending_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

// Every weight of one row, block by block, with the float operations of
// weight_at in the same order (the block's scales decoded once): out[k] ==
// weight_at(type, d, row, k, K) bit for bit for every k.
void decode_row(uint32_t type, const uint8_t* d, uint64_t row, uint64_t K, float* out) {
  switch (type) {
    case 0:
    case 1:
      for (uint64_t k = 0; k < K; ++k) out[k] = weight_at(type, d, row, k, K);
      return;
    case 6:
    case 7: {
      const uint64_t bb = type == 6 ? 22 : 24, qo = type == 6 ? 6 : 8, ho = type == 6 ? 2 : 4;
      for (uint64_t b = 0; b < K / 32; ++b) {
        const uint64_t base = (row * (K / 32) + b) * bb;
        const float dd = f16_at(d, base);
        const float mm = type == 7 ? f16_at(d, base + 2) : 0.0f;
        const uint32_t qh = u32_at(d, base + ho);
        for (uint32_t j = 0; j < 32; ++j) {
          const uint32_t qb = byte_at(d, base + qo + (j & 15));
          const uint32_t qv = (j >= 16 ? qb >> 4 : qb & 15u) | (((qh >> j) & 1u) << 4);
          if (type == 6) {
            out[b * 32 + j] = dd * (float)((int32_t)qv - 16);
          } else {
            const float prod = dd * (float)qv;
            out[b * 32 + j] = prod + mm;
          }
        }
      }
      return;
    }
    case 8:
      for (uint64_t b = 0; b < K / 32; ++b) {
        const uint64_t base = (row * (K / 32) + b) * 34;
        const float dd = f16_at(d, base);
        for (uint32_t j = 0; j < 32; ++j) out[b * 32 + j] = (float)i8_at(d, base + 2 + j) * dd;
      }
      return;
    case 12:
    case 13: {
      const uint64_t bb = type == 12 ? 144 : 176;
      for (uint64_t sb = 0; sb < K / 256; ++sb) {
        const uint64_t base = (row * (K / 256) + sb) * bb;
        const float dd = f16_at(d, base), dmin = f16_at(d, base + 2);
        for (uint32_t j = 0; j < 8; ++j) {  // 32-element sub-block j = 2 * group64 + high
          uint32_t sc, m;
          scale_min(j, d, base + 4, &sc, &m);
          const float a = dd * (float)sc;
          const float c = dmin * (float)m;
          const uint32_t g = j >> 1;
          const bool high = (j & 1) != 0;
          for (uint32_t l = 0; l < 32; ++l) {
            uint32_t q;
            if (type == 12) {
              const uint32_t qb = byte_at(d, base + 16 + g * 32 + l);
              q = high ? qb >> 4 : qb & 15u;
            } else {
              const uint32_t qb = byte_at(d, base + 48 + g * 32 + l);
              const uint32_t mask = (high ? 2u : 1u) << (g * 2);
              q = (high ? qb >> 4 : qb & 15u) + ((byte_at(d, base + 16 + l) & mask) != 0 ? 16u : 0u);
            }
            const float b = a * (float)q;
            out[sb * 256 + g * 64 + (high ? 32 : 0) + l] = b - c;
          }
        }
      }
      return;
    }
    case 14:
      for (uint64_t sb = 0; sb < K / 256; ++sb) {
        const uint64_t base = (row * (K / 256) + sb) * 210;
        const float dd = f16_at(d, base + 208);
        for (uint32_t i = 0; i < 256; ++i) {
          const uint32_t half = i >> 7, local = i & 127, lane = local & 31, quarter = local >> 5;
          const uint32_t ql = byte_at(d, base + half * 64 + lane + ((quarter & 1) ? 32 : 0));
          const uint32_t lo = quarter < 2 ? ql & 15u : ql >> 4;
          const uint32_t qh = (byte_at(d, base + 128 + half * 32 + lane) >> (quarter * 2)) & 3u;
          const int32_t q = (int32_t)(lo | (qh << 4)) - 32;
          const float a = dd * (float)i8_at(d, base + 192 + half * 8 + (lane >> 4) + quarter * 2);
          out[sb * 256 + i] = a * (float)q;
        }
      }
      return;
  }
  for (uint64_t k = 0; k < K; ++k) out[k] = NAN;
}

// One output row of the GGUF matvec (llama-wgsl-runtime.ts:2412-2442): lane
// t of 128 sums x[k] * w(n, k) over k = t, t + 128, ... in increasing k
// (sum = sum + input[k] * w, :2420-2422), then the stride 64..1 tree. The 128
// lane sums advance together over each 128-wide slice of k, which is the same
// per-lane order.
float matvec_row(uint32_t type, const uint8_t* w, uint64_t row, uint64_t K, const float* x) {
  thread_local std::vector<float> wrow;
  if (wrow.size() < K) wrow.resize(K);
  decode_row(type, w, row, K, wrow.data());
  const float* wr = wrow.data();
  float partial[128];
  for (uint32_t t = 0; t < 128; ++t) partial[t] = 0.0f;
  uint64_t kb = 0;
  for (; kb + 128 <= K; kb += 128)
    for (uint32_t t = 0; t < 128; ++t) {
      const float prod = x[kb + t] * wr[kb + t];
      partial[t] = partial[t] + prod;
    }
  for (uint32_t t = 0; kb + t < K; ++t) {
    const float prod = x[kb + t] * wr[kb + t];
    partial[t] = partial[t] + prod;
  }
  for (uint32_t stride = 64; stride >= 1; stride >>= 1)
    for (uint32_t t = 0; t < stride; ++t) partial[t] = partial[t] + partial[t + stride];
  return partial[0];
}

void matvec(Pool& pool, uint32_t type, const uint8_t* w, uint64_t N, uint64_t K, const float* x, float* y) {
  pool.run((int64_t)N, [&](int64_t b, int64_t e) {
    for (int64_t n = b; n < e; ++n) y[n] = matvec_row(type, w, (uint64_t)n, K, x);
  });
}

// ---------------------------------------------------------------------------
// GGUF header reader (restates src/lib/gguf.ts:59-101; independent of the
// product's reader).
struct Value {
  uint32_t type = 0;
  double num = 0;
  std::string str;
  std::vector<Value> arr;
};
struct Tensor {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t type = 0;
  uint64_t offset = 0, nbytes = 0;
};
struct Gguf {
  std::map<std::string, Value> kv;
  std::map<std::string, Tensor> tensors;
  uint64_t data_offset = 0;
  std::vector<uint8_t> file;
};

struct Cursor {
  const std::vector<uint8_t>& b;
  uint64_t o = 0;
  template <typename T>
  T get() {
    if (o + sizeof(T) > b.size()) throw std::runtime_error("GGUF header truncated");
    T v;
    std::memcpy(&v, b.data() + o, sizeof(T));
    o += sizeof(T);
    return v;
  }
  std::string str() {
    uint64_t n = get<uint64_t>();
    if (o + n > b.size()) throw std::runtime_error("GGUF header truncated");
    std::string s((const char*)b.data() + o, (size_t)n);
    o += n;
    return s;
  }
  Value value(uint32_t t) {
    Value v;
    v.type = t;
    switch (t) {
      case 0: v.num = get<uint8_t>(); break;
      case 1: v.num = get<int8_t>(); break;
      case 2: v.num = get<uint16_t>(); break;
      case 3: v.num = get<int16_t>(); break;
      case 4: v.num = get<uint32_t>(); break;
      case 5: v.num = get<int32_t>(); break;
      case 6: v.num = get<float>(); break;
      case 7: v.num = get<uint8_t>() != 0; break;
      case 8: v.str = str(); break;
      case 9: {
        uint32_t it = get<uint32_t>();
        uint64_t n = get<uint64_t>();
        for (uint64_t i = 0; i < n; ++i) v.arr.push_back(value(it));
        break;
      }
      case 10: v.num = (double)get<uint64_t>(); break;
      case 11: v.num = (double)get<int64_t>(); break;
      case 12: v.num = get<double>(); break;
      default: throw std::runtime_error("unsupported GGUF metadata value type " + std::to_string(t));
    }
    return v;
  }
};

void load_gguf(const char* path, Gguf* g) {
  FILE* f = std::fopen(path, "rb");
  if (!f) throw std::runtime_error(std::string("cannot open ") + path);
  std::fseek(f, 0, SEEK_END);
  long sz = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  g->file.resize((size_t)sz);
  size_t got = std::fread(g->file.data(), 1, (size_t)sz, f);
  std::fclose(f);
  if (got != (size_t)sz) throw std::runtime_error("short read");
  Cursor c{g->file};
  if (c.get<uint32_t>() != 0x46554747u) throw std::runtime_error("invalid GGUF magic");
  c.get<uint32_t>();
  uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
  for (uint64_t i = 0; i < nkv; ++i) {
    std::string k = c.str();
    uint32_t t = c.get<uint32_t>();
    g->kv[k] = c.value(t);
  }
  for (uint64_t i = 0; i < nt; ++i) {
    Tensor t;
    t.name = c.str();
    uint32_t nd = c.get<uint32_t>();
    uint64_t ne = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      t.shape.push_back(c.get<uint64_t>());
      ne *= t.shape.back();
    }
    t.type = c.get<uint32_t>();
    t.offset = c.get<uint64_t>();
    BlockGeom bg;
    if (!geom(t.type, &bg)) throw std::runtime_error("unsupported GGML tensor type " + std::to_string(t.type));
    if (ne % (uint64_t)bg.elems) throw std::runtime_error("tensor not a multiple of its block size");
    t.nbytes = ne / bg.elems * bg.bytes;
    g->tensors[t.name] = t;
  }
  g->data_offset = (c.o + 31) / 32 * 32;
  for (auto& kv : g->tensors)
    if (g->data_offset + kv.second.offset + kv.second.nbytes > g->file.size())
      throw std::runtime_error("tensor " + kv.first + " extends past end of file");
}

// ggufNumberArray (llama-wgsl-runtime.ts:474-486)
std::vector<int> num_array(const Gguf& g, const std::string& k) {
  auto it = g.kv.find(k);
  if (it == g.kv.end() || it->second.type != 9)
    throw std::runtime_error("GGUF metadata " + k + " is missing or not a numeric array");
  std::vector<int> out;
  for (size_t i = 0; i < it->second.arr.size(); ++i) {
    const Value& v = it->second.arr[i];
    if (v.type == 8 || v.type == 9 || v.type == 7)
      throw std::runtime_error("GGUF metadata " + k + "[" + std::to_string(i) + "] is not numeric");
    out.push_back((int)v.num);
  }
  return out;
}

double num(const Gguf& g, const std::string& k, double fallback, bool required) {
  auto it = g.kv.find(k);
  if (it != g.kv.end() && it->second.type != 8 && it->second.type != 9) return it->second.num;
  if (!required) return fallback;
  throw std::runtime_error("GGUF metadata " + k + " is missing or not numeric");
}

// ---------------------------------------------------------------------------
constexpr float kNegBig = -3.402823e38f;  // the WGSL literal -3.402823e38

struct Matrix {
  uint32_t type = 0;
  const uint8_t* data = nullptr;
  uint64_t n = 0, k = 0;
};

struct Layer {
  int heads, kv_heads, qdim, kvdim, ffn, window;
  uint32_t theta_u32;
  std::vector<float> in_norm, post_norm, pre_ffn_norm, post_ffn_norm, q_norm, k_norm;
  Matrix q, k, v, o, gate, up, down;
  // GPT-2: fused q|k|v, LayerNorm biases (in_norm / post_norm hold the weights), linear biases
  Matrix qkv;
  std::vector<float> in_norm_b, post_norm_b, qkv_b, o_b, up_b, down_b;
  std::vector<float> kcache, vcache;  // [kv_heads][C][hd]
  // LFM2 short-convolution layer (lfm-wgsl-runtime.ts:69-78): in_proj rows
  // B | C | x, the [hidden][3] depthwise taps and the [hidden][3] state
  bool conv = false;
  Matrix conv_in, conv_out;
  std::vector<float> conv_w, conv_state;
  // Granite-4.0-H Mamba2 layer (granite-wgsl-runtime.ts:64-76): in_proj rows
  // z | xBC | dt, out_proj, the [conv][4] depthwise taps and bias, per-head dt
  // bias, A (= -exp(A_log)) and D, the gated norm weight, and the state:
  // [conv][4] conv window, [heads][head_dim][state] SSM state
  bool mamba = false;
  Matrix ssm_in, ssm_out;
  std::vector<float> c1d_w, c1d_b, dt_b, a_neg, d_w, ssm_norm, mconv_state, ssm_state;
};

}  // namespace

struct orc_model {
  Gguf g;
  Pool* pool = nullptr;
  // hyper-parameters (buildGgufLlamaManifest, llama-wgsl-runtime.ts:326-425)
  bool gemma = false, interleaved = false, qk_norm = false, kv_f16 = false;
  bool gpt = false;                         // GGUF architecture gpt2 (gpt-wgsl-runtime.ts)
  bool openelm = false;                     // fused attn_qkv, per-layer heads / kv heads / ffn
  bool lfm = false;                         // GGUF architecture lfm2 (lfm-wgsl-runtime.ts)
  bool granite = false;                     // GGUF architecture granitehybrid (granite-wgsl-runtime.ts)
  // granitehybrid: Mamba2 geometry (inner = heads * head_dim, conv = inner + 2 * state)
  int ssm_inner = 0, ssm_conv = 0, ssm_heads = 0, ssm_hdim = 0, ssm_state = 0;
  std::vector<float> pos_embd, final_norm_b;  // GPT-2: [context][hidden] position table, final LayerNorm bias
  int hidden = 0, ffn = 0, vocab = 0, n_layers = 0, heads = 0, kv_heads = 0, hd = 0, ctx = 0;
  float norm_eps = 1e-5f, qk_eps = 1e-5f, attn_scale = 0, embed_scale = 1;
  Matrix embed, lm_head;
  std::vector<float> final_norm;
  std::vector<Layer> layers;
  int pos = 0;
  // scratch of the last step
  std::vector<float> hA, hB, hC, norm, q, k, v, qn, attn, gate, up, ff, logits, scores, qkv, proj, conv_mid;
  std::vector<float> mproj, mconv, my, mnormed;  // granitehybrid Mamba2 scratch
  std::vector<uint8_t> candidates;
  std::vector<float> last_residual;
};

namespace {

void rms_norm(const float* in, const float* w, float* out, int n, float eps) {
  // RMS_NORM_WGSL (llama-wgsl-runtime.ts:1910-1949), 256 threads
  float partial[256];
  for (int t = 0; t < 256; ++t) {
    float sum = 0.0f;
    for (int i = t; i < n; i += 256) {
      const float sq = in[i] * in[i];
      sum = sum + sq;
    }
    partial[t] = sum;
  }
  for (int s = 128; s >= 1; s >>= 1)
    for (int t = 0; t < s; ++t) partial[t] = partial[t] + partial[t + s];
  const float inv = 1.0f / std::sqrt(partial[0] / (float)n + eps);
  for (int i = 0; i < n; ++i) {
    const float a = in[i] * inv;
    out[i] = a * w[i];
  }
}

void add_rms_norm(const float* a, float* io, const float* w, float* out, int n, float eps) {
  // ADD_RMS_NORM_WGSL (:1951-1992)
  for (int i = 0; i < n; ++i) io[i] = a[i] + io[i];
  rms_norm(io, w, out, n, eps);
}

float rope_angle(uint32_t theta, int d, int hd, int pos) {
  // rope_angle (:2884-2887): pow(f32(theta), -2.0 * f32(d) / f32(HEAD_DIM)) * f32(pos)
  const float e = (-2.0f * (float)d) / (float)hd;
  const float inv = std::pow((float)theta, e);
  return (float)pos * inv;
}

inline float kv_round(const orc_model* m, float v) { return m->kv_f16 ? half_to_float(float_to_half(v)) : v; }

// QK_NORM_ROPE_STORE(_INTERLEAVED) (:2929-3023, :3186-3280) and
// ROPE_STORE(_INTERLEAVED) (:2868-2927, :3122-3184).
void qk_rope_store(orc_model* m, Layer& L, int pos, bool use_norm, float* q_out) {
  const int hd = m->hd, half = hd / 2;
  const int group = L.heads / L.kv_heads;
  auto norm_head = [&](const float* x, const float* w, std::vector<float>& out) {
    float partial[256];
    for (int d = 0; d < 256; ++d) partial[d] = d < hd ? x[d] * x[d] : 0.0f;
    for (int s = 128; s >= 1; s >>= 1)
      for (int d = 0; d < s; ++d) partial[d] = partial[d] + partial[d + s];
    const float inv = 1.0f / std::sqrt(partial[0] / (float)hd + m->qk_eps);
    out.assign(hd, 0.0f);
    for (int d = 0; d < hd; ++d) {
      const float a = x[d] * inv;
      out[d] = a * w[d];
    }
  };
  std::vector<float> tmp;
  auto rotate = [&](const float* src, float* dst, int h_pos) {
    for (int d = 0; d < half; ++d) {
      const int ia = m->interleaved ? 2 * d : d;
      const int ib = m->interleaved ? 2 * d + 1 : d + half;
      const float a = src[ia], b = src[ib];
      const float ang = rope_angle(L.theta_u32, d, hd, h_pos);
      const float co = std::cos(ang), si = std::sin(ang);
      const float x0 = a * co, x1 = b * si, y0 = a * si, y1 = b * co;
      dst[ia] = x0 - x1;
      dst[ib] = y0 + y1;
    }
  };
  for (int h = 0; h < L.heads; ++h) {
    const float* src = m->q.data() + h * hd;
    float* dst = q_out + h * hd;
    if (use_norm) {
      norm_head(src, L.q_norm.data(), tmp);
      rotate(tmp.data(), dst, pos);
    } else {
      std::vector<float> copy(src, src + hd);
      rotate(copy.data(), dst, pos);
    }
  }
  (void)group;
  for (int kh = 0; kh < L.kv_heads; ++kh) {
    const float* src = m->k.data() + kh * hd;
    std::vector<float> rk(hd);
    if (use_norm) {
      norm_head(src, L.k_norm.data(), tmp);
      rotate(tmp.data(), rk.data(), pos);
    } else {
      rotate(src, rk.data(), pos);
    }
    float* kc = L.kcache.data() + ((size_t)kh * m->ctx + pos) * hd;
    float* vc = L.vcache.data() + ((size_t)kh * m->ctx + pos) * hd;
    for (int d = 0; d < hd; ++d) {
      kc[d] = kv_round(m, rk[d]);
      vc[d] = kv_round(m, m->v[kh * hd + d]);
    }
  }
}

// ATTENTION_SCORE_WGSL (:3385-3437) + ATTENTION_VALUE_WGSL (:3439-3490)
void attention(orc_model* m, Layer& L, int pos, const float* q, float* out) {
  const int hd = m->hd, C = m->ctx, group = L.heads / L.kv_heads;
  const int start = (L.window != 0 && pos + 1 > L.window) ? pos + 1 - L.window : 0;
  std::vector<float>& scores = m->scores;
  scores.assign((size_t)L.heads * C, 0.0f);
  m->pool->run(L.heads, [&](int64_t hb, int64_t he) {
    float partial[256];
    for (int64_t head = hb; head < he; ++head) {
      const int kvh = (int)head / group;
      for (int t = start; t <= pos; ++t) {
        const float* kr = L.kcache.data() + ((size_t)kvh * C + t) * hd;
        for (int d = 0; d < 256; ++d) partial[d] = d < hd ? q[head * hd + d] * kr[d] : 0.0f;
        for (int s = 128; s >= 1; s >>= 1)
          for (int d = 0; d < s; ++d) partial[d] = partial[d] + partial[d + s];
        scores[(size_t)head * C + t] = partial[0] * m->attn_scale;
      }
      const float* sc = scores.data() + (size_t)head * C;
      float mx = -3.402823e38f;
      for (int t = start; t <= pos; ++t) mx = std::fmax(mx, sc[t]);
      float denom = 0.0f;
      for (int t = start; t <= pos; ++t) denom = denom + std::exp(sc[t] - mx);
      // every output dim d evaluates p_t = exp(s_t - max) / denom with the same
      // operands, so p_t is computed once; acc[d] still sums over t in order
      thread_local std::vector<float> pt;
      pt.resize((size_t)C);
      for (int t = start; t <= pos; ++t) pt[t] = std::exp(sc[t] - mx) / denom;
      float acc[256];
      for (int d = 0; d < hd; ++d) acc[d] = 0.0f;
      for (int t = start; t <= pos; ++t) {
        const float* vr = L.vcache.data() + ((size_t)kvh * C + t) * hd;
        for (int d = 0; d < hd; ++d) {
          const float pv = pt[t] * vr[d];
          acc[d] = acc[d] + pv;
        }
      }
      for (int d = 0; d < hd; ++d) out[head * hd + d] = acc[d];
    }
  });
}

float silu_mul(float g, float u) {  // SILU_MUL_WGSL (:3529-3547)
  const float den = 1.0f + std::exp(-g);
  return (g / den) * u;
}

float gelu_tanh(float x) {  // GELU_TANH_MUL_WGSL (:3568-3599)
  if (x != x) return 0.0f;
  if (x > 10.0f) return x;
  if (x < -10.0f) return 0.0f;
  const float c = 0.7978845608028654f;
  const float cube = ((0.044715f * x) * x) * x;
  const float inner = c * (x + cube);
  const float t = 1.0f + std::tanh(inner);
  return (0.5f * x) * t;
}

// ARGMAX "better" (:3665-3673)
inline bool better(float v, uint32_t i, float bv, uint32_t bi) {
  if (v != v) return false;
  if (bv != bv) return true;
  return v > bv || (v == bv && i < bi);
}

Matrix matrix(orc_model* m, const std::string& name, uint64_t k, uint64_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("Llama WGSL manifest missing tensor " + name);
  const Tensor& t = it->second;
  if (t.type == 0 || t.type == 1)
    throw std::runtime_error("Llama WGSL tensor " + name + " is not a supported GGUF quantized tensor");
  BlockGeom bg{1, 1};
  if (!geom(t.type, &bg)) throw std::runtime_error("unsupported GGUF tensor type in " + name);
  if (k % (uint64_t)bg.elems) throw std::runtime_error("row length not a multiple of the block size for " + name);
  if (t.shape.empty() || t.shape[0] != k) throw std::runtime_error("tensor " + name + " row length mismatch");
  uint64_t rows = t.nbytes / (k / bg.elems * bg.bytes);
  if (rows < n) throw std::runtime_error("tensor " + name + " has fewer rows than required");
  Matrix mx;
  mx.type = t.type;
  mx.data = m->g.file.data() + m->g.data_offset + t.offset;
  mx.n = n;
  mx.k = k;
  return mx;
}

std::vector<float> floats(orc_model* m, const std::string& name, size_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("Llama WGSL manifest missing tensor " + name);
  const Tensor& t = it->second;
  if (t.type != 0 && t.type != 1)
    throw std::runtime_error("Llama WGSL tensor " + name + " is not float32/float16");
  const uint8_t* p = m->g.file.data() + m->g.data_offset + t.offset;
  std::vector<float> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = weight_at(t.type, p, 0, i, n);
  return out;
}

// manifestFromGguf + the engine's buffers (gpt-wgsl-runtime.ts:274-356, :540-640)
void build_gpt(orc_model* m, const orc_model_def* def) {
  const Gguf& g = m->g;
  m->gpt = true;
  m->hidden = (int)num(g, "gpt2.embedding_length", 0, true);
  m->n_layers = (int)num(g, "gpt2.block_count", 0, true);
  m->ffn = (int)num(g, "gpt2.feed_forward_length", 0, true);
  m->heads = (int)num(g, "gpt2.attention.head_count", 0, true);
  const int gguf_ctx = (int)num(g, "gpt2.context_length", 0, true);
  m->norm_eps = (float)num(g, "gpt2.attention.layer_norm_epsilon", 1e-5, false);
  if (m->hidden % m->heads) throw std::runtime_error("GPT WGSL: hidden is not divisible by heads");
  m->hd = m->hidden / m->heads;
  if (m->hd != 64) throw std::runtime_error("GPT WGSL: only 64-wide GPT-2 heads are implemented");
  m->kv_heads = m->heads;
  auto te = g.tensors.find("token_embd.weight");
  if (te == g.tensors.end() || te->second.shape.size() != 2) throw std::runtime_error("GPT WGSL: missing token_embd.weight");
  m->vocab = (int)te->second.shape[1];
  if ((m->vocab + 255) / 256 > 256) throw std::runtime_error("GPT WGSL argmax supports at most 65536 vocab entries");
  m->ctx = std::min(def->max_context, gguf_ctx);
  m->attn_scale = (float)(1.0 / std::sqrt((double)m->hd));  // INV_SQRT_HEAD_DIM (:1066)
  m->kv_f16 = def->kv_f16 != 0;
  m->embed = matrix(m, "token_embd.weight", (uint64_t)m->hidden, (uint64_t)m->vocab);
  m->lm_head = matrix(m, "output.weight", (uint64_t)m->hidden, (uint64_t)m->vocab);
  m->pos_embd = floats(m, "position_embd.weight", (size_t)gguf_ctx * m->hidden);
  m->final_norm = floats(m, "output_norm.weight", m->hidden);
  m->final_norm_b = floats(m, "output_norm.bias", m->hidden);
  const int H = m->hidden;
  for (int i = 0; i < m->n_layers; ++i) {
    Layer L;
    const std::string p = "blk." + std::to_string(i) + ".";
    L.heads = L.kv_heads = m->heads;
    L.qdim = L.kvdim = H;
    L.ffn = m->ffn;
    L.window = 0;
    L.theta_u32 = 0;
    L.in_norm = floats(m, p + "attn_norm.weight", H);
    L.in_norm_b = floats(m, p + "attn_norm.bias", H);
    L.post_norm = floats(m, p + "ffn_norm.weight", H);
    L.post_norm_b = floats(m, p + "ffn_norm.bias", H);
    L.qkv = matrix(m, p + "attn_qkv.weight", H, 3 * (uint64_t)H);
    L.qkv_b = floats(m, p + "attn_qkv.bias", 3 * (size_t)H);
    L.o = matrix(m, p + "attn_output.weight", H, H);
    L.o_b = floats(m, p + "attn_output.bias", H);
    L.up = matrix(m, p + "ffn_up.weight", H, m->ffn);
    L.up_b = floats(m, p + "ffn_up.bias", m->ffn);
    L.down = matrix(m, p + "ffn_down.weight", m->ffn, H);
    L.down_b = floats(m, p + "ffn_down.bias", H);
    L.kcache.assign((size_t)H * m->ctx, 0.0f);
    L.vcache.assign((size_t)H * m->ctx, 0.0f);
    m->layers.push_back(std::move(L));
  }
}

// The LFM runtime's GGUF loader and engine buffers (lfm-wgsl-runtime.ts:313-455,
// :501-580). The reference fixes the LFM2.5-350M shape in code (hidden 1024,
// intermediate 4608, 16 heads, head_dim 64, 65536 ids, eps 1e-5, rope base
// 1e6, three conv taps); here the dimensions come from the file's metadata and
// the constants stay the reference's. A layer is a convolution layer when it
// holds shortconv.conv.weight (lfm2.attention.head_count_kv is 0 there).
Matrix lfm_linear(orc_model* m, const std::string& name, uint64_t k, uint64_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("LFM GGUF missing tensor " + name);
  const uint32_t t = it->second.type;
  if (t != 8 && t != 12 && t != 14)  // ggufLinearKind (:422-427): Q8_0, Q4_K, Q6_K
    throw std::runtime_error("unsupported LFM GGUF linear tensor " + name);
  return matrix(m, name, k, n);
}

std::vector<float> lfm_floats(orc_model* m, const std::string& name, size_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("LFM GGUF missing tensor " + name);
  if (it->second.type != 0 && it->second.type != 1)
    throw std::runtime_error("LFM GGUF tensor " + name + " is not F32/F16");
  return floats(m, name, n);
}

void build_lfm(orc_model* m, const orc_model_def* def) {
  const Gguf& g = m->g;
  m->lfm = true;
  m->n_layers = (int)num(g, "lfm2.block_count", 0, true);
  m->hidden = (int)num(g, "lfm2.embedding_length", 0, true);
  m->ffn = (int)num(g, "lfm2.feed_forward_length", 0, true);
  m->heads = (int)num(g, "lfm2.attention.head_count", 0, true);
  std::vector<int> lkv;
  auto kv_it = g.kv.find("lfm2.attention.head_count_kv");
  if (kv_it != g.kv.end() && kv_it->second.type == 9) {
    lkv = num_array(g, "lfm2.attention.head_count_kv");
    if ((int)lkv.size() != m->n_layers) throw std::runtime_error("LFM GGUF head_count_kv length != layers");
  } else {
    lkv.assign((size_t)m->n_layers, (int)num(g, "lfm2.attention.head_count_kv", 0, true));
  }
  m->hd = (int)num(g, "lfm2.attention.key_length", std::floor((double)m->hidden / m->heads), false);
  if (m->hd > 256) throw std::runtime_error("head_dim above 256 is not supported");
  m->vocab = def->vocab;
  m->ctx = def->max_context;                 // LfmWgslEngine.maxContext (:461)
  m->norm_eps = 1e-5f;                       // RMS_NORM_WGSL / ADD_RMS_NORM_WGSL (:1567-1639)
  m->qk_eps = 1e-5f;                         // QK_NORM_ROPE_STORE_WGSL (:1763)
  m->qk_norm = true;
  m->attn_scale = (float)(1.0 / std::sqrt((double)m->hd));  // 0.125 at head_dim 64 (:1834)
  m->embed_scale = 1.0f;
  m->kv_f16 = def->kv_f16 != 0;
  const int H = m->hidden;
  m->embed = lfm_linear(m, "token_embd.weight", (uint64_t)H, (uint64_t)m->vocab);
  m->lm_head = m->embed;                     // the lm_head is the embedding (:512-519)
  m->final_norm = lfm_floats(m, "token_embd_norm.weight", H);
  m->kv_heads = 0;
  for (int i = 0; i < m->n_layers; ++i) {
    Layer L;
    const std::string p = "blk." + std::to_string(i) + ".";
    L.conv = g.tensors.count(p + "shortconv.conv.weight") != 0;
    L.heads = m->heads;
    L.kv_heads = L.conv ? 0 : lkv[(size_t)i];
    L.qdim = L.heads * m->hd;
    L.kvdim = L.kv_heads * m->hd;
    L.ffn = m->ffn;
    L.theta_u32 = 1000000;                   // rope_angle's pow(1000000.0, ...) (:1739-1742)
    L.window = 0;
    L.in_norm = lfm_floats(m, p + "attn_norm.weight", H);
    L.post_norm = lfm_floats(m, p + "ffn_norm.weight", H);
    L.gate = lfm_linear(m, p + "ffn_gate.weight", H, m->ffn);
    L.up = lfm_linear(m, p + "ffn_up.weight", H, m->ffn);
    L.down = lfm_linear(m, p + "ffn_down.weight", m->ffn, H);
    if (L.conv) {
      const Tensor& cw = g.tensors.at(p + "shortconv.conv.weight");
      if (cw.shape.size() != 2 || cw.shape[0] != 3 || cw.shape[1] != (uint64_t)H)
        throw std::runtime_error("LFM conv weight " + p + "shortconv.conv.weight is not [3, hidden]");
      L.conv_w = lfm_floats(m, p + "shortconv.conv.weight", 3 * (size_t)H);
      L.conv_in = lfm_linear(m, p + "shortconv.in_proj.weight", H, 3 * (uint64_t)H);
      L.conv_out = lfm_linear(m, p + "shortconv.out_proj.weight", H, H);
      L.conv_state.assign(3 * (size_t)H, 0.0f);
    } else {
      if (L.kv_heads <= 0 || L.heads % L.kv_heads != 0)
        throw std::runtime_error("layer heads must be a positive multiple of kv heads");
      m->kv_heads = std::max(m->kv_heads, L.kv_heads);
      L.q_norm = lfm_floats(m, p + "attn_q_norm.weight", m->hd);
      L.k_norm = lfm_floats(m, p + "attn_k_norm.weight", m->hd);
      L.q = lfm_linear(m, p + "attn_q.weight", H, L.qdim);
      L.k = lfm_linear(m, p + "attn_k.weight", H, L.kvdim);
      L.v = lfm_linear(m, p + "attn_v.weight", H, L.kvdim);
      L.o = lfm_linear(m, p + "attn_output.weight", L.qdim, H);
      L.kcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
      L.vcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
    }
    m->layers.push_back(std::move(L));
  }
  if (m->kv_heads == 0) throw std::runtime_error("LFM GGUF has no attention layer");
}

// The Granite runtime's GGUF checks (granite-wgsl-runtime.ts:359-395, :397-491)
// with its wording: tensor types F32 / F16 / Q8_0 / Q4_K / Q6_K only, linear
// tensors quantized with shape [k, n], float tensors F32 / F16.
void granite_check_types(orc_model* m) {
  for (const auto& kv : m->g.tensors) {
    const uint32_t t = kv.second.type;
    if (t != 0 && t != 1 && t != 8 && t != 12 && t != 14)
      throw std::runtime_error("Granite WGSL unsupported GGML tensor type " + std::to_string(t));
  }
}

Matrix granite_linear(orc_model* m, const std::string& name, uint64_t k, uint64_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + name);
  const Tensor& t = it->second;
  if (t.type != 8 && t.type != 12 && t.type != 14)
    throw std::runtime_error("Granite WGSL tensor " + name + " is not a GGUF quantized matrix");
  if (t.shape.size() != 2 || t.shape[0] != k || t.shape[1] != n) {  // validateMatrixShape (:482-486)
    std::string got;
    for (size_t i = 0; i < t.shape.size(); ++i) got += (i ? ", " : "") + std::to_string(t.shape[i]);
    throw std::runtime_error("Granite WGSL tensor " + name + " shape [" + got + "], expected [" + std::to_string(k) +
                             ", " + std::to_string(n) + "]");
  }
  return matrix(m, name, k, n);
}

std::vector<float> granite_floats(orc_model* m, const std::string& name, size_t n) {
  auto it = m->g.tensors.find(name);
  if (it == m->g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + name);
  if (it->second.type != 0 && it->second.type != 1)
    throw std::runtime_error("Granite WGSL tensor " + name + " is not float32/float16");
  return floats(m, name, n);
}

// GraniteWgslEngine.create (:536-624). The reference fixes the
// Granite-4.0-H-350M shape in code (hidden 768, intermediate 2048, 12 heads /
// 4 kv heads of 64, conv 1792, 48 SSM heads of 32, 128 states); here the
// dimensions come from the tensor shapes with the same fixed SSM head width
// (32) and state size (128), and the constants stay the reference's: eps 1e-5,
// embedding x12, residual x0.246, attention x0.015625, logits x1/3, 4096
// positions. A layer holding blk.N.ssm_in.weight is a Mamba2 layer (the
// registry's layerTypes, :48-53).
void build_granite(orc_model* m, const orc_model_def* def) {
  const Gguf& g = m->g;
  m->granite = true;
  // validateGraniteGguf (:359-371)
  auto ft = g.kv.find("general.file_type");
  const double file_type = ft != g.kv.end() && ft->second.type != 8 && ft->second.type != 9 ? ft->second.num : -1;
  if (file_type != 7 && file_type != 15)
    throw std::runtime_error("Granite WGSL: expected GGUF Q8_0 or Q4_K_M file_type, got " +
                             std::to_string((int)file_type));
  for (const char* name : {"token_embd.weight", "output_norm.weight", "blk.0.attn_norm.weight"})
    if (!g.tensors.count(name)) throw std::runtime_error(std::string("Granite WGSL: GGUF missing tensor ") + name);
  granite_check_types(m);
  const Tensor& te = g.tensors.at("token_embd.weight");
  if (te.shape.size() != 2) throw std::runtime_error("Granite WGSL token_embd.weight is not a matrix");
  const int H = (int)te.shape[0];
  m->hidden = H;
  m->vocab = (int)te.shape[1];
  int nl = 0;
  while (g.tensors.count("blk." + std::to_string(nl) + ".attn_norm.weight")) ++nl;
  m->n_layers = nl;
  m->hd = 64;                                // head_dim (:526, the STORE_KV / ATTENTION kernels' 64)
  m->ctx = 4096;                             // GraniteWgslEngine.maxContext (:530)
  m->norm_eps = 1e-5f;                       // RMS_NORM_WGSL / ADD_SCALED_RMS_NORM_WGSL / MAMBA_GATE_NORM_WGSL
  m->attn_scale = 0.015625f;                 // ATTENTION_SCORE_WGSL (:1668)
  m->embed_scale = 12.0f;                    // EMBEDDING_Q8_WGSL (:1362)
  m->kv_f16 = def->kv_f16 != 0;
  m->ssm_hdim = 32;                          // mambaDHead (:533)
  m->ssm_state = 128;                        // the SSM kernel's 128-lane state (:1543-1547)
  m->embed = granite_linear(m, "token_embd.weight", (uint64_t)H, (uint64_t)m->vocab);
  m->lm_head = m->embed;                     // the embedding is the lm_head (:547-555)
  m->final_norm = granite_floats(m, "output_norm.weight", H);
  m->kv_heads = 0;
  m->heads = 0;
  m->ffn = 0;
  for (int i = 0; i < nl; ++i) {
    Layer L;
    const std::string p = "blk." + std::to_string(i) + ".";
    L.mamba = g.tensors.count(p + "ssm_in.weight") != 0;
    L.in_norm = granite_floats(m, p + "attn_norm.weight", H);
    L.post_norm = granite_floats(m, p + "ffn_norm.weight", H);
    const auto& tg = g.tensors.find(p + "ffn_gate.weight");
    if (tg == g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + p + "ffn_gate.weight");
    L.ffn = (int)tg->second.shape.back();
    m->ffn = std::max(m->ffn, L.ffn);
    L.gate = granite_linear(m, p + "ffn_gate.weight", H, L.ffn);
    L.up = granite_linear(m, p + "ffn_up.weight", H, L.ffn);
    L.down = granite_linear(m, p + "ffn_down.weight", L.ffn, H);
    L.window = 0;
    L.theta_u32 = 0;
    if (L.mamba) {
      auto ti = g.tensors.find(p + "ssm_out.weight");
      if (ti == g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + p + "ssm_out.weight");
      const int inner = (int)ti->second.shape[0];
      if (inner % m->ssm_hdim) throw std::runtime_error("Granite WGSL: SSM inner size is not a multiple of 32");
      if (m->ssm_inner && inner != m->ssm_inner) throw std::runtime_error("Granite WGSL: SSM inner size differs by layer");
      m->ssm_inner = inner;
      m->ssm_heads = inner / m->ssm_hdim;
      m->ssm_conv = inner + 2 * m->ssm_state;
      const int nproj = inner + m->ssm_conv + m->ssm_heads;
      L.ssm_in = granite_linear(m, p + "ssm_in.weight", H, nproj);
      L.ssm_out = granite_linear(m, p + "ssm_out.weight", inner, H);
      L.c1d_w = granite_floats(m, p + "ssm_conv1d.weight", 4 * (size_t)m->ssm_conv);
      L.c1d_b = granite_floats(m, p + "ssm_conv1d.bias", m->ssm_conv);
      L.dt_b = granite_floats(m, p + "ssm_dt.bias", m->ssm_heads);
      L.a_neg = granite_floats(m, p + "ssm_a", m->ssm_heads);
      L.d_w = granite_floats(m, p + "ssm_d", m->ssm_heads);
      L.ssm_norm = granite_floats(m, p + "ssm_norm.weight", inner);
      L.mconv_state.assign(4 * (size_t)m->ssm_conv, 0.0f);
      L.ssm_state.assign((size_t)m->ssm_heads * m->ssm_hdim * m->ssm_state, 0.0f);
      L.heads = 0;
      L.kv_heads = 0;
    } else {
      auto tq = g.tensors.find(p + "attn_q.weight"), tk = g.tensors.find(p + "attn_k.weight");
      if (tq == g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + p + "attn_q.weight");
      if (tk == g.tensors.end()) throw std::runtime_error("Granite WGSL manifest missing tensor " + p + "attn_k.weight");
      L.qdim = (int)tq->second.shape.back();
      L.kvdim = (int)tk->second.shape.back();
      L.heads = L.qdim / m->hd;
      L.kv_heads = L.kvdim / m->hd;
      if (L.qdim % m->hd || L.kvdim % m->hd || L.kv_heads <= 0 || L.heads % L.kv_heads != 0)
        throw std::runtime_error("Granite WGSL: attention heads must be whole 64-wide heads in whole groups");
      m->heads = std::max(m->heads, L.heads);
      m->kv_heads = std::max(m->kv_heads, L.kv_heads);
      L.q = granite_linear(m, p + "attn_q.weight", H, L.qdim);
      L.k = granite_linear(m, p + "attn_k.weight", H, L.kvdim);
      L.v = granite_linear(m, p + "attn_v.weight", H, L.kvdim);
      L.o = granite_linear(m, p + "attn_output.weight", L.qdim, H);
      L.kcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
      L.vcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
    }
    m->layers.push_back(std::move(L));
  }
  if (nl == 0) throw std::runtime_error("Granite WGSL: GGUF has no layers");
  if (m->heads == 0) m->heads = 1;
  for (Layer& L : m->layers)
    if (L.mamba) {
      L.qdim = 0;
      L.kvdim = 0;
    }
}

void build(orc_model* m, const orc_model_def* def) {
  const Gguf& g = m->g;
  auto it = g.kv.find("general.architecture");
  if (it == g.kv.end() || it->second.type != 8) throw std::runtime_error("GGUF metadata general.architecture is missing or not a string");
  const std::string arch = it->second.str;
  if (arch == "gpt2") {
    build_gpt(m, def);
    return;
  }
  if (arch == "lfm2") {
    build_lfm(m, def);
    return;
  }
  if (arch == "granitehybrid") {
    build_granite(m, def);
    return;
  }
  if (arch != "qwen3" && arch != "llama" && arch != "gemma3" && arch != "openelm")
    throw std::runtime_error("Llama GGUF WGSL does not support architecture " + arch);
  m->gemma = arch == "gemma3";
  m->openelm = arch == "openelm";
  m->interleaved = arch == "llama";
  m->n_layers = (int)num(g, arch + ".block_count", 0, true);
  m->hidden = (int)num(g, arch + ".embedding_length", 0, true);
  // openelm: per-layer arrays whose maxima are the model's heads / kvHeads /
  // intermediate (buildGgufLlamaManifest, :373-380; validateLayerArray, :1815-1821)
  std::vector<int> lh, lkv, lff;
  if (m->openelm) {
    lh = num_array(g, arch + ".attention.head_count");
    lkv = num_array(g, arch + ".attention.head_count_kv");
    lff = num_array(g, arch + ".feed_forward_length");
    for (const auto* v : {&lh, &lkv, &lff})
      if ((int)v->size() != m->n_layers || v->empty())
        throw std::runtime_error("Llama WGSL manifest layer array length != layers");
    m->heads = *std::max_element(lh.begin(), lh.end());
    m->kv_heads = *std::max_element(lkv.begin(), lkv.end());
    m->ffn = *std::max_element(lff.begin(), lff.end());
  } else {
    m->heads = (int)num(g, arch + ".attention.head_count", 0, true);
    m->kv_heads = (int)num(g, arch + ".attention.head_count_kv", 0, true);
    m->ffn = (int)num(g, arch + ".feed_forward_length", 0, true);
  }
  m->hd = (int)num(g, arch + ".attention.key_length", std::floor((double)m->hidden / m->heads), false);
  if (m->hd > 256) throw std::runtime_error("head_dim above 256 is not supported");
  m->vocab = def->vocab;
  const int gguf_ctx = (int)num(g, arch + ".context_length", def->max_context, false);
  m->ctx = std::min(def->max_context, std::min(def->max_context, gguf_ctx));
  m->norm_eps = (float)num(g, arch + ".attention.layer_norm_rms_epsilon", 1e-5, false);
  m->qk_eps = m->norm_eps;
  m->qk_norm = g.tensors.count("blk.0.attn_q_norm.weight") && g.tensors.count("blk.0.attn_k_norm.weight");
  m->attn_scale = (float)(1.0 / std::sqrt((double)m->hd));
  m->embed_scale = m->gemma ? (float)std::sqrt((double)m->hidden) : 1.0f;
  m->kv_f16 = def->kv_f16 != 0;
  const double theta = m->gemma ? 10000.0 : num(g, arch + ".rope.freq_base", 10000, false);
  const double gtheta = m->gemma ? num(g, "gemma3.rope.freq_base", 1000000, false) : 0;
  const int window = m->gemma ? (int)num(g, "gemma3.attention.sliding_window", 0, false) : 0;

  m->embed = matrix(m, "token_embd.weight", (uint64_t)m->hidden, (uint64_t)m->vocab);
  m->lm_head = g.tensors.count("output.weight") ? matrix(m, "output.weight", m->hidden, m->vocab) : m->embed;
  m->final_norm = floats(m, "output_norm.weight", m->hidden);
  for (int i = 0; i < m->n_layers; ++i) {
    Layer L;
    const std::string p = "blk." + std::to_string(i) + ".";
    L.heads = m->openelm ? lh[(size_t)i] : m->heads;
    L.kv_heads = m->openelm ? lkv[(size_t)i] : m->kv_heads;
    L.qdim = L.heads * m->hd;
    L.kvdim = L.kv_heads * m->hd;
    L.ffn = m->openelm ? lff[(size_t)i] : m->ffn;
    const double th = m->gemma ? (i % 6 == 5 ? gtheta : 10000.0) : theta;
    L.theta_u32 = (uint32_t)std::llround(th);  // Math.round(layer.ropeTheta)
    L.window = m->gemma ? (i % 6 == 5 ? 0 : window) : 0;
    L.in_norm = floats(m, p + "attn_norm.weight", m->hidden);
    L.post_norm = floats(m, p + (m->gemma ? "post_attention_norm.weight" : "ffn_norm.weight"), m->hidden);
    if (m->gemma) {
      L.pre_ffn_norm = floats(m, p + "ffn_norm.weight", m->hidden);
      L.post_ffn_norm = floats(m, p + "post_ffw_norm.weight", m->hidden);
    }
    if (m->qk_norm) {
      L.q_norm = floats(m, p + "attn_q_norm.weight", m->hd);
      L.k_norm = floats(m, p + "attn_k_norm.weight", m->hd);
    }
    if (m->openelm) {
      // attn.qkv_proj aliased to attn_qkv (:359), rows q | k | v (:797)
      L.qkv = matrix(m, p + "attn_qkv.weight", m->hidden, (uint64_t)L.qdim + 2 * L.kvdim);
    } else {
      L.q = matrix(m, p + "attn_q.weight", m->hidden, L.qdim);
      L.k = matrix(m, p + "attn_k.weight", m->hidden, L.kvdim);
      L.v = matrix(m, p + "attn_v.weight", m->hidden, L.kvdim);
    }
    L.o = matrix(m, p + "attn_output.weight", L.qdim, m->hidden);
    L.gate = matrix(m, p + "ffn_gate.weight", m->hidden, L.ffn);
    L.up = matrix(m, p + "ffn_up.weight", m->hidden, L.ffn);
    L.down = matrix(m, p + "ffn_down.weight", L.ffn, m->hidden);
    L.kcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
    L.vcache.assign((size_t)L.kvdim * m->ctx, 0.0f);
    m->layers.push_back(std::move(L));
  }
  if (m->gemma && !m->qk_norm) throw std::runtime_error("Gemma WGSL layer is missing required weights");
  // the packed q|k|v path runs only with q/k norms (:1071-1084)
  if (m->openelm && !m->qk_norm) throw std::runtime_error("Llama WGSL layer is missing attention projection weights");
  for (const Layer& L : m->layers)
    if (L.heads <= 0 || L.kv_heads <= 0 || L.heads % L.kv_heads != 0)
      throw std::runtime_error("layer heads must be a positive multiple of kv heads");
}

// LAYER_NORM_WGSL (gpt-wgsl-runtime.ts:1658-1706): 256 threads, sum and sum of
// squares strided then 128..1 trees; variance = max(E[x^2] - mean^2, 0).
void layer_norm(const float* in, const float* w, const float* b, float* out, int n, float eps) {
  float ps[256], pq[256];
  for (int t = 0; t < 256; ++t) {
    float sum = 0.0f, sq = 0.0f;
    for (int i = t; i < n; i += 256) {
      const float v = in[i];
      sum = sum + v;
      const float v2 = v * v;
      sq = sq + v2;
    }
    ps[t] = sum;
    pq[t] = sq;
  }
  for (int st = 128; st >= 1; st >>= 1)
    for (int t = 0; t < st; ++t) {
      ps[t] = ps[t] + ps[t + st];
      pq[t] = pq[t] + pq[t + st];
    }
  const float mean = ps[0] / (float)n;
  const float m2 = mean * mean;
  const float variance = std::max(pq[0] / (float)n - m2, 0.0f);
  const float inv_std = 1.0f / std::sqrt(variance + eps);
  for (int i = 0; i < n; ++i) {
    const float v = (in[i] - mean) * inv_std;
    const float vw = v * w[i];
    out[i] = vw + b[i];
  }
}

// SANITIZE_WGSL (:1726-1746)
inline float sanitize(float v) { return v != v ? 0.0f : std::min(std::max(v, -10000.0f), 10000.0f); }

// GPT-2 attention: ATTENTION_SCORE_WGSL (:1773-1813, 64-thread tree per
// position) and ATTENTION_VALUE_WGSL (:1815-1845: exp weights summed
// unnormalised, divided once by max(denom, 1e-20)).
void attention_gpt(orc_model* m, Layer& L, int pos, const float* q, float* out) {
  const int hd = m->hd, C = m->ctx;
  std::vector<float>& scores = m->scores;
  scores.assign((size_t)L.heads * C, 0.0f);
  m->pool->run(L.heads, [&](int64_t hb, int64_t he) {
    float partial[64];
    for (int64_t head = hb; head < he; ++head) {
      for (int t = 0; t <= pos; ++t) {
        const float* kr = L.kcache.data() + ((size_t)head * C + t) * hd;
        for (int d = 0; d < 64; ++d) partial[d] = q[head * hd + d] * kr[d];
        for (int st = 32; st >= 1; st >>= 1)
          for (int d = 0; d < st; ++d) partial[d] = partial[d] + partial[d + st];
        scores[(size_t)head * C + t] = partial[0] * m->attn_scale;
      }
      const float* sc = scores.data() + (size_t)head * C;
      float mx = -3.402823e38f;
      for (int t = 0; t <= pos; ++t) mx = std::fmax(mx, sc[t]);
      for (int d = 0; d < hd; ++d) {
        float denom = 0.0f, acc = 0.0f;
        for (int t = 0; t <= pos; ++t) {
          const float p = std::exp(sc[t] - mx);
          denom = denom + p;
          const float pv = p * L.vcache[((size_t)head * C + t) * hd + d];
          acc = acc + pv;
        }
        out[head * hd + d] = acc / std::max(denom, 1e-20f);
      }
    }
  });
}

// ARGMAX_STAGE1/2 of the GPT-2 runtime (:1896-2004): trees keeping the left
// slot unless the right one is strictly greater (so NaN in the left slot stays
// and ties go by tree position), padding -3.402823e38 with index 0; the
// penalty applies to the listed ids whenever it is not 1.
void argmax_gpt(const float* logits, int64_t vocab, const std::vector<int32_t>& sorted_ids, float pen,
                uint8_t* pairs, int32_t* token) {
  const int64_t groups = (vocab + 255) / 256;
  float cv[256];
  uint32_t ci[256];
  for (int64_t gidx = 0; gidx < groups; ++gidx) {
    float vals[256];
    uint32_t idx[256];
    for (int t = 0; t < 256; ++t) {
      const int64_t i = gidx * 256 + t;
      if (i < vocab) {
        float v = logits[i];
        if (!sorted_ids.empty() && std::binary_search(sorted_ids.begin(), sorted_ids.end(), (int32_t)i))
          v = v > 0.0f ? v / pen : v * pen;
        vals[t] = v;
        idx[t] = (uint32_t)i;
      } else {
        vals[t] = kNegBig;
        idx[t] = 0u;
      }
    }
    for (int st = 128; st >= 1; st >>= 1)
      for (int t = 0; t < st; ++t)
        if (vals[t + st] > vals[t]) {
          vals[t] = vals[t + st];
          idx[t] = idx[t + st];
        }
    cv[gidx] = vals[0];
    ci[gidx] = idx[0];
    if (pairs) {
      std::memcpy(pairs + 8 * gidx, &vals[0], 4);
      std::memcpy(pairs + 8 * gidx + 4, &idx[0], 4);
    }
  }
  for (int64_t t = groups; t < 256; ++t) {
    cv[t] = kNegBig;
    ci[t] = 0u;
  }
  for (int st = 128; st >= 1; st >>= 1)
    for (int t = 0; t < st; ++t)
      if (cv[t + st] > cv[t]) {
        cv[t] = cv[t + st];
        ci[t] = ci[t + st];
      }
  *token = (int32_t)ci[0];
}

void embedding(orc_model* m, int32_t token, float* out) {
  // GGUF_*_EMBEDDING_WGSL (:2615-2866): dequant(token row) * EMBEDDING_SCALE
  if (token < 0 || token >= m->vocab) throw std::runtime_error("token id " + std::to_string(token) + " outside embedding table");
  for (int k = 0; k < m->hidden; ++k) {
    const float w = weight_at(m->embed.type, m->embed.data, (uint64_t)token, (uint64_t)k, m->embed.k);
    out[k] = w * m->embed_scale;
  }
}

}  // namespace

extern "C" {

int orc_dequant(uint32_t type, const uint8_t* blocks, int64_t n, float* out) {
  BlockGeom g;
  if (!geom(type, &g) || n % g.elems) return -1;
  for (int64_t i = 0; i < n; ++i) out[i] = weight_at(type, blocks, 0, (uint64_t)i, (uint64_t)n);
  return 0;
}

int orc_decode_rows(uint32_t type, const uint8_t* blocks, int64_t n_rows, int64_t row_len, float* out) {
  BlockGeom g;
  if (!geom(type, &g) || row_len % g.elems || n_rows < 0) return -1;
  for (int64_t r = 0; r < n_rows; ++r) decode_row(type, blocks, (uint64_t)r, (uint64_t)row_len, out + r * row_len);
  return 0;
}

int orc_matvec(uint32_t type, const uint8_t* blocks, int64_t n_rows, int64_t row_len, const float* x, float* y,
               int n_threads) {
  BlockGeom g;
  if (!geom(type, &g) || row_len % g.elems) return -1;
  Pool pool(n_threads);
  matvec(pool, type, blocks, (uint64_t)n_rows, (uint64_t)row_len, x, y);
  return 0;
}

orc_model* orc_model_load(const char* path, const orc_model_def* def, char* err, size_t err_len) {
  orc_model* m = new orc_model();
  try {
    load_gguf(path, &m->g);
    build(m, def);
    m->pool = new Pool(def->n_threads > 0 ? def->n_threads : 1);
    const int H = m->hidden;
    const int qdim = m->heads * m->hd, kvdim = m->kv_heads * m->hd;
    m->hA.assign(H, 0);
    m->hB.assign(H, 0);
    m->hC.assign(H, 0);
    m->norm.assign(H, 0);
    m->q.assign(qdim, 0);
    m->qn.assign(qdim, 0);
    m->k.assign(kvdim, 0);
    m->v.assign(kvdim, 0);
    m->attn.assign(qdim, 0);
    m->gate.assign(m->ffn, 0);
    m->up.assign(m->ffn, 0);
    m->ff.assign(m->ffn, 0);
    m->logits.assign(m->vocab, 0);
    m->candidates.assign((size_t)(m->lfm || m->granite ? 256 : (m->vocab + 255) / 256) * 8, 0);
    if (m->granite) {
      m->mproj.assign((size_t)m->ssm_inner + m->ssm_conv + m->ssm_heads, 0);
      m->mconv.assign(m->ssm_conv, 0);
      m->my.assign(m->ssm_inner, 0);
      m->mnormed.assign(m->ssm_inner, 0);
    }
    if (m->lfm) {
      m->proj.assign(3 * (size_t)H, 0);
      m->conv_mid.assign(H, 0);
    }
    if (m->gpt) m->qkv.assign(3 * (size_t)H, 0);
    if (m->openelm) m->qkv.assign((size_t)qdim + 2 * kvdim, 0);
    return m;
  } catch (const std::exception& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    delete m->pool;
    delete m;
    return nullptr;
  }
}

void orc_model_free(orc_model* m) {
  if (!m) return;
  delete m->pool;
  delete m;
}

int orc_model_context(const orc_model* m) { return m->ctx; }
int orc_model_is_gpt(const orc_model* m) { return m->gpt ? 1 : 0; }
int orc_model_vocab(const orc_model* m) { return m->vocab; }
int orc_model_position(const orc_model* m) { return m->pos; }

void orc_model_reset(orc_model* m) {
  m->pos = 0;
  for (auto& L : m->layers) {
    std::fill(L.kcache.begin(), L.kcache.end(), 0.0f);
    std::fill(L.vcache.begin(), L.vcache.end(), 0.0f);
    std::fill(L.conv_state.begin(), L.conv_state.end(), 0.0f);  // LfmWgslEngine.reset (:711-724)
    std::fill(L.mconv_state.begin(), L.mconv_state.end(), 0.0f);  // GraniteWgslEngine.reset (:750-763)
    std::fill(L.ssm_state.begin(), L.ssm_state.end(), 0.0f);
  }
}

int orc_model_fake_context(orc_model* m, int pos, uint64_t seed) {
  // Same values as the engine's synthetic fill: element i of layer l's
  // [kv_heads][pos][hd] block is u = ((mix64(seed_l + i*0x9e37..) >> 40) & 0xffff)/65536 - 0.5
  // with seed_l = seed + 1000003*l; K = u, V = -u (rounded like the cache).
  if (pos < 0 || pos > m->ctx) return -1;
  auto mix64 = [](uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  for (size_t l = 0; l < m->layers.size(); ++l) {
    Layer& L = m->layers[l];
    const uint64_t sl = seed + 1000003ull * l;
    for (int kh = 0; kh < L.kv_heads; ++kh)
      for (int t = 0; t < pos; ++t)
        for (int d = 0; d < m->hd; ++d) {
          const uint64_t i = ((uint64_t)kh * pos + t) * m->hd + d;
          const uint64_t z = mix64(sl + i * 0x9e3779b97f4a7c15ull);
          const float a = (float)((z >> 40) & 0xffff) / 65536.0f - 0.5f;
          L.kcache[((size_t)kh * m->ctx + t) * m->hd + d] = kv_round(m, a);
          L.vcache[((size_t)kh * m->ctx + t) * m->hd + d] = kv_round(m, -a);
        }
  }
  m->pos = pos;
  return 0;
}

int orc_argmax_gpt(const float* logits, int64_t vocab, const int32_t* penalized, int64_t n_penalized,
                   double repetition_penalty, uint8_t* candidate_pairs, int32_t* token) {
  // the GPT-2 runtime's stage 1/2 (gpt-wgsl-runtime.ts:1882-2004); its penalty list
  // applies whenever the penalty is not 1 (:789-798)
  if (vocab <= 0 || (vocab + 255) / 256 > 256) return -1;
  std::vector<int32_t> ids;
  if (repetition_penalty != 1.0 && n_penalized > 0) {
    ids.assign(penalized, penalized + n_penalized);
    std::sort(ids.begin(), ids.end());
  }
  const float pen = (float)(uint32_t)std::floor(repetition_penalty * 1000 + 0.5) / 1000.0f;
  argmax_gpt(logits, vocab, ids, pen, candidate_pairs, token);
  return 0;
}

int orc_argmax(const float* logits, int64_t vocab, const int32_t* penalized, int64_t n_penalized,
               double repetition_penalty, uint8_t* candidate_pairs, int32_t* token) {
  // ARGMAX_STAGE1 + ARGMAX_STAGE2 (llama-wgsl-runtime.ts:3645-3791) over a logits vector
  const bool apply = repetition_penalty > 1 && n_penalized > 0;
  std::vector<int32_t> ids(penalized, penalized + (apply ? n_penalized : 0));
  std::sort(ids.begin(), ids.end());
  const float pen = (float)(uint32_t)std::floor(repetition_penalty * 1000 + 0.5) / 1000.0f;
  const int64_t groups = (vocab + 255) / 256;
  std::vector<float> cv(groups);
  std::vector<uint32_t> ci(groups);
  for (int64_t g = 0; g < groups; ++g) {
    float vals[256];
    uint32_t idx[256];
    for (int t = 0; t < 256; ++t) {
      const int64_t i = g * 256 + t;
      if (i < vocab) {
        float v = logits[i];
        if (apply && std::binary_search(ids.begin(), ids.end(), (int32_t)i)) v = v > 0.0f ? v / pen : v * pen;
        vals[t] = v;
        idx[t] = (uint32_t)i;
      } else {
        vals[t] = kNegBig;
        idx[t] = 0xffffffffu;
      }
    }
    for (int st = 128; st >= 1; st >>= 1)
      for (int t = 0; t < st; ++t)
        if (better(vals[t + st], idx[t + st], vals[t], idx[t])) {
          vals[t] = vals[t + st];
          idx[t] = idx[t + st];
        }
    cv[g] = vals[0];
    ci[g] = idx[0];
    if (candidate_pairs) {
      std::memcpy(candidate_pairs + 8 * g, &vals[0], 4);
      std::memcpy(candidate_pairs + 8 * g + 4, &idx[0], 4);
    }
  }
  float bv[256];
  uint32_t bi[256];
  for (int t = 0; t < 256; ++t) {
    float v = -3.402823e38f;
    uint32_t i = 0xffffffffu;
    for (int64_t g = t; g < groups; g += 256)
      if (better(cv[g], ci[g], v, i)) {
        v = cv[g];
        i = ci[g];
      }
    bv[t] = v;
    bi[t] = i;
  }
  for (int st = 128; st >= 1; st >>= 1)
    for (int t = 0; t < st; ++t)
      if (better(bv[t + st], bi[t + st], bv[t], bi[t])) {
        bv[t] = bv[t + st];
        bi[t] = bi[t + st];
      }
  *token = (int32_t)bi[0];
  return 0;
}

double orc_uniform(uint64_t seed, uint64_t step) {
  uint64_t z = seed + 0x9e3779b97f4a7c15ull * (step + 1);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z = z ^ (z >> 31);
  return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

int32_t orc_sample_candidates(const uint8_t* pairs, int64_t n_groups, const orc_sampling* s, const int32_t* seen,
                              int64_t n_seen, double uniform) {
  // sampleFromCandidateBuffer (sampling.ts:23-76)
  struct Cand {
    double val;
    uint32_t id;
  };
  std::vector<int32_t> seen_sorted(seen, seen + n_seen);
  std::sort(seen_sorted.begin(), seen_sorted.end());
  const double rp = std::max((double)s->repetition_penalty, 1e-6);
  std::vector<Cand> c;
  for (int64_t i = 0; i < n_groups; ++i) {
    float fv;
    uint32_t id;
    std::memcpy(&fv, pairs + 8 * i, 4);
    std::memcpy(&id, pairs + 8 * i + 4, 4);
    double val = fv;
    if (!std::isfinite(val) || id == 0xffffffffu) continue;
    if (rp != 1 && std::binary_search(seen_sorted.begin(), seen_sorted.end(), (int32_t)id))
      val = val > 0 ? val / rp : val * rp;
    c.push_back({val, id});
  }
  std::stable_sort(c.begin(), c.end(), [](const Cand& a, const Cand& b) { return b.val - a.val < 0; });
  const int top_k = s->top_k > 0 ? s->top_k : 0;
  std::vector<Cand> lim = top_k > 0 ? std::vector<Cand>(c.begin(), c.begin() + std::min<size_t>(top_k, c.size())) : c;
  const double temp = s->temperature;
  if (temp <= 0) return !lim.empty() ? (int32_t)lim[0].id : !c.empty() ? (int32_t)c[0].id : 0;
  const double top_p = std::min(std::max((double)s->top_p, 0.0), 1.0);
  const double maxv = lim.empty() ? 0 : lim[0].val;
  std::vector<double> probs;
  for (auto& x : lim) probs.push_back(std::exp((x.val - maxv) / temp));
  double total = 0;
  for (double p : probs) total += p;
  size_t cutoff = lim.size();
  if (top_p < 1 && total > 0) {
    double cdf = 0;
    for (size_t i = 0; i < probs.size(); ++i) {
      cdf += probs[i] / total;
      if (cdf >= top_p) {
        cutoff = i + 1;
        break;
      }
    }
  }
  double sample_total = 0;
  for (size_t i = 0; i < cutoff; ++i) sample_total += probs[i];
  double r = uniform * sample_total;
  for (size_t i = 0; i < cutoff; ++i) {
    r -= probs[i];
    if (r <= 0) return (int32_t)lim[i].id;
  }
  if (cutoff >= 1 && cutoff - 1 < lim.size()) return (int32_t)lim[cutoff - 1].id;
  return !lim.empty() ? (int32_t)lim[0].id : 0;
}

// GptWgslEngine.runToken (gpt-wgsl-runtime.ts:749-840)
static int32_t run_token_gpt(orc_model* m, int32_t token, int32_t need_logits, const orc_sampling* s,
                             const int32_t* penalized, int64_t n_penalized, const int32_t* seen, int64_t n_seen,
                             double uniform) {
  if (m->pos >= m->ctx) throw std::runtime_error("GPT WGSL context exhausted at " + std::to_string(m->ctx) + " tokens");
  const int H = m->hidden, pos = m->pos, C = m->ctx;
  Pool& pool = *m->pool;
  float* hidden = m->hA.data();
  embedding(m, token, hidden);
  for (int h = 0; h < H; ++h) hidden[h] = hidden[h] + m->pos_embd[(size_t)pos * H + h];  // ADD_POSITION (:1639-1656)
  for (size_t li = 0; li < m->layers.size(); ++li) {
    Layer& L = m->layers[li];
    layer_norm(hidden, L.in_norm.data(), L.in_norm_b.data(), m->norm.data(), H, m->norm_eps);
    matvec(pool, L.qkv.type, L.qkv.data, L.qkv.n, L.qkv.k, m->norm.data(), m->qkv.data());
    for (int i = 0; i < 3 * H; ++i) m->qkv[i] = m->qkv[i] + L.qkv_b[i];
    for (int hh = 0; hh < L.heads; ++hh)  // STORE_KV (:1748-1771)
      for (int d = 0; d < m->hd; ++d) {
        const size_t ci = ((size_t)hh * C + pos) * m->hd + d;
        L.kcache[ci] = kv_round(m, m->qkv[H + hh * m->hd + d]);
        L.vcache[ci] = kv_round(m, m->qkv[2 * H + hh * m->hd + d]);
      }
    attention_gpt(m, L, pos, m->qkv.data(), m->attn.data());
    matvec(pool, L.o.type, L.o.data, L.o.n, L.o.k, m->attn.data(), m->hB.data());
    for (int i = 0; i < H; ++i) m->hB[i] = m->hB[i] + L.o_b[i];
    for (int i = 0; i < H; ++i) hidden[i] = sanitize(hidden[i] + m->hB[i]);
    layer_norm(hidden, L.post_norm.data(), L.post_norm_b.data(), m->norm.data(), H, m->norm_eps);
    matvec(pool, L.up.type, L.up.data, L.up.n, L.up.k, m->norm.data(), m->ff.data());
    for (int i = 0; i < L.ffn; ++i) m->ff[i] = gelu_tanh(m->ff[i] + L.up_b[i]);
    matvec(pool, L.down.type, L.down.data, L.down.n, L.down.k, m->ff.data(), m->hB.data());
    for (int i = 0; i < H; ++i) m->hB[i] = m->hB[i] + L.down_b[i];
    for (int i = 0; i < H; ++i) hidden[i] = sanitize(hidden[i] + m->hB[i]);
  }
  m->last_residual.assign(hidden, hidden + H);
  int32_t best = 0;
  if (need_logits) {
    layer_norm(hidden, m->final_norm.data(), m->final_norm_b.data(), m->norm.data(), H, m->norm_eps);
    matvec(pool, m->lm_head.type, m->lm_head.data, (uint64_t)m->vocab, m->lm_head.k, m->norm.data(),
           m->logits.data());
    // the penalty list is the last maxContext seen ids whenever the penalty is not 1 (:785-796)
    const double rp = s ? s->repetition_penalty : 1.0;
    std::vector<int32_t> ids;
    if (rp != 1.0 && n_penalized > 0) {
      const int64_t keep = std::min<int64_t>(n_penalized, m->ctx);
      ids.assign(penalized + (n_penalized - keep), penalized + n_penalized);
      std::sort(ids.begin(), ids.end());
    }
    const float pen = (float)(uint32_t)std::floor(rp * 1000 + 0.5) / 1000.0f;
    argmax_gpt(m->logits.data(), m->vocab, ids, pen, m->candidates.data(), &best);
    const bool sampling = s && (s->temperature > 0 || s->top_p < 1 || s->top_k > 0);
    if (sampling) best = orc_sample_candidates(m->candidates.data(), (m->vocab + 255) / 256, s, seen, n_seen, uniform);
  }
  m->pos += 1;
  return best;
}

}  // extern "C"

namespace {

// Q8_MATVEC_WGSL (lfm-wgsl-runtime.ts:1225-1276) over the 36-byte repacked
// blocks: sum = sum + input[k] * q8 * scale, i.e. (x * q) * d with the scale
// widened exactly from binary16 (packQ8_0ForGpu, :433-455); 128 strided lane
// sums, then the stride 64..1 tree.
float matvec_row_lfm_q8(const uint8_t* w, uint64_t row, uint64_t K, const float* x) {
  float partial[128];
  for (int t = 0; t < 128; ++t) partial[t] = 0.0f;
  for (uint64_t k = 0; k < K; ++k) {
    const uint64_t base = (row * (K / 32) + (k >> 5)) * 34;
    const float xq = x[k] * (float)i8_at(w, base + 2 + (k & 31));
    const float prod = xq * f16_at(w, base);
    partial[k & 127] = partial[k & 127] + prod;
  }
  for (int st = 64; st >= 1; st >>= 1)
    for (int t = 0; t < st; ++t) partial[t] = partial[t] + partial[t + st];
  return partial[0];
}

// The LFM runtime's linear layer: Q8_0 in the order above, Q4_K / Q6_K as
// sum + input[k] * dequant(w) (Q4K_MATVEC_WGSL :1398-1444, Q6K_MATVEC_WGSL
// :1446-1492), which is the llama runtime's matvec.
void matvec_lfm(Pool& pool, const Matrix& W, uint64_t N, const float* x, float* y) {
  if (W.type != 8) {
    matvec(pool, W.type, W.data, N, W.k, x, y);
    return;
  }
  pool.run((int64_t)N, [&](int64_t b, int64_t e) {
    for (int64_t n = b; n < e; ++n) y[n] = matvec_row_lfm_q8(W.data, (uint64_t)n, W.k, x);
  });
}

// TOPK256_WGSL (:1925-1947), also the first stage of ARGMAX_WGSL (:1880-1923):
// slot t keeps the first strictly greater logit among ids t, t + 256, ...,
// starting from (-3.402823e38, 0); NaN never replaces it.
void lfm_top256(const float* logits, int64_t vocab, uint8_t* pairs) {
  for (int t = 0; t < 256; ++t) {
    float mx = kNegBig;
    uint32_t id = 0;
    for (int64_t i = t; i < vocab; i += 256)
      if (logits[i] > mx) {
        mx = logits[i];
        id = (uint32_t)i;
      }
    std::memcpy(pairs + 8 * t, &mx, 4);
    std::memcpy(pairs + 8 * t + 4, &id, 4);
  }
}

// ARGMAX_WGSL's second stage (:1903-1922): a stride 128..1 tree keeping the
// left slot unless the right one is strictly greater.
int32_t lfm_argmax(const uint8_t* pairs) {
  float v[256];
  uint32_t id[256];
  for (int t = 0; t < 256; ++t) {
    std::memcpy(&v[t], pairs + 8 * t, 4);
    std::memcpy(&id[t], pairs + 8 * t + 4, 4);
  }
  for (int st = 128; st >= 1; st >>= 1)
    for (int t = 0; t < st; ++t)
      if (v[t + st] > v[t]) {
        v[t] = v[t + st];
        id[t] = id[t + st];
      }
  return (int32_t)id[0];
}

// CONV_BLOCK_WGSL (:1641-1672): cur = B * x; the two previous values of the
// channel's state and cur through the three taps; state shifted; out = C * conv.
void lfm_conv_block(Layer& L, const float* proj, float* out, int H) {
  for (int h = 0; h < H; ++h) {
    const float a = proj[h], b = proj[H + h], c = proj[2 * H + h];
    const float cur = a * c;
    float* st = L.conv_state.data() + 3 * (size_t)h;
    const float* w = L.conv_w.data() + 3 * (size_t)h;
    const float p1 = st[1], p2 = st[2];
    const float t0 = p1 * w[0], t1 = p2 * w[1], t2 = cur * w[2];
    const float conv = (t0 + t1) + t2;
    st[0] = p1;
    st[1] = p2;
    st[2] = cur;
    out[h] = b * conv;
  }
}

// LfmWgslEngine.runToken (:727-809)
int32_t run_token_lfm(orc_model* m, int32_t token, int32_t need_logits, const orc_sampling* s, const int32_t* seen,
                      int64_t n_seen, double uniform) {
  if (m->pos >= m->ctx) throw std::runtime_error("LFM WGSL context exhausted at " + std::to_string(m->ctx) + " tokens");
  const int H = m->hidden, pos = m->pos;
  Pool& pool = *m->pool;
  float* hA = m->hA.data();
  float* hB = m->hB.data();
  embedding(m, token, hA);  // EMBEDDING_{Q8,Q4K,Q6K}_WGSL (:1301-1323, :1494-1540): the dequantized row
  for (size_t li = 0; li < m->layers.size(); ++li) {
    Layer& L = m->layers[li];
    rms_norm(hA, L.in_norm.data(), m->norm.data(), H, m->norm_eps);
    if (L.conv) {
      matvec_lfm(pool, L.conv_in, 3 * (uint64_t)H, m->norm.data(), m->proj.data());
      lfm_conv_block(L, m->proj.data(), m->conv_mid.data(), H);
      matvec_lfm(pool, L.conv_out, (uint64_t)H, m->conv_mid.data(), hB);
    } else {
      matvec_lfm(pool, L.q, (uint64_t)L.qdim, m->norm.data(), m->q.data());
      matvec_lfm(pool, L.k, (uint64_t)L.kvdim, m->norm.data(), m->k.data());
      matvec_lfm(pool, L.v, (uint64_t)L.kvdim, m->norm.data(), m->v.data());
      qk_rope_store(m, L, pos, true, m->qn.data());  // QK_NORM_ROPE_STORE_WGSL (:1709-1786)
      attention(m, L, pos, m->qn.data(), m->attn.data());  // ATTENTION_SCORE / _VALUE_WGSL (:1788-1878)
      matvec_lfm(pool, L.o, (uint64_t)H, m->attn.data(), hB);
    }
    add_rms_norm(hA, hB, L.post_norm.data(), m->norm.data(), H, m->norm_eps);  // opAddNorm: hB = hA + hB
    matvec_lfm(pool, L.gate, (uint64_t)L.ffn, m->norm.data(), m->gate.data());
    matvec_lfm(pool, L.up, (uint64_t)L.ffn, m->norm.data(), m->up.data());
    for (int i = 0; i < L.ffn; ++i) m->ff[i] = silu_mul(m->gate[i], m->up[i]);
    matvec_lfm(pool, L.down, (uint64_t)H, m->ff.data(), hA);  // mlpDown writes hiddenA
    for (int i = 0; i < H; ++i) hA[i] = hB[i] + hA[i];       // ffnAdd: hiddenA = hiddenB + hiddenA
  }
  m->last_residual.assign(hA, hA + H);
  int32_t best = 0;
  if (need_logits) {
    rms_norm(hA, m->final_norm.data(), m->norm.data(), H, m->norm_eps);
    matvec_lfm(pool, m->lm_head, (uint64_t)m->vocab, m->norm.data(), m->logits.data());
    lfm_top256(m->logits.data(), m->vocab, m->candidates.data());
    // needsCandidateReadback (sampling.ts:18-21): sampling, or a penalty that is not 1
    const bool cand = s && (s->temperature > 0 || s->top_p < 1 || s->top_k > 0 || s->repetition_penalty != 1);
    best = cand ? orc_sample_candidates(m->candidates.data(), 256, s, seen, n_seen, uniform)
                : lfm_argmax(m->candidates.data());
  }
  m->pos += 1;
  return best;
}

float silu_g(float x) {  // silu of MAMBA_CONV / MAMBA_GATE_NORM / SILU_MUL (:1484-1486, :1579-1581)
  return x / (1.0f + std::exp(-x));
}

float softplus_g(float x) {  // MAMBA_SSM_WGSL's softplus (:1524-1526)
  return x > 20.0f ? x + std::log(1.0f + std::exp(-x)) : std::log(1.0f + std::exp(x));
}

// MAMBA_CONV_WGSL (:1476-1511): the channel's window shifts by one (slot 0
// drops out, the new xBC value enters slot 3), then four taps over the
// previous three values and the new one, the bias, and silu.
void granite_conv(orc_model* m, Layer& L, const float* proj, float* out) {
  const int inner = m->ssm_inner;
  for (int c = 0; c < m->ssm_conv; ++c) {
    const float nv = proj[inner + c];
    float* st = L.mconv_state.data() + 4 * (size_t)c;
    const float p1 = st[1], p2 = st[2], p3 = st[3];
    st[0] = p1;
    st[1] = p2;
    st[2] = p3;
    st[3] = nv;
    const float* w = L.c1d_w.data() + 4 * (size_t)c;
    const float y = (((p1 * w[0] + p2 * w[1]) + p3 * w[2]) + nv * w[3]) + L.c1d_b[c];
    out[c] = silu_g(y);
  }
}

// MAMBA_SSM_WGSL (:1513-1562): per (head n, channel h) a 128-state selective
// scan step with dt = softplus(dt_raw + dt_bias), decay = exp(dt * A), the
// shared B and C of the single group, the state sum through the stride 64..1
// tree, plus D * x.
void granite_ssm(orc_model* m, Layer& L, const float* proj, const float* conv, float* y) {
  const int inner = m->ssm_inner, S = m->ssm_state, hdim = m->ssm_hdim;
  m->pool->run(m->ssm_heads, [&](int64_t nb, int64_t ne) {
    float partial[128];
    for (int64_t n = nb; n < ne; ++n) {
      const float dt = softplus_g(proj[inner + m->ssm_conv + n] + L.dt_b[n]);
      const float decay = std::exp(dt * L.a_neg[n]);
      for (int h = 0; h < hdim; ++h) {
        const int nh = (int)n * hdim + h;
        const float hs = conv[nh];
        for (int st = 0; st < S; ++st) {
          const float b = conv[inner + st], c = conv[inner + S + st];
          float& sv = L.ssm_state[(size_t)nh * S + st];
          const float next = sv * decay + (dt * b) * hs;
          sv = next;
          partial[st] = next * c;
        }
        for (int stride = 64; stride >= 1; stride >>= 1)
          for (int t = 0; t < stride; ++t) partial[t] = partial[t] + partial[t + stride];
        y[nh] = partial[0] + L.d_w[n] * hs;
      }
    }
  });
}

// MAMBA_GATE_NORM_WGSL (:1564-1608): v = y * silu(z) over the inner size,
// RMSNorm over the 256-lane strided sums, ((y * silu(z)) * inv) * w.
void granite_gate_norm(orc_model* m, const Layer& L, const float* z, const float* y, float* out) {
  const int n = m->ssm_inner;
  float partial[256];
  for (int t = 0; t < 256; ++t) {
    float sum = 0.0f;
    for (int i = t; i < n; i += 256) {
      const float v = y[i] * silu_g(z[i]);
      sum = sum + v * v;
    }
    partial[t] = sum;
  }
  for (int s = 128; s >= 1; s >>= 1)
    for (int t = 0; t < s; ++t) partial[t] = partial[t] + partial[t + s];
  const float inv = 1.0f / std::sqrt(partial[0] / (float)n + m->norm_eps);
  for (int i = 0; i < n; ++i) out[i] = ((y[i] * silu_g(z[i])) * inv) * L.ssm_norm[i];
}

// ADD_SCALED_RMS_NORM_WGSL (:1415-1456): residual += add * 0.246, then RMSNorm.
void granite_add_norm(float* residual, const float* add, const float* w, float* out, int n, float eps) {
  for (int i = 0; i < n; ++i) residual[i] = residual[i] + add[i] * 0.246f;
  rms_norm(residual, w, out, n, eps);
}

// GraniteWgslEngine.runToken (:769-858)
int32_t run_token_granite(orc_model* m, int32_t token, int32_t need_logits, const orc_sampling* s,
                          const int32_t* seen, int64_t n_seen, double uniform) {
  if (m->pos >= m->ctx)
    throw std::runtime_error("Granite WGSL context exhausted at " + std::to_string(m->ctx) + " tokens");
  const int H = m->hidden, pos = m->pos;
  Pool& pool = *m->pool;
  float* hA = m->hA.data();
  float* hB = m->hB.data();
  embedding(m, token, hA);  // EMBEDDING_{Q8,Q4_K,Q6_K}_WGSL (:1348-1372): dequant * 12
  for (size_t li = 0; li < m->layers.size(); ++li) {
    Layer& L = m->layers[li];
    rms_norm(hA, L.in_norm.data(), m->norm.data(), H, m->norm_eps);
    if (L.mamba) {
      matvec(pool, L.ssm_in.type, L.ssm_in.data, L.ssm_in.n, L.ssm_in.k, m->norm.data(), m->mproj.data());
      granite_conv(m, L, m->mproj.data(), m->mconv.data());
      granite_ssm(m, L, m->mproj.data(), m->mconv.data(), m->my.data());
      granite_gate_norm(m, L, m->mproj.data(), m->my.data(), m->mnormed.data());
      matvec(pool, L.ssm_out.type, L.ssm_out.data, L.ssm_out.n, L.ssm_out.k, m->mnormed.data(), hB);
    } else {
      matvec(pool, L.q.type, L.q.data, L.q.n, L.q.k, m->norm.data(), m->q.data());
      matvec(pool, L.k.type, L.k.data, L.k.n, L.k.k, m->norm.data(), m->k.data());
      matvec(pool, L.v.type, L.v.data, L.v.n, L.v.k, m->norm.data(), m->v.data());
      // STORE_KV_WGSL (:1610-1631): no rotary embedding
      for (int i = 0; i < L.kvdim; ++i) {
        const int kh = i / m->hd, d = i % m->hd;
        const size_t at = ((size_t)kh * m->ctx + pos) * m->hd + d;
        L.kcache[at] = kv_round(m, m->k[i]);
        L.vcache[at] = kv_round(m, m->v[i]);
      }
      attention(m, L, pos, m->q.data(), m->attn.data());  // ATTENTION_SCORE / _VALUE_WGSL (:1633-1718)
      matvec(pool, L.o.type, L.o.data, L.o.n, L.o.k, m->attn.data(), hB);
    }
    granite_add_norm(hA, hB, L.post_norm.data(), m->norm.data(), H, m->norm_eps);
    matvec(pool, L.gate.type, L.gate.data, L.gate.n, L.gate.k, m->norm.data(), m->gate.data());
    matvec(pool, L.up.type, L.up.data, L.up.n, L.up.k, m->norm.data(), m->up.data());
    for (int i = 0; i < L.ffn; ++i) m->ff[i] = silu_mul(m->gate[i], m->up[i]);
    matvec(pool, L.down.type, L.down.data, L.down.n, L.down.k, m->ff.data(), hB);
    for (int i = 0; i < H; ++i) hA[i] = hA[i] + hB[i] * 0.246f;  // ADD_SCALED_WGSL (:1458-1474)
  }
  m->last_residual.assign(hA, hA + H);
  int32_t best = 0;
  if (need_logits) {
    rms_norm(hA, m->final_norm.data(), m->norm.data(), H, m->norm_eps);
    matvec(pool, m->lm_head.type, m->lm_head.data, (uint64_t)m->vocab, m->lm_head.k, m->norm.data(),
           m->logits.data());
    for (int i = 0; i < m->vocab; ++i) m->logits[i] = m->logits[i] * 0.333333333333333333f;  // SCALE_LOGITS_WGSL
    lfm_top256(m->logits.data(), m->vocab, m->candidates.data());  // TOPK256_WGSL / ARGMAX_WGSL (:1753-1820)
    const bool cand = s && (s->temperature > 0 || s->top_p < 1 || s->top_k > 0 || s->repetition_penalty != 1);
    best = cand ? orc_sample_candidates(m->candidates.data(), 256, s, seen, n_seen, uniform)
                : lfm_argmax(m->candidates.data());
  }
  m->pos += 1;
  return best;
}

}  // namespace

extern "C" {

int orc_model_is_lfm(const orc_model* m) { return m->lfm ? 1 : 0; }
int orc_model_is_granite(const orc_model* m) { return m->granite ? 1 : 0; }

int orc_lfm_select(const float* logits, int64_t vocab, uint8_t* candidate_pairs, int32_t* token) {
  uint8_t pairs[256 * 8];
  lfm_top256(logits, vocab, pairs);
  if (candidate_pairs) std::memcpy(candidate_pairs, pairs, sizeof pairs);
  if (token) *token = lfm_argmax(pairs);
  return 0;
}

int orc_model_run_token(orc_model* m, int32_t token, int32_t need_logits, const orc_sampling* s,
                        const int32_t* penalized, int64_t n_penalized, const int32_t* seen, int64_t n_seen,
                        double uniform, int32_t* out_token, char* err, size_t err_len) {
  try {
    if (m->lfm) {
      *out_token = run_token_lfm(m, token, need_logits, s, seen, n_seen, uniform);
      return 0;
    }
    if (m->granite) {
      *out_token = run_token_granite(m, token, need_logits, s, seen, n_seen, uniform);
      return 0;
    }
    if (m->gpt) {
      *out_token = run_token_gpt(m, token, need_logits, s, penalized, n_penalized, seen, n_seen, uniform);
      return 0;
    }
    if (m->pos >= m->ctx)
      throw std::runtime_error("Llama WGSL context exhausted at " + std::to_string(m->ctx) + " tokens");
    const int H = m->hidden, pos = m->pos;
    Pool& pool = *m->pool;
    embedding(m, token, m->hA.data());
    float* residual = m->hA.data();
    float* other = m->hB.data();
    for (size_t li = 0; li < m->layers.size(); ++li) {
      Layer& L = m->layers[li];
      if (m->gemma) {
        // :1044-1067
        rms_norm(residual, L.in_norm.data(), m->norm.data(), H, m->norm_eps);
        matvec(pool, L.q.type, L.q.data, L.q.n, L.q.k, m->norm.data(), m->q.data());
        matvec(pool, L.k.type, L.k.data, L.k.n, L.k.k, m->norm.data(), m->k.data());
        matvec(pool, L.v.type, L.v.data, L.v.n, L.v.k, m->norm.data(), m->v.data());
        qk_rope_store(m, L, pos, true, m->qn.data());
        attention(m, L, pos, m->qn.data(), m->attn.data());
        matvec(pool, L.o.type, L.o.data, L.o.n, L.o.k, m->attn.data(), m->hB.data());
        rms_norm(m->hB.data(), L.post_norm.data(), m->hC.data(), H, m->norm_eps);
        for (int i = 0; i < H; ++i) m->hC[i] = std::min(std::max(residual[i] + m->hC[i], -65000.0f), 65000.0f);
        residual = m->hC.data();
        rms_norm(residual, L.pre_ffn_norm.data(), m->norm.data(), H, m->norm_eps);
        matvec(pool, L.gate.type, L.gate.data, L.gate.n, L.gate.k, m->norm.data(), m->gate.data());
        matvec(pool, L.up.type, L.up.data, L.up.n, L.up.k, m->norm.data(), m->up.data());
        for (int i = 0; i < L.ffn; ++i) m->ff[i] = gelu_tanh(m->gate[i]) * m->up[i];
        matvec(pool, L.down.type, L.down.data, L.down.n, L.down.k, m->ff.data(), m->hB.data());
        rms_norm(m->hB.data(), L.post_ffn_norm.data(), m->hA.data(), H, m->norm_eps);
        for (int i = 0; i < H; ++i) m->hA[i] = std::min(std::max(residual[i] + m->hA[i], -65000.0f), 65000.0f);
        residual = m->hA.data();
        other = m->hB.data();
      } else {
        // :1069-1103
        rms_norm(residual, L.in_norm.data(), m->norm.data(), H, m->norm_eps);
        if (m->openelm) {
          // q4Matvec(norm, qkvProj, qkv), then qkvNormRopeStore (:1071-1074, :3025-3120),
          // whose arithmetic is qkNormRopeStore's over the packed row
          matvec(pool, L.qkv.type, L.qkv.data, L.qkv.n, L.qkv.k, m->norm.data(), m->qkv.data());
          std::copy(m->qkv.begin(), m->qkv.begin() + L.qdim, m->q.begin());
          std::copy(m->qkv.begin() + L.qdim, m->qkv.begin() + L.qdim + L.kvdim, m->k.begin());
          std::copy(m->qkv.begin() + L.qdim + L.kvdim, m->qkv.begin() + L.qdim + 2 * L.kvdim, m->v.begin());
        } else {
          matvec(pool, L.q.type, L.q.data, L.q.n, L.q.k, m->norm.data(), m->q.data());
          matvec(pool, L.k.type, L.k.data, L.k.n, L.k.k, m->norm.data(), m->k.data());
          matvec(pool, L.v.type, L.v.data, L.v.n, L.v.k, m->norm.data(), m->v.data());
        }
        const float* qa;
        if (m->qk_norm) {
          qk_rope_store(m, L, pos, true, m->qn.data());
          qa = m->qn.data();
        } else {
          qk_rope_store(m, L, pos, false, m->q.data());  // in place on q
          qa = m->q.data();
        }
        attention(m, L, pos, qa, m->attn.data());
        matvec(pool, L.o.type, L.o.data, L.o.n, L.o.k, m->attn.data(), other);
        add_rms_norm(residual, other, L.post_norm.data(), m->norm.data(), H, m->norm_eps);
        std::swap(residual, other);
        matvec(pool, L.gate.type, L.gate.data, L.gate.n, L.gate.k, m->norm.data(), m->gate.data());
        matvec(pool, L.up.type, L.up.data, L.up.n, L.up.k, m->norm.data(), m->up.data());
        for (int i = 0; i < L.ffn; ++i) m->ff[i] = silu_mul(m->gate[i], m->up[i]);
        matvec(pool, L.down.type, L.down.data, L.down.n, L.down.k, m->ff.data(), other);
        for (int i = 0; i < H; ++i) other[i] = residual[i] + other[i];
        std::swap(residual, other);
      }
    }
    m->last_residual.assign(residual, residual + H);
    int32_t best = 0;
    if (need_logits) {
      rms_norm(residual, m->final_norm.data(), m->norm.data(), H, m->norm_eps);
      matvec(pool, m->lm_head.type, m->lm_head.data, (uint64_t)m->vocab, m->lm_head.k, m->norm.data(),
             m->logits.data());
      // ARGMAX_STAGE1 (:3645-3726) with the penalty list of argmax() (:1647-1665)
      const bool apply = s && s->repetition_penalty > 1 && n_penalized > 0;
      std::vector<int32_t> ids;
      if (apply) {
        const int64_t keep = std::min<int64_t>(n_penalized, m->ctx);
        ids.assign(penalized + (n_penalized - keep), penalized + n_penalized);
        std::sort(ids.begin(), ids.end());
      }
      const uint32_t milli = apply ? (uint32_t)std::floor((double)s->repetition_penalty * 1000 + 0.5) : 0;
      const float pen = (float)milli / 1000.0f;
      const int64_t groups = (m->vocab + 255) / 256;
      for (int64_t gidx = 0; gidx < groups; ++gidx) {
        float vals[256];
        uint32_t idx[256];
        for (int t = 0; t < 256; ++t) {
          const int64_t i = gidx * 256 + t;
          if (i < m->vocab) {
            float v = m->logits[i];
            if (!ids.empty() && std::binary_search(ids.begin(), ids.end(), (int32_t)i)) v = v > 0.0f ? v / pen : v * pen;
            vals[t] = v;
            idx[t] = (uint32_t)i;
          } else {
            vals[t] = kNegBig;
            idx[t] = 0xffffffffu;
          }
        }
        for (int st = 128; st >= 1; st >>= 1)
          for (int t = 0; t < st; ++t)
            if (better(vals[t + st], idx[t + st], vals[t], idx[t])) {
              vals[t] = vals[t + st];
              idx[t] = idx[t + st];
            }
        std::memcpy(m->candidates.data() + 8 * gidx, &vals[0], 4);
        std::memcpy(m->candidates.data() + 8 * gidx + 4, &idx[0], 4);
      }
      const bool sampling = s && (s->temperature > 0 || s->top_p < 1 || s->top_k > 0);
      if (sampling) {
        best = orc_sample_candidates(m->candidates.data(), groups, s, seen, n_seen, uniform);
      } else {
        // ARGMAX_STAGE2 (:3728-3791)
        float bv[256];
        uint32_t bi[256];
        for (int t = 0; t < 256; ++t) {
          float v = -3.402823e38f;
          uint32_t i = 0xffffffffu;
          for (int64_t g = t; g < groups; g += 256) {
            float cv;
            uint32_t ci;
            std::memcpy(&cv, m->candidates.data() + 8 * g, 4);
            std::memcpy(&ci, m->candidates.data() + 8 * g + 4, 4);
            if (better(cv, ci, v, i)) {
              v = cv;
              i = ci;
            }
          }
          bv[t] = v;
          bi[t] = i;
        }
        for (int st = 128; st >= 1; st >>= 1)
          for (int t = 0; t < st; ++t)
            if (better(bv[t + st], bi[t + st], bv[t], bi[t])) {
              bv[t] = bv[t + st];
              bi[t] = bi[t + st];
            }
        best = (int32_t)bi[0];
      }
    }
    m->pos += 1;
    *out_token = best;
    return 0;
  } catch (const std::exception& e) {
    if (err && err_len) std::snprintf(err, err_len, "%s", e.what());
    return -1;
  }
}

int orc_model_read(const orc_model* m, int which, void* out, int64_t n_bytes) {
  const void* src = nullptr;
  size_t bytes = 0;
  switch (which) {
    case 0: src = m->logits.data(); bytes = m->logits.size() * 4; break;
    case 1: src = m->last_residual.data(); bytes = m->last_residual.size() * 4; break;
    case 2: src = m->norm.data(); bytes = m->norm.size() * 4; break;
    case 3: src = m->candidates.data(); bytes = m->candidates.size(); break;
    case 4: src = (m->qk_norm ? m->qn : m->q).data(); bytes = m->q.size() * 4; break;
    case 5: src = m->attn.data(); bytes = m->attn.size() * 4; break;
    default: return -1;
  }
  if ((size_t)n_bytes < bytes) return -1;
  std::memcpy(out, src, bytes);
  return (int)bytes;
}

int orc_model_read_kv(const orc_model* m, int layer, int is_value, int pos, float* out) {
  if (layer < 0 || layer >= (int)m->layers.size() || pos < 0 || pos >= m->ctx) return -1;
  const Layer& L = m->layers[layer];
  const std::vector<float>& c = is_value ? L.vcache : L.kcache;
  for (int kh = 0; kh < L.kv_heads; ++kh)
    for (int d = 0; d < m->hd; ++d) out[kh * m->hd + d] = c[((size_t)kh * m->ctx + pos) * m->hd + d];
  return 0;
}

}  // extern "C"
