// GGML tensor type table and IEEE half-precision conversion shared by the
// GGUF reader/writer, the quantizers and the weight repacker.
//
// Type ids and block geometry follow src/lib/gguf.ts:5-14 and :103-130 of the
// reference (which in turn follow the GGUF specification / ggml.h).
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace chonk {

enum GgmlType : uint32_t {
  GGML_F32 = 0,
  GGML_F16 = 1,
  GGML_Q5_0 = 6,
  GGML_Q5_1 = 7,
  GGML_Q8_0 = 8,
  GGML_Q4_K = 12,
  GGML_Q5_K = 13,
  GGML_Q6_K = 14,
};

struct TypeTraits {
  uint32_t block_elems;  // elements per block
  uint32_t block_bytes;  // bytes per block
  bool quantized;
  const char* name;
};

// Returns false for types the decode path does not support.
inline bool type_traits(uint32_t type, TypeTraits* out) {
  switch (type) {
    case GGML_F32: *out = {1, 4, false, "F32"}; return true;
    case GGML_F16: *out = {1, 2, false, "F16"}; return true;
    case GGML_Q5_0: *out = {32, 22, true, "Q5_0"}; return true;
    case GGML_Q5_1: *out = {32, 24, true, "Q5_1"}; return true;
    case GGML_Q8_0: *out = {32, 34, true, "Q8_0"}; return true;
    case GGML_Q4_K: *out = {256, 144, true, "Q4_K"}; return true;
    case GGML_Q5_K: *out = {256, 176, true, "Q5_K"}; return true;
    case GGML_Q6_K: *out = {256, 210, true, "Q6_K"}; return true;
    default: return false;
  }
}

inline std::string type_name(uint32_t type) {
  TypeTraits t;
  if (type_traits(type, &t)) return t.name;
  return "type-" + std::to_string(type);
}

// Byte length of a tensor of n elements; mirrors ggmlTensorByteLength
// (src/lib/gguf.ts:103-130), including its error messages.
inline uint64_t tensor_byte_length(uint32_t type, uint64_t n_elements) {
  TypeTraits t;
  if (!type_traits(type, &t)) {
    throw std::runtime_error("unsupported GGML tensor type " + std::to_string(type));
  }
  if (n_elements % t.block_elems != 0) {
    throw std::runtime_error("GGML tensor type " + std::to_string(type) + " requires " +
                             std::to_string(t.block_elems) + "-element blocks, got " +
                             std::to_string(n_elements));
  }
  return n_elements / t.block_elems * t.block_bytes;
}

// Exact binary16 -> binary32 (every half value is representable).
inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      // subnormal: normalise the mantissa
      int e = -1;
      uint32_t m = man;
      do {
        m <<= 1;
        ++e;
      } while ((m & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + (127 - 15)) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// binary32 -> binary16 with round-to-nearest-even (IEEE default), the same
// rounding ggml's FP32_TO_FP16 performs.
inline uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {  // inf / nan
    return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0));
  }
  const int e = (int)exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);  // overflow -> inf
  if (e <= 0) {
    // subnormal half (or zero)
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e;  // 14..24
    uint32_t half_man = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half_man & 1u))) ++half_man;
    return (uint16_t)(sign | half_man);
  }
  uint32_t half = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half;  // may carry into exp: correct
  return (uint16_t)half;
}

}  // namespace chonk
