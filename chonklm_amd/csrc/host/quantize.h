// Reference GGUF block quantizers (Q8_0, Q5_0, Q5_1, Q4_K, Q6_K, plus F32/F16
// pass-through) used by the synthetic-model writer.
#pragma once

#include <cstdint>

namespace chonk {

// Quantizes n_elements consecutive floats (a multiple of the type's block
// size) into GGUF blocks at dst. Returns false for unsupported types/sizes.
bool quantize_rows(uint32_t type, const float* src, uint8_t* dst, int64_t n_elements);

}  // namespace chonk
