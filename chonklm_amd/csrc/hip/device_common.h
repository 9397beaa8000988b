// Device-side data layouts shared by the kernels and the engine.
//
// Quantized matrices are stored as "stripes": the GGUF block fields of a
// [N][K] matrix split into separately packed streams, so that a lane's
// 32-element unit is one or two aligned vector loads. The bytes per matrix are
// exactly the GGUF bytes (no padding inside a row). Row r's share of stream s
// starts at s + r * row_stride(s).
//
//   type   unit (32 elements) reads                 streams
//   Q4_K   16 B qs + 16 B superblock header         s0 qs[K/2]   s1 hdr[K/256][16] (d, dmin, scales[12])
//   Q5_K   16 B qs + 16 B header + 16 B qh          s0 qs[K/2]   s1 hdr[K/256][16]  s2 qh[K/256][32]
//   Q6_K   8+8 B ql + 8 B qh + 4 scales + d         s0 ql[K/2]   s1 qh[K/4]  s2 sc[K/16] (int8)  s3 d[K/256] (f16)
//   Q8_0   32 B qs + d                              s0 qs[K]     s1 d[K/32] (f16)
//   Q5_0   16 B qs + 4 B qh + d                     s0 qs[K/2]   s1 qh[K/32] (u32)  s2 d[K/32] (f16)
//   Q5_1   16 B qs + 4 B qh + d + m                 s0 qs[K/2]   s1 qh[K/32]  s2 d[K/32]  s3 m[K/32]
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chonk {

enum : int32_t {
  QT_Q5_0 = 6,
  QT_Q5_1 = 7,
  QT_Q8_0 = 8,
  QT_Q4_K = 12,
  QT_Q5_K = 13,
  QT_Q6_K = 14,
};

struct QMat {
  const uint8_t* s0;
  const uint8_t* s1;
  const uint8_t* s2;
  const uint8_t* s3;
  int32_t type;
  int32_t n;  // rows
  int32_t k;  // row length (multiple of 32; of 256 for K-quants)
  int32_t pad;
};

// Mutable per-engine state the step graph reads; the host writes it only
// between graph launches.
struct DevState {
  int32_t pos;            // positions already in the K/V cache
  int32_t stopped;        // device-driven generation finished: kernels return at entry
  int32_t generating;     // 1: select appends to gen[] and checks EOS / budget
  int32_t n_generated;
  int32_t max_generated;
  int32_t error;          // 1: a kernel saw pos >= context; 2: token id out of range; 4: the decode attention's
                          // chunk rows, 5: the fused launch's q|k|v rows did not arrive within the wait bound
  int32_t last_token;     // token selected by the last logits step
  int32_t pad;
};

// Sampling parameters of the select kernel (device copy of chonk_sampling).
struct DevSampling {
  double temperature;
  double top_p;
  double repetition_penalty;  // host-style second penalty factor, max(rp, 1e-6)
  uint64_t seed;
  int32_t top_k;
  int32_t sample_mode;     // 0 greedy argmax, 1 candidate sampler
  int32_t stage1_penalty;  // 1: divide/multiply logits of penalized ids (GPU stage 1)
  float stage1_pen;        // f32(round(rp*1000)) / 1000
  int32_t seen_penalty;    // 1: second penalty over seen ids in the sampler
  int32_t n_eos;
  int32_t eos[16];
};

constexpr int kWg = 256;  // threads per workgroup for every kernel here

// Global-memory view of a pointer. A load through a generic pointer is a FLAT
// instruction, which also counts as an LDS access: every later wait for LDS
// data then waits for the outstanding memory loads too. Pointers read from
// device-memory tables are generic unless cast.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gbl(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gblw(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}
// Load of a workgroup-uniform address through the scalar data cache, for data
// that nothing writes while the kernel runs (row tables, page tables). Scalar
// loads have their own counter, so waiting for one never waits for the vector
// loads in flight. (A non-uniform address falls back to a vector load.)
template <class T>
__device__ __forceinline__ T ld_scalar(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
// 16 / 8 / 4-byte global loads (HIP's uint4 / uint2 cannot be assigned from
// an address-space-qualified object, so the load goes through clang vectors)
__device__ __forceinline__ uint4 ldg4(const void* p) {
  const u32x4_t v = *gbl((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg2(const void* p) {
  const u32x2_t v = *gbl((const u32x2_t*)p);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ldg1(const void* p) { return *gbl((const uint32_t*)p); }
__device__ __forceinline__ float4 ldg4f(const float* p) {
  const uint4 v = ldg4(p);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// Group candidate written by the lm_head epilogue (ARGMAX_STAGE1 output).
struct Candidate {
  float value;
  uint32_t index;
};

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

}  // namespace chonk
