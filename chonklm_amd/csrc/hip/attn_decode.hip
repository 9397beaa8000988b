// Decode attention over the fp16 K/V cache for one new token (the reference's
// qkNormRopeStore + attention score/value passes, src/lib/llama-wgsl-runtime.ts
// :1467-1509, :1548-1570, WGSL :2868-3490), laid out for latency on gfx950.
//
// One workgroup per (kv head, chunk of 64 positions). A wave64 VALU
// instruction occupies its 16-lane SIMD for four cycles and the grid leaves
// about one workgroup per CU, so the kernel is laid out to keep each wave's
// instruction count after the loads small:
//   A  the position by a scalar load, then every load of the workgroup: K rows
//      (four lanes per position, HD/4 dims each) and V rows (wave w holds
//      dims [w*HD/4, (w+1)*HD/4) of all 64 positions, a lane 2 or 4 dims of
//      every PG-th position) into registers, q heads, new k/v and norm weights
//      into LDS, the rotary (cos, sin) of the position from the engine's table.
//   B  the G q heads, the new k and the new v are G + 2 items over the four
//      waves: RMSNorm and rotary into one shared q copy; k (normalised,
//      rotated) and v rounded to fp16 like the cache, stored by the newest
//      chunk.
//   C  scores by quads of lanes; the chunk maximum per head through LDS; the
//      weights exp(s - max) into LDS; weighted V from registers, each wave
//      summing its dims over the position groups in registers (no cross-wave
//      rescale).
//   D  the chunk's row [max, sum, acc] per head goes out as tagged words
//      {f32, u32 tag} (no wait), the new position's score is formed, then
//      every active chunk merges a slice of the output dims: it polls the
//      rows' (max, sum) words and its dims' acc words until all carry this
//      launch's tag (addresses formed once), forms exp(m_c - M) / L once per
//      (head, chunk), and writes one weighted sum per output element, the new
//      position joining as one more term. The chunks of a launch wait for
//      each other, so the engine uses this kernel only when its whole grid
//      fits on the device at once; every wait is also bounded in time
//      (DevState.error = 4 past the bound).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attn_dec_body.h"
#include "kernel_common.h"
#include "kernels.h"

namespace chonk {
namespace {

// One workgroup per (kv head blockIdx.x, chunk blockIdx.y); WALK: the workgroup
// walks a.sub sub-chunks (long contexts).
template <int G, int HD, bool WALK>
__global__ __launch_bounds__(kWg) void k_attn_dec(const AttnArgs a) {
  attn_dec_body<G, HD, WALK, false>(a, (int)blockIdx.x, (int)blockIdx.y);
}

}  // namespace

bool attn_dec_supported(int group, int hd, int ctx, int kv_f16) {
  // (registers: at head_dim 256 groups 7 and 8 spill to scratch in both variants,
  // group 6 in the one that walks sub-chunks, used past 128 chunks)
  const int chunks = (ctx + kDecChunk - 1) / kDecChunk;
  if (hd == 256 && group >= 6 && chunks > 128) return false;
  return kv_f16 && (hd == 64 || hd == 128 || hd == 256) && group >= 1 && group <= 8 && group * hd <= 1536 &&
         chunks <= 128 * kDecSubMax;
}

int attn_dec_sub(int ctx, int per_head) {
  const int cap = std::max(1, std::min(128, per_head));
  return ((ctx + kDecChunk - 1) / kDecChunk + cap - 1) / cap;
}

int attn_dec_chunk() { return kDecChunk; }

size_t attn_dec_shared_bytes(int group, int hd, int nchunk) {
  // q_s, qn [G][hd]; kx, vx, nq, nk [hd]; wmx [4][G], ew [G][64], hv [G][4]; cs [hd]
  (void)nchunk;
  const size_t g = (size_t)group;
  return sizeof(float) * (2 * g * hd + 5 * (size_t)hd + g * (4 + kDecChunk + 4));
}

namespace {
// cs[p][d] = (cos, sin) of the rotary angle p * inv[d], the expression the
// decode and prompt kernels evaluate inline.
__global__ __launch_bounds__(kWg) void k_rope_cs(const float* inv, int half, int ctx, float2* cs) {
  const int64_t i = (int64_t)blockIdx.x * kWg + threadIdx.x;
  if (i >= (int64_t)ctx * half) return;
  const int p = (int)(i / half), d = (int)(i % half);
  const float ang = __fmul_rn((float)p, inv[d]);
  cs[i] = make_float2(cosf(ang), sinf(ang));
}

template <int G, int HD>
const void* dec_fn(bool walk) {
  return walk ? (const void*)k_attn_dec<G, HD, true> : (const void*)k_attn_dec<G, HD, false>;
}
const void* dec_kernel(int group, int hd, bool walk) {
#define CHONK_DEC_FN(GG)                              \
  if (group == GG) {                                  \
    if (hd == 64) return dec_fn<GG, 64>(walk);        \
    if (hd == 128) return dec_fn<GG, 128>(walk);      \
    if (hd == 256) return dec_fn<GG, 256>(walk);      \
  }
  CHONK_DEC_FN(1)
  CHONK_DEC_FN(2)
  CHONK_DEC_FN(3)
  CHONK_DEC_FN(4)
  CHONK_DEC_FN(5)
  CHONK_DEC_FN(6)
  CHONK_DEC_FN(7)
  CHONK_DEC_FN(8)
#undef CHONK_DEC_FN
  return nullptr;
}
}  // namespace

int attn_dec_resident(int device, int group, int hd, size_t shmem, bool walk) {
  const void* f = dec_kernel(group, hd, walk);
  if (!f) return 0;
  // an instance that spills to scratch is not used (0: cannot run)
  hipFuncAttributes at{};
  if (hipFuncGetAttributes(&at, f) != hipSuccess || at.localSizeBytes != 0) return 0;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, kWg, shmem) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return per_cu * cus;
}

hipError_t launch_rope_cs(const float* inv, int half, int ctx, float2* cs, hipStream_t s) {
  const int64_t n = (int64_t)ctx * half;
  hipLaunchKernelGGL(k_rope_cs, dim3((unsigned)((n + kWg - 1) / kWg)), dim3(kWg), 0, s, inv, half, ctx, cs);
  return hipGetLastError();
}

hipError_t launch_attn_dec(const AttnArgs& a, size_t shmem, hipStream_t s) {
  const int group = a.heads / a.kv_heads;
  const dim3 grid(a.kv_heads, a.nchunk);
#define CHONK_DEC_CASE(GG, HH) \
  if (group == GG && a.hd == HH) {                                                                 \
    if (a.sub > 1)                                                                                 \
      hipLaunchKernelGGL((k_attn_dec<GG, HH, true>), grid, dim3(kWg), shmem, s, a);                 \
    else                                                                                           \
      hipLaunchKernelGGL((k_attn_dec<GG, HH, false>), grid, dim3(kWg), shmem, s, a);                \
    return hipGetLastError();                                                                      \
  }
#define CHONK_DEC_G(GG) CHONK_DEC_CASE(GG, 64) CHONK_DEC_CASE(GG, 128) CHONK_DEC_CASE(GG, 256)
  CHONK_DEC_G(1)
  CHONK_DEC_G(2)
  CHONK_DEC_G(3)
  CHONK_DEC_G(4)
  CHONK_DEC_G(5)
  CHONK_DEC_G(6)
  CHONK_DEC_G(7)
  CHONK_DEC_G(8)
#undef CHONK_DEC_G
#undef CHONK_DEC_CASE
  return hipErrorInvalidValue;
}

}  // namespace chonk
