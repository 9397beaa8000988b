// Reference (non-imatrix) GGUF block quantizers used to build synthetic
// models: Q8_0, Q5_0, Q5_1, Q4_K, Q5_K and Q6_K.
//
// These restate the published algorithm of llama.cpp's ggml-quants.c
// (quantize_row_*_ref, make_qkx2_quants, make_qx_quants, nearest_int) in code
// of our own. llama.cpp is not a dependency of the reference and is not in
// this image; the reference only *decodes* these blocks
// (src/lib/llama-wgsl-runtime.ts:2202-2613). The block byte layouts written
// here are the ones that decoder reads.
#include "quantize.h"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "ggml_types.h"

namespace chonk {
namespace {

constexpr float kGroupMaxEps = 1e-15f;

// Round-half-to-even via the 1.5*2^23 magic constant (valid for |x| < 2^22).
inline int nearest_int(float fval) {
  float val = fval + 12582912.f;
  int i;
  std::memcpy(&i, &val, 4);
  return (i & 0x007fffff) - 0x00400000;
}

// Affine (scale, min) fit of n values to [0, nmax] with weighted least
// squares refinement over nstep candidate scales.
float fit_scale_min(int n, int nmax, const float* x, const float* weights, uint8_t* L,
                    float* the_min, uint8_t* Laux, float rmin, float rdelta, int nstep) {
  float min = x[0], max = x[0];
  float sum_w = weights[0];
  float sum_x = sum_w * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < min) min = x[i];
    if (x[i] > max) max = x[i];
    const float w = weights[i];
    sum_w += w;
    sum_x += w * x[i];
  }
  if (min > 0) min = 0;
  if (max == min) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -min;
    return 0.f;
  }
  float iscale = nmax / (max - min);
  float scale = 1 / iscale;
  float best_err = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * (x[i] - min));
    L[i] = (uint8_t)std::max(0, std::min(nmax, l));
    float diff = scale * L[i] + min - x[i];
    best_err += weights[i] * (diff * diff);
  }
  if (nstep < 1) {
    *the_min = -min;
    return scale;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (max - min);
    float sum_l = 0, sum_l2 = 0, sum_xl = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - min));
      l = std::max(0, std::min(nmax, l));
      Laux[i] = (uint8_t)l;
      const float w = weights[i];
      sum_l += w * l;
      sum_l2 += w * l * l;
      sum_xl += w * l * x[i];
    }
    const float D = sum_w * sum_l2 - sum_l * sum_l;
    if (D > 0) {
      float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
      float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
      if (this_min > 0) {
        this_min = 0;
        this_scale = sum_xl / sum_l2;
      }
      float err = 0;
      for (int i = 0; i < n; ++i) {
        float diff = this_scale * Laux[i] + this_min - x[i];
        err += weights[i] * (diff * diff);
      }
      if (err < best_err) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best_err = err;
        scale = this_scale;
        min = this_min;
      }
    }
  }
  *the_min = -min;
  return scale;
}

// Symmetric fit of n values to [-nmax, nmax-1] with weights x^2 (the
// "rmse_type 1" search over 19 candidate scales).
float fit_symmetric(int n, int nmax, const float* x, int8_t* L) {
  float max = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    const float ax = std::fabs(x[i]);
    if (ax > amax) {
      amax = ax;
      max = x[i];
    }
  }
  if (amax < kGroupMaxEps) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / max;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = std::max(-nmax, std::min(nmax - 1, l));
    L[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / max;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * x[i]);
      l = std::max(-nmax, std::min(nmax - 1, l));
      const float w = x[i] * x[i];
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        L[i] = (int8_t)(nmax + std::max(-nmax, std::min(nmax - 1, l)));
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

inline void put_f16(uint8_t* p, float v) {
  const uint16_t h = f32_to_f16(v);
  std::memcpy(p, &h, 2);
}
inline float get_f16(const uint8_t* p) {
  uint16_t h;
  std::memcpy(&h, p, 2);
  return f16_to_f32(h);
}

void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
  }
}

// ---- per-type block quantizers -------------------------------------------------

void quant_q8_0(const float* x, uint8_t* y, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b, x += 32, y += 34) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / ((1 << 7) - 1);
    const float id = d ? 1.0f / d : 0.0f;
    put_f16(y, d);
    for (int j = 0; j < 32; ++j) y[2 + j] = (uint8_t)(int8_t)std::roundf(x[j] * id);
  }
}

void quant_q5_0(const float* x, uint8_t* y, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b, x += 32, y += 22) {
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; ++j) {
      if (amax < std::fabs(x[j])) {
        amax = std::fabs(x[j]);
        max = x[j];
      }
    }
    const float d = max / -16;
    const float id = d ? 1.0f / d : 0.0f;
    put_f16(y, d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
      const float x0 = x[j] * id;
      const float x1 = x[16 + j] * id;
      const uint8_t xi0 = (uint8_t)std::min(31, (int)(int8_t)(x0 + 16.5f));
      const uint8_t xi1 = (uint8_t)std::min(31, (int)(int8_t)(x1 + 16.5f));
      y[6 + j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
      qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
      qh |= ((xi1 & 0x10u) >> 4) << (j + 16);
    }
    std::memcpy(y + 2, &qh, 4);
  }
}

void quant_q5_1(const float* x, uint8_t* y, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b, x += 32, y += 24) {
    float min = x[0], max = x[0];
    for (int j = 1; j < 32; ++j) {
      min = std::min(min, x[j]);
      max = std::max(max, x[j]);
    }
    const float d = (max - min) / ((1 << 5) - 1);
    const float id = d ? 1.0f / d : 0.0f;
    put_f16(y, d);
    put_f16(y + 2, min);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
      const float x0 = (x[j] - min) * id;
      const float x1 = (x[16 + j] - min) * id;
      const uint8_t xi0 = (uint8_t)(x0 + 0.5f);
      const uint8_t xi1 = (uint8_t)(x1 + 0.5f);
      y[8 + j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
      qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
      qh |= ((xi1 & 0x10u) >> 4) << (j + 16);
    }
    std::memcpy(y + 4, &qh, 4);
  }
}

void quant_q4_k(const float* x, uint8_t* y, int64_t nblocks) {
  uint8_t L[256], Laux[32];
  float weights[32], mins[8], scales[8];
  for (int64_t b = 0; b < nblocks; ++b, x += 256, y += 144) {
    uint8_t* sc = y + 4;
    uint8_t* qs = y + 16;
    std::memset(y, 0, 144);
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
      float sum_x2 = 0;
      for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
      const float av_x = std::sqrt(sum_x2 / 32);
      for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
      scales[j] = fit_scale_min(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < 8; ++j) {
      uint8_t ls = (uint8_t)std::min(63, nearest_int(inv_scale * scales[j]));
      uint8_t lm = (uint8_t)std::min(63, nearest_int(inv_min * mins[j]));
      if (j < 4) {
        sc[j] = ls;
        sc[j + 4] = lm;
      } else {
        sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
        sc[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    put_f16(y, max_scale / 63.f);
    put_f16(y + 2, max_min / 63.f);
    const float dd = get_f16(y), dmn = get_f16(y + 2);
    for (int j = 0; j < 8; ++j) {
      uint8_t s, m;
      scale_min_k4(j, sc, &s, &m);
      const float d = dd * s;
      if (!d) continue;
      const float dm = dmn * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = nearest_int((x[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)std::max(0, std::min(15, l));
      }
    }
    for (int j = 0; j < 256; j += 64) {
      for (int l = 0; l < 32; ++l) qs[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
      qs += 32;
    }
  }
}

// Q5_K: Q4_K's super-block with 5-bit values (0..31), the fifth bits in
// qh[32]: value 32n + j of the 64-value group n sets bit 2n of qh[j], value
// 32n + 32 + j bit 2n + 1; block d, dmin, scales[12], qh[32], qs[128].
void quant_q5_k(const float* x, uint8_t* y, int64_t nblocks) {
  uint8_t L[256], Laux[32];
  float weights[32], mins[8], scales[8];
  for (int64_t b = 0; b < nblocks; ++b, x += 256, y += 176) {
    uint8_t* sc = y + 4;
    uint8_t* qh = y + 16;
    uint8_t* qs = y + 48;
    std::memset(y, 0, 176);
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
      float sum_x2 = 0;
      for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
      const float av_x = std::sqrt(sum_x2 / 32);
      for (int l = 0; l < 32; ++l) weights[l] = av_x + std::fabs(x[32 * j + l]);
      scales[j] = fit_scale_min(32, 31, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < 8; ++j) {
      uint8_t ls = (uint8_t)std::min(63, nearest_int(inv_scale * scales[j]));
      uint8_t lm = (uint8_t)std::min(63, nearest_int(inv_min * mins[j]));
      if (j < 4) {
        sc[j] = ls;
        sc[j + 4] = lm;
      } else {
        sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
        sc[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    put_f16(y, max_scale / 63.f);
    put_f16(y + 2, max_min / 63.f);
    const float dd = get_f16(y), dmn = get_f16(y + 2);
    for (int j = 0; j < 8; ++j) {
      uint8_t s, m;
      scale_min_k4(j, sc, &s, &m);
      const float d = dd * s;
      if (!d) continue;
      const float dm = dmn * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = nearest_int((x[32 * j + ii] + dm) / d);
        L[32 * j + ii] = (uint8_t)std::max(0, std::min(31, l));
      }
    }
    for (int n = 0; n < 4; ++n) {
      for (int j = 0; j < 32; ++j) {
        int l1 = L[64 * n + j], l2 = L[64 * n + j + 32];
        if (l1 > 15) {
          l1 -= 16;
          qh[j] |= (uint8_t)(1u << (2 * n));
        }
        if (l2 > 15) {
          l2 -= 16;
          qh[j] |= (uint8_t)(2u << (2 * n));
        }
        qs[32 * n + j] = (uint8_t)(l1 | (l2 << 4));
      }
    }
  }
}

void quant_q6_k(const float* x, uint8_t* y, int64_t nblocks) {
  int8_t L[256];
  float scales[16];
  for (int64_t b = 0; b < nblocks; ++b, x += 256, y += 210) {
    uint8_t* ql = y;
    uint8_t* qh = y + 128;
    int8_t* sc = (int8_t*)(y + 192);
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < 16; ++ib) {
      const float scale = fit_symmetric(16, 32, x + 16 * ib, L + 16 * ib);
      scales[ib] = scale;
      const float abs_scale = std::fabs(scale);
      if (abs_scale > max_abs_scale) {
        max_abs_scale = abs_scale;
        max_scale = scale;
      }
    }
    if (max_abs_scale < kGroupMaxEps) {
      std::memset(y, 0, 210);
      continue;
    }
    const float iscale = -128.f / max_scale;
    put_f16(y + 208, 1 / iscale);
    for (int ib = 0; ib < 16; ++ib) sc[ib] = (int8_t)std::min(127, nearest_int(iscale * scales[ib]));
    const float dd = get_f16(y + 208);
    for (int j = 0; j < 16; ++j) {
      const float d = dd * sc[j];
      if (!d) continue;
      for (int ii = 0; ii < 16; ++ii) {
        int l = nearest_int(x[16 * j + ii] / d);
        l = std::max(-32, std::min(31, l));
        L[16 * j + ii] = (int8_t)(l + 32);
      }
    }
    for (int j = 0; j < 256; j += 128) {
      for (int l = 0; l < 32; ++l) {
        const uint8_t q1 = L[j + l + 0] & 0xF;
        const uint8_t q2 = L[j + l + 32] & 0xF;
        const uint8_t q3 = L[j + l + 64] & 0xF;
        const uint8_t q4 = L[j + l + 96] & 0xF;
        ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
        ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
        qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                          ((L[j + l + 96] >> 4) << 6));
      }
      ql += 64;
      qh += 32;
    }
  }
}

}  // namespace

bool quantize_rows(uint32_t type, const float* src, uint8_t* dst, int64_t n_elements) {
  TypeTraits t;
  if (!type_traits(type, &t) || n_elements % t.block_elems != 0) return false;
  const int64_t nb = n_elements / t.block_elems;
  switch (type) {
    case GGML_F32: std::memcpy(dst, src, (size_t)n_elements * 4); return true;
    case GGML_F16:
      for (int64_t i = 0; i < n_elements; ++i) {
        const uint16_t h = f32_to_f16(src[i]);
        std::memcpy(dst + 2 * i, &h, 2);
      }
      return true;
    case GGML_Q8_0: quant_q8_0(src, dst, nb); return true;
    case GGML_Q5_0: quant_q5_0(src, dst, nb); return true;
    case GGML_Q5_1: quant_q5_1(src, dst, nb); return true;
    case GGML_Q4_K: quant_q4_k(src, dst, nb); return true;
    case GGML_Q5_K: quant_q5_k(src, dst, nb); return true;
    case GGML_Q6_K: quant_q6_k(src, dst, nb); return true;
    default: return false;  // Q5_K: decode-only here
  }
}

}  // namespace chonk
