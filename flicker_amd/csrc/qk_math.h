// Per-row arithmetic of qk_prep (src/flicker/kernels.py:35-53), shared by the qk_prep kernel
// and the int8 projection's fused epilogue so that both round at exactly the same points.
//
// One 128-wide head row is held by a 16-lane DPP row, 8 elements per lane (lane l owns
// elements 8l .. 8l+7); the mean of squares is a 16-lane butterfly and each RoPE pair
// (2j, 2j+1) stays inside one lane.
#pragma once

#include "common.h"

namespace flk {

constexpr int kQkHeadDim = 128;

template <bool kScaleF32>
__device__ __forceinline__ void load_scale8(const void* scale, int lane, float out[8]) {
  if constexpr (kScaleF32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(scale) + lane * 8);
    float4 a = p[0], b = p[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(scale) + lane * 8);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = flk::bf16_lo(ws[i]);
      out[2 * i + 1] = flk::bf16_hi(ws[i]);
    }
  }
}

__device__ __forceinline__ void load_table8(const float* row, int lane, float out[8]) {
  const float4* p = reinterpret_cast<const float4*>(row + lane * 8);
  float4 a = p[0], b = p[1];
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// RMSNorm * scale and the RoPE rotation of the 8 elements this lane holds, in float32:
// r = cos * y + sin * swap(y) with y = bf16(x * (1 / sqrt(mean x^2 + eps))) * scale, the
// product rounded to bf16 for a bf16 scale and kept in float32 for a float32 one.
template <bool kScaleF32>
__device__ __forceinline__ void norm_rotate_f32(uint4 raw, const float sc[8], const float c[8],
                                                const float s[8], float r[8]) {
#pragma clang fp contract(off)
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = flk::bf16_lo(w[i]);
    x[2 * i + 1] = flk::bf16_hi(w[i]);
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  ss = flk::row16_sum(ss);
  const float ms = ss * (1.0f / kQkHeadDim);
  const float inv = 1.0f / sqrtf(ms + 1e-6f);
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float n = flk::round_bf16(x[i] * inv);
    y[i] = kScaleF32 ? n * sc[i] : flk::round_bf16(n * sc[i]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[2 * j] = c[2 * j] * y[2 * j] + s[2 * j] * y[2 * j + 1];
    r[2 * j + 1] = c[2 * j + 1] * y[2 * j + 1] + s[2 * j + 1] * y[2 * j];
  }
}

// RMSNorm * scale, RoPE rotation and optional gain on the 8 elements this lane holds,
// rounded to bf16 once at the end.
template <bool kScaleF32, bool kGain>
__device__ __forceinline__ uint4 norm_rotate(uint4 raw, const float sc[8], const float c[8],
                                             const float s[8], float gain) {
#pragma clang fp contract(off)
  float r[8];
  norm_rotate_f32<kScaleF32>(raw, sc, c, s, r);
  if constexpr (kGain) {
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = gain * r[i];
  }
  return make_uint4(flk::pack_bf16x2(r[0], r[1]), flk::pack_bf16x2(r[2], r[3]),
                    flk::pack_bf16x2(r[4], r[5]), flk::pack_bf16x2(r[6], r[7]));
}

}  // namespace flk
