// qk_prep: fused head transpose + QK-RMSNorm + multi-axis RoPE for gfx950.
//
// Semantics follow the reference tile body (src/flicker/kernels.py:35-53) per (b, t, h):
//   x  = f32(qkv[b, t, sec*H*D + h*D : ... + D])                    sec = 0 (q), 1 (k), 2 (v)
//   ms = mean(x*x);  n = bf16(x * (1/sqrt(ms + 1e-6)))
//   y  = f32(bf16(n * scale))            (bf16 scale; a float32 scale keeps the f32 product)
//   r[2j]   = cos[t,2j]   * y[2j]   + sin[t,2j]   * y[2j+1]
//   r[2j+1] = cos[t,2j+1] * y[2j+1] + sin[t,2j+1] * y[2j]
//   out = bf16(gain * r) for q, bf16(r) for k;  v is copied bit for bit
// and the output is written head-major, (b, h, t, :), which is the transpose the
// reference performs with its output index map (kernels.py:81).
//
// Mapping: one head row of 128 bf16 = 256 bytes is held by 16 lanes, 8 elements
// (one 128-bit load) per lane, so the RMS reduction is a 16-lane DPP butterfly and
// each RoPE pair (2j, 2j+1) stays inside one lane.  A 256-thread block holds 16
// consecutive tokens; the 4 groups of a wave therefore write 4 consecutive tokens of
// the same head = 1 KiB contiguous per store instruction.  Each group handles
// kHeads heads of its token, issuing all 3*kHeads loads (nontemporal: the activation is
// read once) before any math, and keeps the token's cos/sin lanes in registers across
// those heads.
//
// The kernel is HBM-bound: per (b, t, h) it moves 3*256 bytes in and 3*256 out.

#include "qk_math.h"

namespace {

constexpr int kHeadDim = 128;
constexpr int kLanesPerRow = 16;
constexpr int kThreads = 256;
constexpr int kTokensPerBlock = kThreads / kLanesPerRow;

// Cache policy of the streaming accesses (bit 0: QKV loads, bit 1: Q/K/V stores) and a
// forced heads-per-group (0 = automatic); compile-time knobs for tuning sweeps.  The QKV
// activation is read exactly once, so its loads are nontemporal: measured at the 1024^2
// Klein shape this lifts the pass from ~4.5 to ~6.0 TB/s, the store stream and the
// cos/sin tables (re-read by every head group) keep the default policy.
#ifndef FLK_QK_NT
#define FLK_QK_NT 1
#endif
#ifndef FLK_QK_HPG
#define FLK_QK_HPG 0
#endif

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  if constexpr (FLK_QK_NT & 1) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ void store16(uint16_t* p, uint4 v) {
  if constexpr (FLK_QK_NT & 2) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = v;
  }
}

template <bool kScaleF32, bool kGain, int kHeads>
__global__ __launch_bounds__(kThreads) void qk_prep_kernel(
    const uint16_t* __restrict__ qkv, int64_t batch_stride, int64_t row_stride,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int64_t table_stride,
    const void* __restrict__ q_scale, const void* __restrict__ k_scale, float q_gain,
    int length, int num_heads, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, int64_t out_length, int64_t out_offset) {
  const int lane = threadIdx.x & (kLanesPerRow - 1);
  const int t = blockIdx.x * kTokensPerBlock + (threadIdx.x >> 4);
  if (t >= length) return;  // whole 16-lane rows exit together, so DPP rows stay intact
  const int h0 = blockIdx.y * kHeads;
  const int b = blockIdx.z;

  const uint16_t* row = qkv + (int64_t)b * batch_stride + (int64_t)t * row_stride + lane * 8;
  uint4 rq[kHeads], rk[kHeads], rv[kHeads];
#pragma unroll
  for (int i = 0; i < kHeads; ++i) {
    rq[i] = load16(row + (int64_t)(h0 + i) * kHeadDim);
    rk[i] = load16(row + (int64_t)(num_heads + h0 + i) * kHeadDim);
    rv[i] = load16(row + (int64_t)(2 * num_heads + h0 + i) * kHeadDim);
  }
  float c[8], s[8], qs[8], ks[8];
  flk::load_table8(cos_t + (int64_t)t * table_stride, lane, c);
  flk::load_table8(sin_t + (int64_t)t * table_stride, lane, s);
  flk::load_scale8<kScaleF32>(q_scale, lane, qs);
  flk::load_scale8<kScaleF32>(k_scale, lane, ks);

#pragma unroll
  for (int i = 0; i < kHeads; ++i) {
    const int64_t o =
        (((int64_t)b * num_heads + h0 + i) * out_length + out_offset + t) * kHeadDim + lane * 8;
    store16(q_out + o, flk::norm_rotate<kScaleF32, kGain>(rq[i], qs, c, s, q_gain));
    store16(k_out + o, flk::norm_rotate<kScaleF32, false>(rk[i], ks, c, s, 1.0f));
    store16(v_out + o, rv[i]);
  }
}

template <bool kScaleF32, bool kGain>
int launch(int heads_per_group, dim3 grid, hipStream_t stream, const uint16_t* qkv,
           int64_t bs, int64_t rs, const float* cos_t, const float* sin_t, int64_t ts,
           const void* qsc, const void* ksc, float gain, int length, int num_heads,
           uint16_t* q, uint16_t* k, uint16_t* v, int64_t out_len, int64_t out_off) {
#define FLK_QK_LAUNCH(NH)                                                                    \
  hipLaunchKernelGGL((qk_prep_kernel<kScaleF32, kGain, NH>), grid, dim3(kThreads), 0, stream, \
                     qkv, bs, rs, cos_t, sin_t, ts, qsc, ksc, gain, length, num_heads, q, k, v, \
                     out_len, out_off)
  switch (heads_per_group) {
    case 6: FLK_QK_LAUNCH(6); break;
    case 4: FLK_QK_LAUNCH(4); break;
    case 3: FLK_QK_LAUNCH(3); break;
    case 2: FLK_QK_LAUNCH(2); break;
    default: FLK_QK_LAUNCH(1); break;
  }
#undef FLK_QK_LAUNCH
  return flk_launch_status();
}

}  // namespace

extern "C" int flk_qk_prep(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                           const float* cos, const float* sin, int64_t table_row_stride,
                           const void* q_scale, const void* k_scale, int scale_is_f32,
                           float q_gain, int batch, int length, int num_heads, int head_dim,
                           void* q_out, void* k_out, void* v_out, int64_t out_length,
                           int64_t out_offset, void* stream) {
  if (head_dim != kHeadDim) return FLK_E_UNSUPPORTED;
  if (batch < 0 || length < 0 || num_heads <= 0 || out_offset < 0 ||
      out_offset + length > out_length)
    return FLK_E_INVALID;
  if (batch == 0 || length == 0) return FLK_OK;
  if (qkv_row_stride < 3LL * num_heads * head_dim || table_row_stride < head_dim ||
      (batch > 1 && qkv_batch_stride < (int64_t)(length - 1) * qkv_row_stride + 3LL * num_heads * head_dim))
    return FLK_E_INVALID;
  if (!qkv || !cos || !sin || !q_scale || !k_scale || !q_out || !k_out || !v_out)
    return FLK_E_INVALID;
  if (qkv_row_stride % 8 || qkv_batch_stride % 8 || table_row_stride % 4 ||
      !flk_host_aligned(qkv, 16) || !flk_host_aligned(cos, 16) || !flk_host_aligned(sin, 16) ||
      !flk_host_aligned(q_scale, 16) || !flk_host_aligned(k_scale, 16) ||
      !flk_host_aligned(q_out, 16) || !flk_host_aligned(k_out, 16) || !flk_host_aligned(v_out, 16))
    return FLK_E_ALIGN;

  // Two heads per 16-lane group measured best at the Klein shapes (6 loads in flight per lane
  // and 2x more blocks than four heads per group).
  int hpg = (num_heads % 2 == 0) ? 2 : (num_heads % 3 == 0) ? 3 : 1;
  if (FLK_QK_HPG > 0 && num_heads % FLK_QK_HPG == 0) hpg = FLK_QK_HPG;
  const dim3 grid((length + kTokensPerBlock - 1) / kTokensPerBlock, num_heads / hpg, batch);
  const bool gain = q_gain != 1.0f;
  auto* s = static_cast<hipStream_t>(stream);
  auto* in = static_cast<const uint16_t*>(qkv);
  auto* q = static_cast<uint16_t*>(q_out);
  auto* k = static_cast<uint16_t*>(k_out);
  auto* v = static_cast<uint16_t*>(v_out);
  if (scale_is_f32) {
    return gain ? launch<true, true>(hpg, grid, s, in, qkv_batch_stride, qkv_row_stride, cos, sin,
                                     table_row_stride, q_scale, k_scale, q_gain, length, num_heads,
                                     q, k, v, out_length, out_offset)
                : launch<true, false>(hpg, grid, s, in, qkv_batch_stride, qkv_row_stride, cos, sin,
                                      table_row_stride, q_scale, k_scale, q_gain, length, num_heads,
                                      q, k, v, out_length, out_offset);
  }
  return gain ? launch<false, true>(hpg, grid, s, in, qkv_batch_stride, qkv_row_stride, cos, sin,
                                    table_row_stride, q_scale, k_scale, q_gain, length, num_heads,
                                    q, k, v, out_length, out_offset)
              : launch<false, false>(hpg, grid, s, in, qkv_batch_stride, qkv_row_stride, cos, sin,
                                     table_row_stride, q_scale, k_scale, q_gain, length, num_heads,
                                     q, k, v, out_length, out_offset);
}
