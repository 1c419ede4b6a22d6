// RoPE tables on the GPU: rope.embed_nd (src/flicker/rope.py:9-21), kernels.lane_pair
// (src/flicker/kernels.py:28-31) and the two fused.  The angle arithmetic lives in
// rope_math.h.  Each thread produces one (token, pair) entry; the tables are built once
// per forward, not per block.

#include "rope_math.h"

namespace {

using flk::Axes;
constexpr int kThreads = 256;

__device__ __forceinline__ void angle_of(const float* __restrict__ ids, int64_t stride,
                                         int64_t t, int pair, const Axes& ax, float theta,
                                         float& c, float& s) {
  int a;
  const float omega = flk::pair_omega(pair, ax, theta, a);
  flk::pair_cos_sin(ids[t * stride + a], omega, c, s);
}

__global__ __launch_bounds__(kThreads) void rope_embed_kernel(const float* __restrict__ ids,
                                                              int64_t stride, int64_t length,
                                                              Axes ax, float theta,
                                                              float* __restrict__ pe) {
  const int pairs = ax.first_pair[ax.count];
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= length * pairs) return;
  const int64_t t = idx / pairs;
  const int pair = (int)(idx - t * pairs);
  float c, s;
  angle_of(ids, stride, t, pair, ax, theta, c, s);
  reinterpret_cast<float4*>(pe)[idx] = make_float4(c, -s, s, c);
}

__global__ __launch_bounds__(kThreads) void lane_pair_kernel(const float* __restrict__ pe,
                                                             int64_t length, int pairs,
                                                             float* __restrict__ cos_t,
                                                             float* __restrict__ sin_t) {
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= length * pairs) return;
  const float4 m = reinterpret_cast<const float4*>(pe)[idx];  // (cos, -sin, sin, cos)
  reinterpret_cast<float2*>(cos_t)[idx] = make_float2(m.x, m.x);
  reinterpret_cast<float2*>(sin_t)[idx] = make_float2(-m.z, m.z);
}

__global__ __launch_bounds__(kThreads) void rope_lanes_kernel(const float* __restrict__ ids,
                                                              int64_t stride, int64_t length,
                                                              Axes ax, float theta,
                                                              float* __restrict__ cos_t,
                                                              float* __restrict__ sin_t) {
  const int pairs = ax.first_pair[ax.count];
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= length * pairs) return;
  const int64_t t = idx / pairs;
  const int pair = (int)(idx - t * pairs);
  float c, s;
  angle_of(ids, stride, t, pair, ax, theta, c, s);
  reinterpret_cast<float2*>(cos_t)[idx] = make_float2(c, c);
  reinterpret_cast<float2*>(sin_t)[idx] = make_float2(-s, s);
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

extern "C" int flk_rope_embed(const float* ids, int64_t ids_row_stride, int64_t length,
                              int n_axes, const int* axes_dim, float theta, float* pe,
                              void* stream) {
  Axes ax;
  const int st = flk_make_axes(n_axes, axes_dim, ax);
  if (st != FLK_OK) return st;
  if (length < 0 || ids_row_stride < n_axes) return FLK_E_INVALID;
  const int64_t n = length * ax.first_pair[n_axes];
  if (n == 0) return FLK_OK;
  if (!ids || !pe) return FLK_E_INVALID;
  if (!flk_host_aligned(pe, 16)) return FLK_E_ALIGN;
  if (n / kThreads >= INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(rope_embed_kernel, dim3(blocks_for(n)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), ids, ids_row_stride, length, ax, theta, pe);
  return flk_launch_status();
}

extern "C" int flk_lane_pair(const float* pe, int64_t length, int pairs, float* cos,
                             float* sin, void* stream) {
  if (length < 0 || pairs < 0) return FLK_E_INVALID;
  const int64_t n = length * pairs;
  if (n == 0) return FLK_OK;
  if (!pe || !cos || !sin) return FLK_E_INVALID;
  if (!flk_host_aligned(pe, 16) || !flk_host_aligned(cos, 8) || !flk_host_aligned(sin, 8))
    return FLK_E_ALIGN;
  if (n / kThreads >= INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(lane_pair_kernel, dim3(blocks_for(n)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), pe, length, pairs, cos, sin);
  return flk_launch_status();
}

extern "C" int flk_rope_lanes(const float* ids, int64_t ids_row_stride, int64_t length,
                              int n_axes, const int* axes_dim, float theta, float* cos,
                              float* sin, void* stream) {
  Axes ax;
  const int st = flk_make_axes(n_axes, axes_dim, ax);
  if (st != FLK_OK) return st;
  if (length < 0 || ids_row_stride < n_axes) return FLK_E_INVALID;
  const int64_t n = length * ax.first_pair[n_axes];
  if (n == 0) return FLK_OK;
  if (!ids || !cos || !sin) return FLK_E_INVALID;
  if (!flk_host_aligned(cos, 8) || !flk_host_aligned(sin, 8)) return FLK_E_ALIGN;
  if (n / kThreads >= INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(rope_lanes_kernel, dim3(blocks_for(n)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), ids, ids_row_stride, length, ax, theta,
                     cos, sin);
  return flk_launch_status();
}
