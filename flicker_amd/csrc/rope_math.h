// RoPE angle arithmetic (src/flicker/rope.py:9-21), shared by the table kernels (rope.hip)
// and qk_prep's on-the-fly variant, so that a cos/sin computed inside qk_prep is the same
// value, bit for bit, as the one the table kernels store.
//
// For pair k of an axis of width dim (k < dim/2) and position x:
//   omega = 1 / theta^(2k/dim)   (f32: 2k/dim divided in f32, powf, 1/x)
//   angle = x * omega            (f32)
//   pe    = [[cos, -sin], [sin, cos]](angle)
// Pairs of the axes are concatenated in axis order.
#pragma once

#include "common.h"

namespace flk {

constexpr int kMaxAxes = 8;

struct Axes {
  int count;
  int dim[kMaxAxes];
  int first_pair[kMaxAxes + 1];  // prefix sums of dim/2
};

// Axis of a pair index and that pair's frequency omega.  The axis's fields are picked by
// selects over constant indices: indexing the (kernel-argument) arrays with a per-lane axis
// would compile to memory loads, whose wait then also waits for every load issued before.
__device__ __forceinline__ float pair_omega(int pair, const Axes& ax, float theta, int& axis) {
  int a = 0, first = ax.first_pair[0], dim = ax.dim[0];
#pragma unroll
  for (int i = 1; i < kMaxAxes; ++i) {
    const bool in = i < ax.count && pair >= ax.first_pair[i];
    a = in ? i : a;
    first = in ? ax.first_pair[i] : first;
    dim = in ? ax.dim[i] : dim;
  }
  axis = a;
  const int kk = pair - first;
  const float scale = (float)(2 * kk) / (float)dim;
  return 1.0f / powf(theta, scale);
}

__device__ __forceinline__ void pair_cos_sin(float position, float omega, float& c, float& s) {
  const float angle = position * omega;
  c = cosf(angle);
  s = sinf(angle);
}

}  // namespace flk

// Host: validate per-axis widths and fill an Axes table.
static inline int flk_make_axes(int n_axes, const int* axes_dim, flk::Axes& ax) {
  if (n_axes < 1 || n_axes > flk::kMaxAxes || !axes_dim) return FLK_E_INVALID;
  ax.count = n_axes;
  ax.first_pair[0] = 0;
  for (int i = 0; i < flk::kMaxAxes; ++i) ax.dim[i] = 2;
  for (int i = 0; i < n_axes; ++i) {
    if (axes_dim[i] <= 0 || axes_dim[i] % 2) return FLK_E_INVALID;
    ax.dim[i] = axes_dim[i];
    ax.first_pair[i + 1] = ax.first_pair[i] + axes_dim[i] / 2;
  }
  for (int i = n_axes + 1; i <= flk::kMaxAxes; ++i) ax.first_pair[i] = ax.first_pair[n_axes];
  return FLK_OK;
}
