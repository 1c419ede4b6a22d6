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
// each RoPE pair (2j, 2j+1) stays inside one lane.  A 128-thread block holds 8
// consecutive tokens (measured as fast as 256 threads with tables and 3% faster with ids,
// whose per-block setup then overlaps more blocks); the 4 groups of a wave write 4
// consecutive tokens of the same head = 1 KiB contiguous per store instruction.  Each group handles
// kHeads heads of its token, issuing all 3*kHeads loads (nontemporal: the activation is
// read once) before any math, and keeps the token's cos/sin lanes in registers across
// those heads.
//
// The RoPE lanes come from one of two sources: the (L, 128) f32 cos / sin tables
// (kernels.py:28-31), or -- flk_qk_prep_ids -- the token's position ids, from which each
// lane computes the cos / sin of its 4 pairs (rope.py:9-21) while its loads are in flight.
// The pair frequencies are computed once per block, into LDS.  Both use the table kernels'
// arithmetic (rope_math.h), so the two sources give identical bits.
//
// The kernel is HBM-bound: per (b, t, h) it moves 3*256 bytes in and 3*256 out.

#include "qk_math.h"
#include "rope_math.h"

namespace {

constexpr int kHeadDim = 128;
constexpr int kLanesPerRow = 16;
#ifndef FLK_QK_THREADS
#define FLK_QK_THREADS 128
#endif
constexpr int kThreads = FLK_QK_THREADS;   // block size (a tuning knob): 16 lanes per token row
constexpr int kTokensPerBlock = kThreads / kLanesPerRow;
static_assert(kThreads % 64 == 0 && kThreads <= 1024, "whole waves, at most 1024 threads");

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
#ifndef FLK_QK_IDS_HPG
#define FLK_QK_IDS_HPG 0
#endif

// Where the RoPE lanes of token t come from: tables (cos / sin rows of table_stride floats)
// or position ids (rows of ids_stride floats, one per axis of ax).
struct RopeSource {
  const float* cos;
  const float* sin;
  int64_t table_stride;
  const float* ids;
  int64_t ids_stride;
  flk::Axes ax;
  float theta;
};

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

// 8 float32 values of a head row (32 bytes per lane) for the float32 outputs of the plain
// branch; the default cache policy, as for the bf16 stores.
__device__ __forceinline__ void store_f32x8(float* p, const float r[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(r[0], r[1], r[2], r[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(r[4], r[5], r[6], r[7]);
}

// kOutF32: q and k are stored as float32 (no gain, no final rounding): the plain branch of
// qkv_prep with float32 scales (flk_qk_prep_f32); q_out / k_out then point at floats.
template <bool kScaleF32, bool kGain, int kHeads, bool kOutF32 = false>
__global__ __launch_bounds__(kThreads) void qk_prep_kernel(
    const uint16_t* __restrict__ qkv, int64_t batch_stride, int64_t row_stride, RopeSource rope,
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
  flk::load_table8(rope.cos + (int64_t)t * rope.table_stride, lane, c);
  flk::load_table8(rope.sin + (int64_t)t * rope.table_stride, lane, s);
  flk::load_scale8<kScaleF32>(q_scale, lane, qs);
  flk::load_scale8<kScaleF32>(k_scale, lane, ks);

#pragma unroll
  for (int i = 0; i < kHeads; ++i) {
    const int64_t o =
        (((int64_t)b * num_heads + h0 + i) * out_length + out_offset + t) * kHeadDim + lane * 8;
    if constexpr (kOutF32) {
      float r[8];
      flk::norm_rotate_f32<kScaleF32>(rq[i], qs, c, s, r);
      store_f32x8(reinterpret_cast<float*>(q_out) + o, r);
      flk::norm_rotate_f32<kScaleF32>(rk[i], ks, c, s, r);
      store_f32x8(reinterpret_cast<float*>(k_out) + o, r);
    } else {
      store16(q_out + o, flk::norm_rotate<kScaleF32, kGain>(rq[i], qs, c, s, q_gain));
      store16(k_out + o, flk::norm_rotate<kScaleF32, false>(rk[i], ks, c, s, 1.0f));
    }
    store16(v_out + o, rv[i]);
  }
}

// The ids form.  Each 16-lane group computes the cos / sin of its 4 pairs once and applies
// them to kRounds rounds of kHeads heads of its token; the next round's loads are issued
// before the current round's math, so each lane keeps two rounds in flight while the trig of
// one token serves kRounds * kHeads heads.  The block's first 64 threads compute the
// (token-independent) pair frequencies into LDS after the first loads are issued.
//
// The trig must not wait for the QKV data.  Loads complete in issue order as far as the
// wait counter is concerned, so the positions are loaded first, and every load is issued
// unconditionally (a lane past the end reads the last token's row and stores nothing): a
// load under a branch makes the compiler wait for all outstanding loads where the paths
// join, which put the whole frequency -> barrier -> trig chain behind the first round's data.
template <bool kScaleF32, bool kGain, int kHeads, int kRounds>
__global__ __launch_bounds__(kThreads) void qk_prep_ids_kernel(
    const uint16_t* __restrict__ qkv, int64_t batch_stride, int64_t row_stride, RopeSource rope,
    const void* __restrict__ q_scale, const void* __restrict__ k_scale, float q_gain,
    int length, int num_heads, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
    uint16_t* __restrict__ v_out, int64_t out_length, int64_t out_offset) {
  constexpr int kPairs = kHeadDim / 2;
  __shared__ float pair_freq[kPairs];
  __shared__ int pair_axis[kPairs];
  const int lane = threadIdx.x & (kLanesPerRow - 1);
  const int t = blockIdx.x * kTokensPerBlock + (threadIdx.x >> 4);
  const int h0 = blockIdx.y * kHeads * kRounds;
  const int b = blockIdx.z;
  const bool live = t < length;
  const int tl = live ? t : length - 1;
  const uint16_t* row = qkv + (int64_t)b * batch_stride + (int64_t)tl * row_stride + lane * 8;

  uint4 buf[2][3 * kHeads];
  auto load_round = [&](int r, uint4 (&dst)[3 * kHeads]) {
#pragma unroll
    for (int i = 0; i < kHeads; ++i) {
      const int h = h0 + r * kHeads + i;
      dst[3 * i] = load16(row + (int64_t)h * kHeadDim);
      dst[3 * i + 1] = load16(row + (int64_t)(num_heads + h) * kHeadDim);
      dst[3 * i + 2] = load16(row + (int64_t)(2 * num_heads + h) * kHeadDim);
    }
  };
  // The token's positions on every axis (each lane then picks the axis of each of its pairs),
  // loaded before the QKV rows; axes past the count re-read axis 0 and go unused.
  const float* pos = rope.ids + (int64_t)tl * rope.ids_stride;
  float pa[flk::kMaxAxes];
#pragma unroll
  for (int a = 0; a < flk::kMaxAxes; ++a) pa[a] = pos[a < rope.ax.count ? a : 0];
  load_round(0, buf[0]);
  if (threadIdx.x < kPairs) {
    int axis;
    pair_freq[threadIdx.x] = flk::pair_omega(threadIdx.x, rope.ax, rope.theta, axis);
    pair_axis[threadIdx.x] = axis;
  }
  __syncthreads();
  if (!live) return;   // whole 16-lane rows exit together, so DPP rows stay intact

  // lane l holds lane-table columns 8l .. 8l+7 = pairs 4l .. 4l+3:
  // cos column 2p, 2p+1 = cos(angle_p); sin columns = -sin(angle_p), +sin(angle_p)
  float c[8], s[8], qs[8], ks[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int axis = pair_axis[lane * 4 + j];
    float position = pa[0];
#pragma unroll
    for (int a = 1; a < flk::kMaxAxes; ++a) position = axis == a ? pa[a] : position;
    float cj, sj;
    flk::pair_cos_sin(position, pair_freq[lane * 4 + j], cj, sj);
    c[2 * j] = cj;
    c[2 * j + 1] = cj;
    s[2 * j] = -sj;
    s[2 * j + 1] = sj;
  }
  flk::load_scale8<kScaleF32>(q_scale, lane, qs);
  flk::load_scale8<kScaleF32>(k_scale, lane, ks);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    if (r + 1 < kRounds) load_round(r + 1, buf[(r + 1) & 1]);
    const uint4 (&cur)[3 * kHeads] = buf[r & 1];
#pragma unroll
    for (int i = 0; i < kHeads; ++i) {
      const int h = h0 + r * kHeads + i;
      const int64_t o = (((int64_t)b * num_heads + h) * out_length + out_offset + t) * kHeadDim + lane * 8;
      store16(q_out + o, flk::norm_rotate<kScaleF32, kGain>(cur[3 * i], qs, c, s, q_gain));
      store16(k_out + o, flk::norm_rotate<kScaleF32, false>(cur[3 * i + 1], ks, c, s, 1.0f));
      store16(v_out + o, cur[3 * i + 2]);
    }
  }
}

struct Launch {
  const uint16_t* qkv;
  int64_t batch_stride, row_stride;
  RopeSource rope;
  const void* q_scale;
  const void* k_scale;
  float q_gain;
  int length, num_heads;
  uint16_t *q, *k, *v;
  int64_t out_length, out_offset;
};

#ifndef FLK_QK_IDS_ROUNDS
#define FLK_QK_IDS_ROUNDS 2
#endif

// Launches the kernel built for `heads_per_group` heads per 16-lane group (the grid's y size
// is num_heads / heads_per_group); FLK_E_UNSUPPORTED, with nothing launched, for a count that
// has no kernel (a forced tuning knob), so the grid and the kernel always agree.
template <bool kScaleF32, bool kGain, bool kIds>
int launch(int heads_per_group, dim3 grid, hipStream_t stream, const Launch& a) {
#define FLK_QK_ARGS                                                                                \
  a.qkv, a.batch_stride, a.row_stride, a.rope, a.q_scale, a.k_scale, a.q_gain, a.length, a.num_heads, \
      a.q, a.k, a.v, a.out_length, a.out_offset
#define FLK_QK_LAUNCH(NH) \
  hipLaunchKernelGGL((qk_prep_kernel<kScaleF32, kGain, NH>), grid, dim3(kThreads), 0, stream, FLK_QK_ARGS)
#define FLK_QK_IDS(NH, R) \
  hipLaunchKernelGGL((qk_prep_ids_kernel<kScaleF32, kGain, NH, R>), grid, dim3(kThreads), 0, stream, FLK_QK_ARGS)
  int status = FLK_OK;
  if constexpr (kIds) {
    // heads_per_group = heads per round x rounds
    if (heads_per_group == 2 * FLK_QK_IDS_ROUNDS) FLK_QK_IDS(2, FLK_QK_IDS_ROUNDS);
    else if (heads_per_group == 2) FLK_QK_IDS(2, 1);
    else if (heads_per_group == 3) FLK_QK_IDS(3, 1);
    else if (heads_per_group == 1) FLK_QK_IDS(1, 1);
    else status = FLK_E_UNSUPPORTED;
  } else {
    switch (heads_per_group) {
      case 6: FLK_QK_LAUNCH(6); break;
      case 4: FLK_QK_LAUNCH(4); break;
      case 3: FLK_QK_LAUNCH(3); break;
      case 2: FLK_QK_LAUNCH(2); break;
      case 1: FLK_QK_LAUNCH(1); break;
      default: status = FLK_E_UNSUPPORTED; break;
    }
  }
#undef FLK_QK_IDS
#undef FLK_QK_LAUNCH
#undef FLK_QK_ARGS
  return status;
}

// Checks shared by both entry points: FLK_OK = launch, kEmpty = nothing to do (an empty
// batch or sequence is accepted before any pointer or stride check), else an error status.
constexpr int kEmpty = 1;

int check_common(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                 const void* q_scale, const void* k_scale, int batch, int length, int num_heads,
                 int head_dim, const void* q_out, const void* k_out, const void* v_out,
                 int64_t out_length, int64_t out_offset) {
  if (head_dim != kHeadDim) return FLK_E_UNSUPPORTED;
  if (batch < 0 || length < 0 || num_heads <= 0 || out_offset < 0 ||
      out_offset + length > out_length)
    return FLK_E_INVALID;
  if (batch == 0 || length == 0) return kEmpty;
  if (length > INT32_MAX - kTokensPerBlock) return FLK_E_INVALID;   // token index of the last block's lanes
  if (qkv_row_stride < 3LL * num_heads * head_dim ||
      (batch > 1 && qkv_batch_stride < (int64_t)(length - 1) * qkv_row_stride + 3LL * num_heads * head_dim))
    return FLK_E_INVALID;
  if (!qkv || !q_scale || !k_scale || !q_out || !k_out || !v_out) return FLK_E_INVALID;
  if (qkv_row_stride % 8 || qkv_batch_stride % 8 || !flk_host_aligned(qkv, 16) ||
      !flk_host_aligned(q_scale, 16) || !flk_host_aligned(k_scale, 16) ||
      !flk_host_aligned(q_out, 16) || !flk_host_aligned(k_out, 16) || !flk_host_aligned(v_out, 16))
    return FLK_E_ALIGN;
  return FLK_OK;
}

template <bool kIds>
int dispatch(int hpg, int batch, int scale_is_f32, hipStream_t stream, const Launch& a) {
  const dim3 grid((unsigned)(((int64_t)a.length + kTokensPerBlock - 1) / kTokensPerBlock), a.num_heads / hpg, batch);
  const bool gain = a.q_gain != 1.0f;
  int st;
  if (scale_is_f32) st = gain ? launch<true, true, kIds>(hpg, grid, stream, a) : launch<true, false, kIds>(hpg, grid, stream, a);
  else st = gain ? launch<false, true, kIds>(hpg, grid, stream, a) : launch<false, false, kIds>(hpg, grid, stream, a);
  return st != FLK_OK ? st : flk_launch_status();
}

// Heads per 16-lane group.  With tables, two measured best at the Klein shapes (6 loads in
// flight per lane and 2x more blocks than four heads per group).  With ids, each group
// computes 4 cos/sin pairs per token, which more heads share: two rounds of two measured
// best (three rounds: the same at 1024^2, 1.3 us slower at 512^2, 2 us at 2048^2).
int heads_per_group(int num_heads, bool ids, int forced) {
  int hpg = (num_heads % 2 == 0) ? 2 : (num_heads % 3 == 0) ? 3 : 1;
  if (ids && num_heads % (2 * FLK_QK_IDS_ROUNDS) == 0) hpg = 2 * FLK_QK_IDS_ROUNDS;
  if (forced > 0 && num_heads % forced == 0) hpg = forced;
  return hpg;
}

}  // namespace

extern "C" int flk_qk_prep(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                           const float* cos, const float* sin, int64_t table_row_stride,
                           const void* q_scale, const void* k_scale, int scale_is_f32,
                           float q_gain, int batch, int length, int num_heads, int head_dim,
                           void* q_out, void* k_out, void* v_out, int64_t out_length,
                           int64_t out_offset, void* stream) {
  const int st = check_common(qkv, qkv_batch_stride, qkv_row_stride, q_scale, k_scale, batch,
                              length, num_heads, head_dim, q_out, k_out, v_out, out_length, out_offset);
  if (st != FLK_OK) return st == kEmpty ? FLK_OK : st;
  if (table_row_stride < head_dim || !cos || !sin) return FLK_E_INVALID;
  if (table_row_stride % 4 || !flk_host_aligned(cos, 16) || !flk_host_aligned(sin, 16))
    return FLK_E_ALIGN;
  Launch a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.batch_stride = qkv_batch_stride;
  a.row_stride = qkv_row_stride;
  a.rope.cos = cos;
  a.rope.sin = sin;
  a.rope.table_stride = table_row_stride;
  a.q_scale = q_scale;
  a.k_scale = k_scale;
  a.q_gain = q_gain;
  a.length = length;
  a.num_heads = num_heads;
  a.q = static_cast<uint16_t*>(q_out);
  a.k = static_cast<uint16_t*>(k_out);
  a.v = static_cast<uint16_t*>(v_out);
  a.out_length = out_length;
  a.out_offset = out_offset;
  return dispatch<false>(heads_per_group(num_heads, false, FLK_QK_HPG), batch, scale_is_f32,
                         static_cast<hipStream_t>(stream), a);
}

extern "C" int flk_qk_prep_f32(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                               const float* cos, const float* sin, int64_t table_row_stride,
                               const float* q_scale, const float* k_scale, int batch, int length,
                               int num_heads, int head_dim, float* q_out, float* k_out, void* v_out,
                               int64_t out_length, int64_t out_offset, void* stream) {
  const int st = check_common(qkv, qkv_batch_stride, qkv_row_stride, q_scale, k_scale, batch,
                              length, num_heads, head_dim, q_out, k_out, v_out, out_length, out_offset);
  if (st != FLK_OK) return st == kEmpty ? FLK_OK : st;
  if (table_row_stride < head_dim || !cos || !sin) return FLK_E_INVALID;
  if (table_row_stride % 4 || !flk_host_aligned(cos, 16) || !flk_host_aligned(sin, 16))
    return FLK_E_ALIGN;
  RopeSource rope{};
  rope.cos = cos;
  rope.sin = sin;
  rope.table_stride = table_row_stride;
  const int hpg = num_heads % 2 == 0 ? 2 : 1;
  const dim3 grid((unsigned)(((int64_t)length + kTokensPerBlock - 1) / kTokensPerBlock), num_heads / hpg, batch);
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(qkv);
  uint16_t* qo = reinterpret_cast<uint16_t*>(q_out);
  uint16_t* ko = reinterpret_cast<uint16_t*>(k_out);
  uint16_t* vo = static_cast<uint16_t*>(v_out);
  if (hpg == 2)
    hipLaunchKernelGGL((qk_prep_kernel<true, false, 2, true>), grid, dim3(kThreads), 0, hs, x, qkv_batch_stride,
                       qkv_row_stride, rope, q_scale, k_scale, 1.0f, length, num_heads, qo, ko, vo, out_length,
                       out_offset);
  else
    hipLaunchKernelGGL((qk_prep_kernel<true, false, 1, true>), grid, dim3(kThreads), 0, hs, x, qkv_batch_stride,
                       qkv_row_stride, rope, q_scale, k_scale, 1.0f, length, num_heads, qo, ko, vo, out_length,
                       out_offset);
  return flk_launch_status();
}

extern "C" int flk_qk_prep_ids(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                               const float* ids, int64_t ids_row_stride, int n_axes,
                               const int* axes_dim, float theta, const void* q_scale,
                               const void* k_scale, int scale_is_f32, float q_gain, int batch,
                               int length, int num_heads, int head_dim, void* q_out, void* k_out,
                               void* v_out, int64_t out_length, int64_t out_offset, void* stream) {
  const int st = check_common(qkv, qkv_batch_stride, qkv_row_stride, q_scale, k_scale, batch,
                              length, num_heads, head_dim, q_out, k_out, v_out, out_length, out_offset);
  Launch a{};
  const int ax_st = flk_make_axes(n_axes, axes_dim, a.rope.ax);
  if (ax_st != FLK_OK) return ax_st;
  if (2 * a.rope.ax.first_pair[n_axes] != kHeadDim || ids_row_stride < n_axes) return FLK_E_INVALID;
  if (st != FLK_OK) return st == kEmpty ? FLK_OK : st;
  if (!ids) return FLK_E_INVALID;
  if (!flk_host_aligned(ids, 4)) return FLK_E_ALIGN;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.batch_stride = qkv_batch_stride;
  a.row_stride = qkv_row_stride;
  a.rope.ids = ids;
  a.rope.ids_stride = ids_row_stride;
  a.rope.theta = theta;
  a.q_scale = q_scale;
  a.k_scale = k_scale;
  a.q_gain = q_gain;
  a.length = length;
  a.num_heads = num_heads;
  a.q = static_cast<uint16_t*>(q_out);
  a.k = static_cast<uint16_t*>(k_out);
  a.v = static_cast<uint16_t*>(v_out);
  a.out_length = out_length;
  a.out_offset = out_offset;
  return dispatch<true>(heads_per_group(num_heads, true, FLK_QK_IDS_HPG), batch, scale_is_f32,
                        static_cast<hipStream_t>(stream), a);
}
