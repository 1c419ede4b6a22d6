// w8a8: SmoothQuant int8 QKV projection for gfx950 (int8 MFMA, int32 accumulate).
//
// The reference projects x @ w in bf16 (src/flicker/nn.py:13-14, called for the QKV
// projection at src/flicker/modules.py:128,132,186) and has no quantisation.  This file
// implements the replacement defined by the formula below; every integer and every
// float32 rounding is reproduced exactly (each float op is one IEEE f32 operation with
// round-to-nearest-even; division and sqrt correctly rounded; rint ties-to-even):
//
//   calibration   s_j = sqrt(max_t |X[t,j]|) / sqrt(max_o |W[j,o]|)  (1 if either is 0)
//                 inv_s_j = 1 / s_j
//   weight        Wh[j,o] = f32(W[j,o]) * s_j;  w_o = max_j |Wh[j,o]| / 127 (1 if 0)
//                 Wq[j,o] = clamp(rint(Wh[j,o] / w_o), -127, 127)           int8
//   activation    Xh[t,j] = f32(X[t,j]) * inv_s_j;  a_t = max_j |Xh[t,j]| / 127 (1 if 0)
//                 Xq[t,j] = clamp(rint(Xh[t,j] / a_t), -127, 127)           int8
//   GEMM          acc[t,o] = sum_j Xq[t,j] * Wq[j,o]                          int32, exact
//   rescale       Y[t,o] = bf16((f32(acc[t,o]) * a_t) * w_o)
//
// Layouts: X (M, K) and W (K, N) bf16 row-major with row strides (W as the reference
// stores it: in x out); Xq (M, K) int8; the quantised weight is stored transposed,
// WqT (N, K) int8, so both GEMM operands are K-contiguous rows; Y (M, N) bf16 with a
// row stride; optional acc (M, N) int32.
//
// GEMM.  A block of 8 waves (two per SIMD) owns a 256 (n) x 256 (m) output tile and
// computes it transposed, Y^T = WqT . Xq^T, with v_mfma_i32_16x16x64_i8: A operand = 16 WqT
// rows x 64 k bytes, B operand = 16 Xq rows x 64 k bytes, both one ds_read_b128 per lane.
// Under random int8 data the chip runs at its power limit, where the 16x16x64 form does the
// same ops on less energy than 32x32x32 (a quarter of the accumulator traffic per
// instruction; an MFMA stream with random operands issues 12-17% more ops per second).  In
// the 16x16 accumulator a lane owns one token and 4 consecutive output channels.  Each wave
// holds a 128 (n) x 64 (m) sub-tile: 32 accumulators of 4 int32 (128 registers), 12 operand
// reads per 32 MFMAs.  k advances in 128-byte stages (one full 128-byte line per operand
// row) through two 64 KiB LDS buffers filled by global_load_lds_dwordx4 (no registers); a
// row's 16-byte chunk c is stored at c ^ gswz(row), which keeps every operand read on
// distinct banks.  Integer sums are exact in any order, so the products are those of any
// other tiling, bit for bit.  The epilogue rescales into LDS and
// stores whole 256-byte output rows.  Blocks are renumbered so consecutive output tiles
// share an XCD (and its L2), and grouped so that 4 token tiles sweep the channel tiles
// together.
//
// A launch of more than one round (the Klein projection: 648 tiles, 2.53 rounds of 256 CUs)
// takes the rounds order: each XCD runs whole rounds of 32 of its tiles, then cuts the tiles
// left over into tiles of 192 tokens (waves of 128 x 48: three token fragments), so the
// partial last round has up to 4/3 as many blocks with 3/4 of the work each (measured 1-5%
// faster for the plain GEMM, 3-6% with the qk_prep epilogue).
//
// A launch takes up to two problems (GemmGroup; the activation quantiser likewise takes a
// QuantGroup): a double block's text and image projections share one grid, so the small
// text projection runs on the CUs the image projection leaves idle in its last round.

#include <algorithm>

#include "qk_math.h"

namespace {

using flk::f32x4;
using flk::i32x4;
using flk::i32x16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kQMax = 127.0f;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}

__device__ __forceinline__ float absmax_scale(float amax) { return amax > 0.0f ? amax / kQMax : 1.0f; }

// clamp(rint(v / scale), -127, 127) as an integer.
__device__ __forceinline__ int quantize(float v, float scale) {
  const float q = __builtin_rintf(v / scale);
  return (int)fminf(fmaxf(q, -kQMax), kQMax);
}

// quantize(v, scale) without a division per element.  r = 1/scale is rounded once per row;
// p = v * r is then within 3 * 2^-24 |p| < 2^-22 |p| of the correctly rounded quotient q
// (r, p and q each carry at most half an ulp of relative error).  When p is farther than
// 2^-21 |p| from a rounding boundary (a half-integer), q lies on the same side and
// rint(p) == rint(q); otherwise -- p near a tie, or not finite -- the division is done.
// p - rint(p) is exact (Sterbenz), so the test itself does not round.
__device__ __forceinline__ int quantize_recip(float v, float scale, float r) {
  const float p = v * r;
  float t = __builtin_rintf(p);
  if (!(fabsf(p - t) < 0.5f - fabsf(p) * 0x1p-21f)) t = __builtin_rintf(v / scale);
  return (int)fminf(fmaxf(t, -kQMax), kQMax);
}

__device__ __forceinline__ uint32_t pack_i8x4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
         ((uint32_t)(d & 0xFF) << 24);
}

__device__ __forceinline__ void unpack_bf16x8(const uint4& r, float (&f)[8]) {
  f[0] = flk::bf16_lo(r.x); f[1] = flk::bf16_hi(r.x);
  f[2] = flk::bf16_lo(r.y); f[3] = flk::bf16_hi(r.y);
  f[4] = flk::bf16_lo(r.z); f[5] = flk::bf16_hi(r.z);
  f[6] = flk::bf16_lo(r.w); f[7] = flk::bf16_hi(r.w);
}

// ---------------------------------------------------------------- calibration ----------

// out[r] = max_c |x[r, c]|; one wave per row, 8 columns per lane step (cols % 8 == 0).
__global__ __launch_bounds__(256) void absmax_rows_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                          int64_t cols, int64_t stride,
                                                          float* __restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const uint16_t* p = x + row * stride;
  float m = 0.0f;
  for (int64_t c = (int64_t)lane * 8; c < cols; c += 512) {
    float f[8];
    unpack_bf16x8(*reinterpret_cast<const uint4*>(p + c), f);
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
  }
  m = wave_max(m);
  if (lane == 0) out[row] = m;
}

// out[c] = max_r |x[r, c]| (or max with the existing out[c] when accumulating over
// calibration batches).  A block covers 128 columns: 16 lane groups of 8 columns x 16 row
// groups, reduced through LDS; each column has exactly one writer.
__global__ __launch_bounds__(256) void absmax_cols_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                          int64_t cols, int64_t stride, int accumulate,
                                                          float* __restrict__ out) {
  __shared__ float red[16][129];
  const int cg = threadIdx.x & 15, rg = threadIdx.x >> 4;
  const int64_t c0 = (int64_t)blockIdx.x * 128 + cg * 8;
  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (c0 < cols) {
    for (int64_t r = rg; r < rows; r += 16) {
      float f[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(x + r * stride + c0), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = fmaxf(m[i], fabsf(f[i]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[rg][cg * 8 + i] = m[i];
  __syncthreads();
  if (threadIdx.x < 128) {
    const int64_t c = (int64_t)blockIdx.x * 128 + threadIdx.x;
    if (c < cols) {
      float v = 0.0f;
#pragma unroll
      for (int g = 0; g < 16; ++g) v = fmaxf(v, red[g][threadIdx.x]);
      if (accumulate) v = fmaxf(v, out[c]);
      out[c] = v;
    }
  }
}

// s = sqrt(xa) / sqrt(wa) (1 where either maximum is 0), inv_s = 1 / s.
__global__ void smooth_factors_kernel(const float* __restrict__ xa, const float* __restrict__ wa, int64_t k,
                                      float* __restrict__ s, float* __restrict__ inv_s) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= k) return;
  const float a = xa[i], b = wa[i];
  const float v = (a > 0.0f && b > 0.0f) ? __builtin_sqrtf(a) / __builtin_sqrtf(b) : 1.0f;
  s[i] = v;
  inv_s[i] = 1.0f / v;
}

// ---------------------------------------------------------------- quantisation ---------

// Weight (offline): one block per 64 output channels.  Pass 1: column absmax of Wh over all
// K (8 channel groups x 32 row groups, LDS reduction) -> w_scale.  Pass 2: 64-row k tiles
// are quantised into an LDS tile [channel][k] and written as 64-byte runs of WqT rows.
__global__ __launch_bounds__(256) void quantize_weight_kernel(const uint16_t* __restrict__ w, int64_t w_stride,
                                                              const float* __restrict__ s, int K, int N,
                                                              int8_t* __restrict__ wqt,
                                                              float* __restrict__ w_scale) {
  __shared__ float red[32][65];
  __shared__ float scale[64];
  __shared__ __attribute__((aligned(16))) uint8_t tile[64][80];
  const int tid = threadIdx.x;
  const int cg = tid & 7, rg = tid >> 3;
  const int n0 = blockIdx.x * 64;
  const int nc = n0 + cg * 8;
  const bool active = nc < N;

  float m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (active) {
    for (int j = rg; j < K; j += 32) {
      const float sj = s[j];
      float f[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(w + (int64_t)j * w_stride + nc), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) m[i] = fmaxf(m[i], fabsf(f[i] * sj));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[rg][cg * 8 + i] = m[i];
  __syncthreads();
  if (tid < 64) {
    float v = 0.0f;
#pragma unroll 8
    for (int g = 0; g < 32; ++g) v = fmaxf(v, red[g][tid]);
    const float sc = absmax_scale(v);
    scale[tid] = sc;
    if (n0 + tid < N) w_scale[n0 + tid] = sc;
  }
  __syncthreads();

  float sc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) sc[i] = scale[cg * 8 + i];
  for (int k0 = 0; k0 < K; k0 += 64) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int r = rg + it * 32;
      const int j = k0 + r;
      if (active) {
        const float sj = s[j];
        float f[8];
        unpack_bf16x8(*reinterpret_cast<const uint4*>(w + (int64_t)j * w_stride + nc), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) tile[cg * 8 + i][r] = (uint8_t)quantize(f[i] * sj, sc[i]);
      }
    }
    __syncthreads();
    const int n = tid >> 2, ch = tid & 3;
    if (n0 + n < N)
      *reinterpret_cast<uint4*>(wqt + (int64_t)(n0 + n) * K + k0 + ch * 16) =
          *reinterpret_cast<const uint4*>(&tile[n][ch * 16]);
    __syncthreads();
  }
}

// Activation (per forward): one wave per token row, the row held in registers
// (kChunks x 8 elements per lane), absmax reduced across the wave.
//
// kModulate: the row is first the block input x and becomes the projection input
//   X = bf16(bf16((bf16(1 + scale) * bf16(layer_norm(x)))) + shift)      (modules.py:38-40)
// with layer_norm(x) = bf16((x - mean) * (1 / sqrt(var + 1e-6))) (nn.py:17-21), the mean and
// the variance each summed in float64 and rounded to float32 once (bf16 inputs make the f64
// sum of the row exact, so the mean does not depend on the summation order), every other
// step one f32 operation.  scale / shift are the modulation rows of the token's batch entry;
// X is optionally stored (bf16) for other consumers of the modulated input.
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// One activation of a quantisation launch (rows of M tokens, all of width K).
struct QuantProblem {
  const uint16_t* x;
  int64_t x_stride;
  const float* inv_s;
  int M;
  int8_t* xq;
  float* a_scale;
  const uint16_t* shift;    // kModulate: modulation rows of each batch entry
  const uint16_t* scale;
  int64_t mod_stride;
  int tokens_per_batch;
  uint16_t* x_mod;          // kModulate: optional store of the modulated input
  int64_t x_mod_stride;
};

// Up to two activations in one launch (a double block's text and image streams): blocks
// [0, first_blocks) take p[0], the rest p[1]; four rows per block.
struct QuantGroup {
  QuantProblem p[2];
  int first_blocks;
  int K;
};

template <int kChunks, bool kModulate>
__global__ __launch_bounds__(256) void quantize_act_kernel(const QuantGroup grp) {
  const bool second = (int)blockIdx.x >= grp.first_blocks;
  const QuantProblem& P = second ? grp.p[1] : grp.p[0];   // wave-uniform, read from the kernel arguments
  const uint16_t* __restrict__ x = P.x;
  const int64_t x_stride = P.x_stride;
  const float* __restrict__ inv_s = P.inv_s;
  const int M = P.M, K = grp.K;
  int8_t* __restrict__ xq = P.xq;
  float* __restrict__ a_scale = P.a_scale;
  const uint16_t* __restrict__ shift = P.shift;
  const uint16_t* __restrict__ scale = P.scale;
  const int64_t mod_stride = P.mod_stride;
  const int tokens_per_batch = P.tokens_per_batch;
  uint16_t* __restrict__ x_mod = P.x_mod;
  const int64_t x_mod_stride = P.x_mod_stride;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = ((int)blockIdx.x - (second ? grp.first_blocks : 0)) * 4 + wave;
  if (row >= M) return;
  const int nch = K >> 3;
  const uint16_t* src = x + (int64_t)row * x_stride;
  uint4 raw[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int idx = c * 64 + lane;
    u32x4 v = {0, 0, 0, 0};
    if (idx < nch) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + idx);
    raw[c] = uint4{v.x, v.y, v.z, v.w};
  }
  float xr[kChunks][8];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) unpack_bf16x8(raw[c], xr[c]);

  if constexpr (kModulate) {
    double sum = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += (double)xr[c][i];   // padding lanes hold zeros
    const float mean = (float)(wave_sum(sum) / (double)K);
    double ssq = 0.0;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const bool valid = c * 64 + lane < nch;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        xr[c][i] = xr[c][i] - mean;
        if (valid) ssq += (double)(xr[c][i] * xr[c][i]);
      }
    }
    const float var = (float)(wave_sum(ssq) / (double)K);
    const float inv = 1.0f / sqrtf(var + 1e-6f);
    const int b = row / tokens_per_batch;
    const uint16_t* sh = shift + (int64_t)b * mod_stride;
    const uint16_t* sc = scale + (int64_t)b * mod_stride;
    uint16_t* xm = x_mod ? x_mod + (int64_t)row * x_mod_stride : nullptr;
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      const int idx = c * 64 + lane;
      if (idx >= nch) continue;
      float sf[8], tf[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(sh + idx * 8), sf);
      unpack_bf16x8(*reinterpret_cast<const uint4*>(sc + idx * 8), tf);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float base = flk::round_bf16(xr[c][i] * inv);
        const float one_plus = flk::round_bf16(1.0f + tf[i]);
        xr[c][i] = flk::round_bf16(flk::round_bf16(one_plus * base) + sf[i]);
      }
      if (xm)
        *reinterpret_cast<uint4*>(xm + idx * 8) =
            uint4{flk::pack_bf16x2(xr[c][0], xr[c][1]), flk::pack_bf16x2(xr[c][2], xr[c][3]),
                  flk::pack_bf16x2(xr[c][4], xr[c][5]), flk::pack_bf16x2(xr[c][6], xr[c][7])};
    }
  }

  float xh[kChunks][8];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int idx = c * 64 + lane;
    const f32x4 s0 = idx < nch ? reinterpret_cast<const f32x4*>(inv_s)[2 * idx] : f32x4{0, 0, 0, 0};
    const f32x4 s1 = idx < nch ? reinterpret_cast<const f32x4*>(inv_s)[2 * idx + 1] : f32x4{0, 0, 0, 0};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xh[c][i] = xr[c][i] * sv[i];
      amax = fmaxf(amax, fabsf(xh[c][i]));
    }
  }
  const float a = absmax_scale(wave_max(amax));
  const float ra = 1.0f / a;
  int8_t* dst = xq + (int64_t)row * K;
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int idx = c * 64 + lane;
    if (idx < nch) {
      auto qz = [&](float v) { return quantize_recip(v, a, ra); };
      uint2 packed;
      packed.x = pack_i8x4(qz(xh[c][0]), qz(xh[c][1]), qz(xh[c][2]), qz(xh[c][3]));
      packed.y = pack_i8x4(qz(xh[c][4]), qz(xh[c][5]), qz(xh[c][6]), qz(xh[c][7]));
      reinterpret_cast<uint2*>(dst)[idx] = packed;
    }
  }
  if (lane == 0) a_scale[row] = a;
}

// ---------------------------------------------------------------- GEMM -----------------

constexpr int kGT = 256;                 // tile edge: tokens and output channels
constexpr int kGK = 128;                 // k bytes per stage: one full 128-byte line per row
constexpr int kGHalf = kGT * kGK;        // one operand's stage: 32 KiB
constexpr int kGStage = 2 * kGHalf;      // WqT rows, then Xq rows; two stages fill 128 KiB
constexpr int kGWaves = 8;               // two waves per SIMD
constexpr int kGThreads = kGWaves * 64;
constexpr int kGWaveN = 128;             // a wave's output channels (8 fragments of 16)
constexpr int kGNF = kGWaveN / 16;       // channel fragments per wave
constexpr int kGCopies = kGT / kGWaves / 8;   // WqT copy instructions per wave and stage (4)
constexpr int kGT192 = 192;              // token edge of the tiles that re-tile a partial last round
constexpr int kGRing = 4;                // channel-fragment registers in flight
constexpr int kMaxDim = INT32_MAX - kGT;  // largest token / channel count: a tile past it stays within int
constexpr int kGLead = 3;                // groups between a channel fragment's read and its MFMAs
static_assert(kGNF % kGRing == 0 && kGRing > kGLead, "the fragment ring must divide the groups of a step");
#ifndef FLK_GEMM_GROUP
#define FLK_GEMM_GROUP 4
#endif
constexpr int kGroup = FLK_GEMM_GROUP;   // token tiles that sweep the channel tiles together
constexpr int kXcds = 8;
constexpr int kCUs = 256;                // MI355X compute units

// LDS slot of 16-byte chunk c in row r is c ^ gswz(r).  gfx950's LDS serves 256 B per clock
// from 64 banks, i.e. two 128-byte operand rows; a b128 read is served as lanes 0-7 with
// 32-39, 8-15 with 40-47, and so on.  An operand read takes rows r0 .. r0+15 (lane % 16) and
// chunks 4 ks + perm(lane / 16), perm = 0, 2, 1, 3: lanes l and l + 32 then read chunks c and
// c ^ 1 of the same 8 rows, which the swizzle spreads over the 16 slots of a bank line (as it
// does the 16 rows of lanes l .. l + 15).
__device__ __forceinline__ int gswz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ const uint8_t* a_frag(const uint8_t* stage, int nf, int wn) {
  return stage + (wn * kGWaveN + nf * 16) * kGK;
}
template <int kWaveM>
__device__ __forceinline__ const uint8_t* b_frag(const uint8_t* stage, int mf, int wm) {
  return stage + kGHalf + (wm * kWaveM + mf * 16) * kGK;
}

// The fused epilogue's qk_prep parameters (see flk_w8a8_qk_prep): output row m of the
// projection is token t = m % length of batch b = m / length, and its 128-channel head
// groups are q heads 0..H-1, then k heads, then v heads.
struct QkEpilogue {
  const float* cos;
  const float* sin;
  int64_t table_stride;
  const void* q_scale;
  const void* k_scale;
  float q_gain;
  int length, heads;
  uint16_t* out[3];
  int64_t out_length, out_offset;
};

// One projection Y = X W^T of a launch (xq M x K, wqt N x K), with its outputs.
struct GemmProblem {
  const int8_t* xq;
  const int8_t* wqt;
  const float* a_scale;
  const float* w_scale;
  uint16_t* y;            // plain epilogue: Y rows of y_stride elements
  int64_t y_stride;
  int32_t* acc_out;       // kAcc: the exact int32 products
  int M, K, N, tiles_m, tiles_n;
  QkEpilogue qe;          // kQk: qk_prep epilogue
};

// Up to two projections in one launch, so that a small one (a double block's 512 text
// tokens: 72 tiles) fills the CUs the large one (the image tokens) leaves idle in its last
// round.  Logical blocks [0, first_blocks) take p[0], the rest p[1].
struct GemmGroup {
  GemmProblem p[2];
  int first_blocks;
  int units;    // tiles of both problems (first_blocks + p[1]'s, or first_blocks alone)
  int rounds;   // rounds order (w8a8_gemm_kernel)
};

// One output tile: channels n0 .. n0 + 255 and tokens m0 .. m0 + 64 kMF - 1 (kMF = 4: 256
// tokens; 3: 192), of which tokens below m_limit are stored.  Each of the 2 (channels) x 4
// (tokens) waves holds 128 channels x 16 kMF tokens.  kAcc, kQk, kScaleF32 as for
// w8a8_gemm_kernel.
template <bool kAcc, bool kQk, bool kScaleF32, int kMF>
__device__ __forceinline__ void gemm_tile(uint8_t* smem, const GemmProblem& P, int m0, int n0, int m_limit) {
  constexpr int kWaveM = 16 * kMF;   // a wave's tokens
  constexpr int kBCopies = kMF;      // Xq copy instructions per wave and stage (8 kMF rows)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int8_t* __restrict__ xq = P.xq;
  const int8_t* __restrict__ wqt = P.wqt;
  const float* __restrict__ a_scale = P.a_scale;
  const float* __restrict__ w_scale = P.w_scale;
  uint16_t* __restrict__ y = P.y;
  const int64_t y_stride = P.y_stride;
  int32_t* __restrict__ acc_out = P.acc_out;
  const int M = P.M, K = P.K, N = P.N;
  const QkEpilogue& qe = P.qe;

  // Copy sources: this wave fills rows wave*32 .. +31 of WqT and wave*8kMF .. +8kMF-1 of Xq,
  // 8 rows (64 lanes x 16 B) per instruction; lane i lands at row i/8, slot i%8, and fetches
  // chunk slot^gswz.
  // Rows past the matrix edge repeat the last row (their results are never stored).  The
  // tile's first row (plus the stage's k offset) is a scalar base; lanes add 32-bit offsets.
  const int8_t* abase = wqt + (int64_t)n0 * K;
  const int8_t* bbase = xq + (int64_t)m0 * K;
  uint32_t aoff[kGCopies], boff[kBCopies];
#pragma unroll
  for (int i = 0; i < kGCopies; ++i) {
    const int row = wave * (kGT / kGWaves) + i * 8 + (lane >> 3);
    aoff[i] = (uint32_t)min(row, N - 1 - n0) * (uint32_t)K + (uint32_t)(((lane & 7) ^ gswz(row)) * 16);
  }
#pragma unroll
  for (int i = 0; i < kBCopies; ++i) {
    const int row = wave * 8 * kMF + i * 8 + (lane >> 3);
    boff[i] = (uint32_t)min(row, M - 1 - m0) * (uint32_t)K + (uint32_t)(((lane & 7) ^ gswz(row)) * 16);
  }
  uint8_t* const a_lds = smem + wave * (kGT / kGWaves) * kGK;   // this wave's WqT rows in stage 0
  uint8_t* const b_lds = smem + kGHalf + wave * 8 * kMF * kGK;  // ... and its Xq rows

  const int KT = K / kGK;
  const int wn = wave >> 2, wm = wave & 3;     // 2 (channels) x 4 (tokens) waves
  const int l16 = lane & 15, h4 = lane >> 4;
  const int hperm = ((h4 & 1) << 1) | (h4 >> 1);
  int off[2];   // fragment read offsets of k steps 0, 1: row l16, chunk 4 ks + perm(lane / 16)
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) off[ks] = l16 * kGK + (((4 * ks + hperm) ^ gswz(l16)) * 16);

  i32x4 acc[kGNF][kMF];
#pragma unroll
  for (int a = 0; a < kGNF; ++a)
#pragma unroll
    for (int b = 0; b < kMF; ++b) acc[a][b] = i32x4{};

  // Two stages of 128 k bytes, two 64-byte k steps each.  Stage kt: step 0 reads step 1's
  // fragments as it goes; step 1 reads its own last channel fragments in groups 0-4, then --
  // every wave done reading stage kt, stage kt+1 landed everywhere (the barrier) -- refills
  // stage kt's buffer with stage kt+2 and reads stage kt+1's first fragments in groups 5-7.
  // Past the last stage the copies repeat it (into the buffer no later step reads), so
  // every stage issues the same copies and vmcnt(0) is exact.
  const int k1 = min(1, KT - 1) * kGK;
  auto copy_stage = [&](int k_off, int buf) {   // WqT and Xq copies alternating
#pragma unroll
    for (int i = 0; i < kGCopies; ++i) {
      flk::dma16_at(abase + k_off, aoff[i], a_lds + buf * kGStage + i * 8 * kGK);
      if (i < kBCopies) flk::dma16_at(bbase + k_off, boff[i], b_lds + buf * kGStage + i * 8 * kGK);
    }
  };
  copy_stage(0, 0);
  copy_stage(k1, 1);
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kGCopies + kBCopies) : "memory");   // stage 0 landed
  __syncthreads();
  i32x4 ring[kGRing], b0[kMF], b1[kMF];
#pragma unroll
  for (int mf = 0; mf < kMF; ++mf) b0[mf] = *reinterpret_cast<const i32x4*>(b_frag<kWaveM>(smem, mf, wm) + off[0]);
#pragma unroll
  for (int nf = 0; nf < kGLead; ++nf) ring[nf] = *reinterpret_cast<const i32x4*>(a_frag(smem, nf, wn) + off[0]);

  auto mfma_group = [&](int nf, const i32x4 (&b)[kMF]) {
#pragma unroll
    for (int mf = 0; mf < kMF; ++mf)
      acc[nf][mf] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ring[nf % kGRing], b[mf], acc[nf][mf], 0, 0, 0);
  };
  auto afrag = [&](const uint8_t* st, int nf, int o) { return *reinterpret_cast<const i32x4*>(a_frag(st, nf, wn) + o); };
  auto bfrag = [&](const uint8_t* st, int mf, int o) { return *reinterpret_cast<const i32x4*>(b_frag<kWaveM>(st, mf, wm) + o); };

  for (int kt = 0; kt < KT; ++kt) {
    const uint8_t* cs = smem + (kt & 1) * kGStage;          // stage kt
    const uint8_t* ns = smem + ((kt + 1) & 1) * kGStage;    // stage kt+1
    const int k_next = min(kt + 2, KT - 1) * kGK;
    // step 0
#pragma unroll
    for (int nf = 0; nf < kGNF; ++nf) {
      mfma_group(nf, b0);
      const int nl = nf + kGLead;
      ring[nl % kGRing] = nl < kGNF ? afrag(cs, nl, off[0]) : afrag(cs, nl - kGNF, off[1]);
      if (nf < kMF) b1[nf] = bfrag(cs, nf, off[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // step 1, groups reading stage kt
#pragma unroll
    for (int nf = 0; nf < kGNF - kGLead; ++nf) {
      mfma_group(nf, b1);
      ring[(nf + kGLead) % kGRing] = afrag(cs, nf + kGLead, off[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");   // stage kt read, kt+1 landed
    copy_stage(k_next, kt & 1);
    // step 1, groups reading stage kt+1 (its step 0 fragments)
#pragma unroll
    for (int nf = kGNF - kGLead; nf < kGNF; ++nf) {
      mfma_group(nf, b1);
      ring[(nf + kGLead) % kGRing] = afrag(ns, nf + kGLead - kGNF, off[0]);
      const int j = nf - (kGNF - kGLead);           // 0, 1, 2
      if constexpr (kMF == 4) {                     // token fragments 0-1, 2, 3
        if (j == 0) {
          b0[0] = bfrag(ns, 0, off[0]);
          b0[1] = bfrag(ns, 1, off[0]);
        } else {
          b0[j + 1] = bfrag(ns, j + 1, off[0]);
        }
      } else {                                      // token fragments 0, 1, 2
        b0[j] = bfrag(ns, j, off[0]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (kAcc) {
    // Exact int32 products, straight from the accumulators: the lane owns token l16 and
    // channels 4 * (lane / 16) .. +3 of each 16 x 16 fragment.
#pragma unroll
    for (int nf = 0; nf < kGNF; ++nf) {
      const int n = n0 + wn * kGWaveN + nf * 16 + h4 * 4;
#pragma unroll
      for (int mf = 0; mf < kMF; ++mf) {
        const int m = m0 + wm * kWaveM + mf * 16 + l16;
        if (n < N && m < m_limit) *reinterpret_cast<i32x4*>(acc_out + (int64_t)m * N + n) = acc[nf][mf];
      }
    }
  }

  // Epilogue.  The lane owns token m = mf*16 + l16 and channels n = nf*16 + 4 h4 .. +3 of the
  // wave's 128 x 64 sub-tile.  Rescaled bf16 values go to this wave's 16 KiB of the (now
  // idle) LDS as [m][n] rows of 256 B whose 16-byte chunks are XOR-swizzled by m & 15; then
  // the wave reads back 4 rows per instruction (16 lanes x 16 B per row) and writes each
  // row's 256 contiguous bytes with 16-byte nontemporal stores (Y is streamed out: 1-2%
  // faster, and a qk_prep pass reading Y next measured no slower).
  float am[kMF];
#pragma unroll
  for (int mf = 0; mf < kMF; ++mf) am[mf] = a_scale[min(m0 + wm * kWaveM + mf * 16 + l16, M - 1)];
  __syncthreads();   // every wave is done reading the operand stages
  uint8_t* const out_lds = smem + wave * (kWaveM * 256);
#pragma unroll
  for (int nf = 0; nf < kGNF; ++nf) {
    // w_o of the lane's 4 channels (clamped at the edge; clamped values are never stored)
    const f32x4 w4 = *reinterpret_cast<const f32x4*>(w_scale + min(n0 + wn * kGWaveN + nf * 16 + h4 * 4, N - 4));
#pragma unroll
    for (int mf = 0; mf < kMF; ++mf) {
      const int ml = mf * 16 + l16;
      const float y0 = ((float)acc[nf][mf][0] * am[mf]) * w4.x;
      const float y1 = ((float)acc[nf][mf][1] * am[mf]) * w4.y;
      const float y2 = ((float)acc[nf][mf][2] * am[mf]) * w4.z;
      const float y3 = ((float)acc[nf][mf][3] * am[mf]) * w4.w;
      uint2 packed;
      packed.x = flk::pack_bf16x2(y0, y1);
      packed.y = flk::pack_bf16x2(y2, y3);
      const int chunk = (nf * 2 + (h4 >> 1)) ^ (ml & 15);
      *reinterpret_cast<uint2*>(out_lds + ml * 256 + chunk * 16 + (h4 & 1) * 8) = packed;
    }
  }
  // Each wave reads back only what it wrote itself: its LDS writes complete in order before
  // its reads (the compiler waits on lgkmcnt), so no barrier is needed here.
  constexpr int kReads = kWaveM / 4;
  const int n_lane = n0 + wn * kGWaveN + (lane & 15) * 8;
  if constexpr (kQk) {
    // The wave's 128 channels are one head of the q|k|v thirds (N = 3 H 128, tiles 128-aligned);
    // each 16-lane row of a read-back is one token's finished bf16 head row -- the input of
    // qk_prep, rounded exactly as the unfused path stores it in Y.
    const int head_g = (n0 + wn * kGWaveN) / flk::kQkHeadDim;
    if (n0 + wn * kGWaveN >= N) return;
    const int sec = head_g / qe.heads, h = head_g - sec * qe.heads;
    const int l16 = lane & 15;
    float sc[8];
    if (sec < 2) flk::load_scale8<kScaleF32>(sec == 0 ? qe.q_scale : qe.k_scale, l16, sc);
    uint16_t* const out = qe.out[sec];
    // Row m = b * length + t.  One division for the lane's first row; each read-back moves 4
    // rows on, which wraps into the next batch entry at most once when length >= 4 (shorter
    // sequences divide per row).  A division per row measured 2.4% of the fused kernel.
    const int len = qe.length;
    const bool short_seq = len < 4;
    const int m_first = m0 + wm * kWaveM + (lane >> 4);
    int b = m_first / len, t = m_first - b * len;
#pragma unroll 4
    for (int it = 0; it < kReads; ++it) {
      const int ml = it * 4 + (lane >> 4);
      const int m = m0 + wm * kWaveM + ml;
      if (it > 0) {
        if (short_seq) {
          b = m / len;
          t = m - b * len;
        } else {
          t += 4;
          if (t >= len) {
            t -= len;
            ++b;
          }
        }
      }
      const uint4 v = *reinterpret_cast<const uint4*>(out_lds + ml * 256 + ((l16 ^ (ml & 15)) * 16));
      if (m >= m_limit) continue;   // uniform over the 16-lane row, so the DPP rows stay whole
      uint4 r = v;
      if (sec < 2) {
        float c[8], s[8];
        flk::load_table8(qe.cos + (int64_t)t * qe.table_stride, l16, c);
        flk::load_table8(qe.sin + (int64_t)t * qe.table_stride, l16, s);
        r = sec == 0 ? flk::norm_rotate<kScaleF32, true>(v, sc, c, s, qe.q_gain)
                     : flk::norm_rotate<kScaleF32, false>(v, sc, c, s, 1.0f);
      }
      const int64_t o = (((int64_t)b * qe.heads + h) * qe.out_length + qe.out_offset + t) * flk::kQkHeadDim + l16 * 8;
      *reinterpret_cast<uint4*>(out + o) = r;
    }
    return;
  }
  const bool wide = (y_stride & 7) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;   // 16-byte rows
#pragma unroll 8
  for (int it = 0; it < kReads; ++it) {
    const int ml = it * 4 + (lane >> 4);
    const uint4 v = *reinterpret_cast<const uint4*>(out_lds + ml * 256 + (((lane & 15) ^ (ml & 15)) * 16));
    const int m = m0 + wm * kWaveM + ml;
    if (m < m_limit && n_lane < N) {
      uint16_t* dst = y + (int64_t)m * y_stride + n_lane;
      if (wide && n_lane + 8 <= N) {
        __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(dst));
      } else {
        *reinterpret_cast<uint2*>(dst) = uint2{v.x, v.y};
        if (n_lane + 8 <= N) *reinterpret_cast<uint2*>(dst + 4) = uint2{v.z, v.w};
      }
    }
  }
}

// Logical tile u of a problem -> its token and channel tiles: kGroup token tiles sweep the
// channel tiles together (consecutive logical tiles share a channel tile's WqT rows).
__device__ __forceinline__ void tile_of(int u, int tiles_m, int tiles_n, int& mt, int& nt) {
  const int group_tiles = kGroup * tiles_n;
  const int group = u / group_tiles;
  const int first_m = group * kGroup;
  const int gm = min(kGroup, tiles_m - first_m);
  const int in_group = u - group * group_tiles;
  mt = first_m + in_group % gm;
  nt = in_group / gm;
}

// The rounds order's 192-token tiles: logical tiles [first, end) of a launch's problems (p[0]'s
// tiles, then p[1]'s) taken as runs of one channel tile (consecutive token tiles of one group
// of one problem), each run's tokens cut into 192-token tiles, the last one short.  The j-th
// such tile, or false past the last.  The host's gemm_rounds_grid counts them the same way.
__device__ __forceinline__ bool leftover_tile(const GemmGroup& grp, int first, int end, int j, int& second, int& m0,
                                              int& n0, int& m_end) {
  for (int u = first; u < end;) {
    second = u >= grp.first_blocks;
    const GemmProblem& P = second ? grp.p[1] : grp.p[0];
    const int base = second ? grp.first_blocks : 0;
    const int p_end = second ? end : min(end, grp.first_blocks);
    const int group_tiles = kGroup * P.tiles_n;
    const int group = (u - base) / group_tiles;
    const int first_m = group * kGroup;
    const int gm = min(kGroup, P.tiles_m - first_m);
    const int in_group = u - base - group * group_tiles;
    const int r = in_group % gm;
    const int run = min(gm - r, p_end - u);
    const int s = (first_m + r) * kGT, e = min((first_m + r + run) * kGT, P.M);
    const int count = (e - s + kGT192 - 1) / kGT192;
    if (j < count) {
      m0 = s + j * kGT192;
      m_end = min(m0 + kGT192, e);
      n0 = (in_group / gm) * kGT;
      return true;
    }
    j -= count;
    u += run;
  }
  return false;
}

// kAcc: also write the exact int32 products (a test and debugging path).
// kQk: instead of Y, run qk_prep on each finished bf16 head row (kScaleF32: float32 norm
// scales) and write head-major q, k, v.
template <bool kAcc, bool kQk = false, bool kScaleF32 = false>
__global__ __launch_bounds__(kGThreads, 2) void w8a8_gemm_kernel(const GemmGroup grp) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * kGStage];
  const int xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;   // blocks are dealt round-robin over XCDs
  if (grp.rounds) {
    // Rounds order: each XCD takes a contiguous range of the logical tiles (of one problem,
    // then the next), runs whole rounds of 32 of them, and cuts the ones left over into
    // 192-token tiles, so the partial last round has up to 4/3 as many blocks with 3/4 of the
    // work each.
    constexpr int C = kCUs / kXcds;
    const int ux0 = (int)((int64_t)xcd * grp.units / kXcds);
    const int n = (int)((int64_t)(xcd + 1) * grp.units / kXcds) - ux0;
    const int full = n / C * C;
    if (local < full) {
      const int u = ux0 + local;
      const bool second = u >= grp.first_blocks;
      const GemmProblem& P = second ? grp.p[1] : grp.p[0];
      int mt, nt;
      tile_of(u - (second ? grp.first_blocks : 0), P.tiles_m, P.tiles_n, mt, nt);
      gemm_tile<kAcc, kQk, kScaleF32, 4>(smem, P, mt * kGT, nt * kGT, P.M);
      return;
    }
    int second, m0, n0, m_end;
    if (!leftover_tile(grp, ux0 + full, ux0 + n, local - full, second, m0, n0, m_end)) return;
    gemm_tile<kAcc, kQk, kScaleF32, 3>(smem, second ? grp.p[1] : grp.p[0], m0, n0, m_end);
    return;
  }
  // Tile order: renumber so that each XCD runs a contiguous range of logical tiles (of one
  // problem, then the next).
  const int nblocks = gridDim.x;
  const int per = nblocks / kXcds, extra = nblocks % kXcds;
  const int logical_all = xcd * per + min(xcd, extra) + local;
  const bool second = logical_all >= grp.first_blocks;
  const GemmProblem& P = second ? grp.p[1] : grp.p[0];   // wave-uniform, read from the kernel arguments
  int mt, nt;
  tile_of(logical_all - (second ? grp.first_blocks : 0), P.tiles_m, P.tiles_n, mt, nt);
  gemm_tile<kAcc, kQk, kScaleF32, 4>(smem, P, mt * kGT, nt * kGT, P.M);
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" int flk_absmax_rows(const void* x, int64_t rows, int64_t cols, int64_t row_stride, float* out,
                               void* stream) {
  if (rows < 0 || cols < 0 || row_stride < cols) return FLK_E_INVALID;
  if (rows == 0) return FLK_OK;
  if (!x || !out || cols == 0) return FLK_E_INVALID;
  if (cols % 8 || row_stride % 8 || !flk_host_aligned(x, 16) || !flk_host_aligned(out, 4)) return FLK_E_ALIGN;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(absmax_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(x), rows, cols, row_stride, out);
  return flk_launch_status();
}

extern "C" int flk_absmax_cols(const void* x, int64_t rows, int64_t cols, int64_t row_stride, int accumulate,
                               float* out, void* stream) {
  if (rows < 0 || cols < 0 || row_stride < cols) return FLK_E_INVALID;
  if (cols == 0 || (rows == 0 && accumulate)) return FLK_OK;
  if (!out || (rows > 0 && !x)) return FLK_E_INVALID;
  if (cols % 8 || row_stride % 8 || (x && !flk_host_aligned(x, 16)) || !flk_host_aligned(out, 4))
    return FLK_E_ALIGN;
  const int64_t blocks = (cols + 127) / 128;
  if (blocks > INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(absmax_cols_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(x), rows, cols, row_stride, accumulate, out);
  return flk_launch_status();
}

extern "C" int flk_smooth_factors(const float* x_absmax, const float* w_absmax, int64_t k, float* s,
                                  float* inv_s, void* stream) {
  if (k < 0) return FLK_E_INVALID;
  if (k == 0) return FLK_OK;
  if (!x_absmax || !w_absmax || !s || !inv_s) return FLK_E_INVALID;
  const int64_t blocks = (k + 255) / 256;
  if (blocks > INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(smooth_factors_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), x_absmax,
                     w_absmax, k, s, inv_s);
  return flk_launch_status();
}

extern "C" int flk_quantize_weight(const void* w, int64_t w_row_stride, const float* s, int k, int n,
                                   int8_t* wq_t, float* w_scale, void* stream) {
  if (k < 0 || n < 0 || w_row_stride < n) return FLK_E_INVALID;
  if (k == 0 || n == 0) return FLK_OK;
  if (k > INT32_MAX - 64 || n > INT32_MAX - 64) return FLK_E_INVALID;   // a block's last row / column index
  if (!w || !s || !wq_t || !w_scale) return FLK_E_INVALID;
  if (k % 64 || n % 8 || w_row_stride % 8) return FLK_E_UNSUPPORTED;
  if (!flk_host_aligned(w, 16) || !flk_host_aligned(wq_t, 16) || !flk_host_aligned(s, 4) ||
      !flk_host_aligned(w_scale, 4))
    return FLK_E_ALIGN;
  hipLaunchKernelGGL(quantize_weight_kernel, dim3((unsigned)((n + 63) / 64)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(w), w_row_stride, s, k, n, wq_t, w_scale);
  return flk_launch_status();
}

namespace {

template <bool kModulate>
int launch_quantize_act(const QuantGroup& g, int64_t blocks, void* stream) {
  if (blocks > INT32_MAX) return FLK_E_INVALID;
  const int chunks = (g.K / 8 + 63) / 64;
  const dim3 grid((unsigned)blocks), block(256);
  const hipStream_t st = as_stream(stream);
#define FLK_QA(C) hipLaunchKernelGGL((quantize_act_kernel<C, kModulate>), grid, block, 0, st, g)
  if (chunks <= 1) FLK_QA(1);
  else if (chunks <= 2) FLK_QA(2);
  else if (chunks <= 4) FLK_QA(4);
  else if (chunks <= 6) FLK_QA(6);
  else if (chunks <= 8) FLK_QA(8);
  else if (chunks <= 12) FLK_QA(12);
  else FLK_QA(16);
#undef FLK_QA
  return flk_launch_status();
}

// Status of a checked problem with nothing to launch (empty input).
constexpr int kNoWork = 1;

// Checks one modulated activation (flk_quantize_act_modulated's arguments) and fills its
// problem: FLK_OK, kNoWork, or an error status.
int modulated_problem(const void* x, int64_t x_row_stride, const void* shift, const void* scale,
                      int64_t mod_batch_stride, int tokens_per_batch, const float* inv_s, int m, int k, int8_t* xq,
                      float* a_scale, void* x_mod, int64_t x_mod_row_stride, QuantProblem& p) {
  if (m < 0 || k < 0 || x_row_stride < k || mod_batch_stride < 0 || (x_mod && x_mod_row_stride < k))
    return FLK_E_INVALID;
  if (m == 0 || k == 0) return kNoWork;   // an empty input (its sequence length may be 0 too)
  if (tokens_per_batch <= 0 || m > INT32_MAX - 4) return FLK_E_INVALID;
  if (!x || !shift || !scale || !inv_s || !xq || !a_scale) return FLK_E_INVALID;
  if ((m - 1) / tokens_per_batch > 0 && mod_batch_stride < k) return FLK_E_INVALID;
  if (k % 8 || k > 8192) return FLK_E_UNSUPPORTED;
  if (x_row_stride % 8 || mod_batch_stride % 8 || !flk_host_aligned(x, 16) || !flk_host_aligned(shift, 16) ||
      !flk_host_aligned(scale, 16) || !flk_host_aligned(inv_s, 16) || !flk_host_aligned(xq, 8) ||
      !flk_host_aligned(a_scale, 4) || (x_mod && (!flk_host_aligned(x_mod, 16) || x_mod_row_stride % 8)))
    return FLK_E_ALIGN;
  p = QuantProblem{static_cast<const uint16_t*>(x), x_row_stride, inv_s, m, xq, a_scale,
                   static_cast<const uint16_t*>(shift), static_cast<const uint16_t*>(scale), mod_batch_stride,
                   tokens_per_batch, static_cast<uint16_t*>(x_mod), x_mod_row_stride};
  return FLK_OK;
}

int64_t row_blocks(const QuantProblem& p) { return ((int64_t)p.M + 3) / 4; }

}  // namespace

extern "C" int flk_quantize_act(const void* x, int64_t x_row_stride, const float* inv_s, int m, int k,
                                int8_t* xq, float* a_scale, void* stream) {
  if (m < 0 || k < 0 || x_row_stride < k) return FLK_E_INVALID;
  if (m == 0 || k == 0) return FLK_OK;
  if (m > INT32_MAX - 4) return FLK_E_INVALID;   // the last block's row index
  if (!x || !inv_s || !xq || !a_scale) return FLK_E_INVALID;
  if (k % 8 || k > 8192) return FLK_E_UNSUPPORTED;
  if (x_row_stride % 8 || !flk_host_aligned(x, 16) || !flk_host_aligned(inv_s, 16) || !flk_host_aligned(xq, 8) ||
      !flk_host_aligned(a_scale, 4))
    return FLK_E_ALIGN;
  const QuantProblem p{static_cast<const uint16_t*>(x), x_row_stride, inv_s, m, xq, a_scale, nullptr, nullptr, 0, 1,
                       nullptr, 0};
  const int64_t blocks = row_blocks(p);
  return launch_quantize_act<false>(QuantGroup{{p, p}, (int)std::min<int64_t>(blocks, INT32_MAX), k}, blocks,
                                    stream);
}

extern "C" int flk_quantize_act_modulated(const void* x, int64_t x_row_stride, const void* shift,
                                          const void* scale, int64_t mod_batch_stride, int tokens_per_batch,
                                          const float* inv_s, int m, int k, int8_t* xq, float* a_scale,
                                          void* x_mod, int64_t x_mod_row_stride, void* stream) {
  QuantProblem p{};
  const int st = modulated_problem(x, x_row_stride, shift, scale, mod_batch_stride, tokens_per_batch, inv_s, m, k,
                                   xq, a_scale, x_mod, x_mod_row_stride, p);
  if (st != FLK_OK) return st == kNoWork ? FLK_OK : st;
  const int64_t blocks = row_blocks(p);
  return launch_quantize_act<true>(QuantGroup{{p, p}, (int)std::min<int64_t>(blocks, INT32_MAX), k}, blocks,
                                   stream);
}

extern "C" int flk_quantize_act_modulated_pair(
    const void* x0, int64_t x_row_stride0, const void* shift0, const void* scale0, int64_t mod_batch_stride0,
    int tokens_per_batch0, const float* inv_s0, int m0, int8_t* xq0, float* a_scale0, void* x_mod0,
    int64_t x_mod_row_stride0,
    const void* x1, int64_t x_row_stride1, const void* shift1, const void* scale1, int64_t mod_batch_stride1,
    int tokens_per_batch1, const float* inv_s1, int m1, int8_t* xq1, float* a_scale1, void* x_mod1,
    int64_t x_mod_row_stride1, int k, void* stream) {
  QuantGroup g{};
  g.K = k;
  const int st0 = modulated_problem(x0, x_row_stride0, shift0, scale0, mod_batch_stride0, tokens_per_batch0, inv_s0,
                                    m0, k, xq0, a_scale0, x_mod0, x_mod_row_stride0, g.p[0]);
  if (st0 != FLK_OK && st0 != kNoWork) return st0;
  const int st1 = modulated_problem(x1, x_row_stride1, shift1, scale1, mod_batch_stride1, tokens_per_batch1, inv_s1,
                                    m1, k, xq1, a_scale1, x_mod1, x_mod_row_stride1, g.p[1]);
  if (st1 != FLK_OK && st1 != kNoWork) return st1;
  if (st0 == kNoWork && st1 == kNoWork) return FLK_OK;
  // An empty problem gives its place to the other one, which then takes every block.
  if (st0 == kNoWork) g.p[0] = g.p[1];
  if (st1 == kNoWork) g.p[1] = g.p[0];
  const bool both = st0 == FLK_OK && st1 == FLK_OK;
  const int64_t b0 = row_blocks(g.p[0]);
  const int64_t blocks = both ? b0 + row_blocks(g.p[1]) : b0;
  g.first_blocks = (int)std::min<int64_t>(b0, INT32_MAX);
  return launch_quantize_act<true>(g, blocks, stream);
}

namespace {

int64_t problem_blocks(const GemmProblem& p) { return (int64_t)p.tiles_m * p.tiles_n; }

// Grid of the rounds order of a launch (w8a8_gemm_kernel), or 0 when it is not the choice: it
// needs a full round of 32 tiles on every XCD, tiles left over, and at most one round of
// 192-token tiles for them (counted as leftover_tile walks them).
int64_t gemm_rounds_grid(const GemmGroup& g) {
  constexpr int C = kCUs / kXcds;
  const int64_t units = g.units;
  if (units < kCUs) return 0;
  int64_t most = 0, left_max = 0;
  for (int x = 0; x < kXcds; ++x) {
    const int64_t ux0 = x * units / kXcds, n = (x + 1) * units / kXcds - ux0;
    const int64_t full = n / C * C;
    int64_t count = 0;
    for (int64_t u = ux0 + full; u < ux0 + n;) {
      const bool second = u >= g.first_blocks;
      const GemmProblem& p = second ? g.p[1] : g.p[0];
      const int64_t base = second ? g.first_blocks : 0;
      const int64_t p_end = second ? ux0 + n : std::min<int64_t>(ux0 + n, g.first_blocks);
      const int64_t group_tiles = (int64_t)kGroup * p.tiles_n;
      const int64_t group = (u - base) / group_tiles, first_m = group * kGroup;
      const int64_t gm = std::min<int64_t>(kGroup, p.tiles_m - first_m);
      const int64_t r = (u - base - group * group_tiles) % gm;
      const int64_t run = std::min(gm - r, p_end - u);
      const int64_t e = std::min<int64_t>((first_m + r + run) * kGT, p.M);
      count += (e - (first_m + r) * kGT + kGT192 - 1) / kGT192;
      u += run;
    }
    if (count > C) return 0;
    left_max = std::max(left_max, n - full);
    most = std::max(most, full + count);
  }
  return left_max > 0 ? most * kXcds : 0;
}

// Fills a launch's tile count and order; returns its grid.
int64_t plan_group(GemmGroup& g, int64_t units) {
  g.units = (int)std::min<int64_t>(units, INT32_MAX);
  const int64_t rounds = units <= INT32_MAX ? gemm_rounds_grid(g) : 0;
  g.rounds = rounds > 0;
  return rounds ? rounds : units;
}

template <bool kAcc, bool kQk, bool kScaleF32>
int launch_group(const GemmGroup& g, int64_t blocks, void* stream) {
  if (blocks > INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL((w8a8_gemm_kernel<kAcc, kQk, kScaleF32>), dim3((unsigned)blocks), dim3(kGThreads), 0,
                     as_stream(stream), g);
  return flk_launch_status();
}

// Checks one fused projection + qk_prep (flk_w8a8_qk_prep's arguments) and fills its
// problem.  FLK_OK = launch, kNoWork = empty (nothing to launch), else an error status.

int qk_problem(const int8_t* xq, const int8_t* wq_t, const float* a_scale, const float* w_scale, int k,
               const float* cos, const float* sin, int64_t table_row_stride, const void* q_scale,
               const void* k_scale, float q_gain, int batch, int length, int num_heads, int head_dim,
               void* q_out, void* k_out, void* v_out, int64_t out_length, int64_t out_offset, GemmProblem& p) {
  if (head_dim != flk::kQkHeadDim) return FLK_E_UNSUPPORTED;
  if (batch < 0 || length < 0 || num_heads <= 0 || k < 0 || out_offset < 0 || out_offset + length > out_length)
    return FLK_E_INVALID;
  if (batch == 0 || length == 0) return kNoWork;
  if (!xq || !wq_t || !a_scale || !w_scale || !cos || !sin || !q_scale || !k_scale || !q_out || !k_out ||
      !v_out || k == 0 || table_row_stride < head_dim)
    return FLK_E_INVALID;
  if (k % 128) return FLK_E_UNSUPPORTED;
  if ((int64_t)k * 127 * 127 > INT32_MAX) return FLK_E_UNSUPPORTED;
  const int64_t m64 = (int64_t)batch * length, n = 3LL * num_heads * head_dim;
  if (m64 > kMaxDim || n > kMaxDim) return FLK_E_INVALID;
  if (!flk_host_aligned(xq, 16) || !flk_host_aligned(wq_t, 16) || !flk_host_aligned(w_scale, 16) ||
      !flk_host_aligned(a_scale, 4) || !flk_host_aligned(cos, 16) || !flk_host_aligned(sin, 16) ||
      table_row_stride % 4 || !flk_host_aligned(q_scale, 16) || !flk_host_aligned(k_scale, 16) ||
      !flk_host_aligned(q_out, 16) || !flk_host_aligned(k_out, 16) || !flk_host_aligned(v_out, 16))
    return FLK_E_ALIGN;
  p = GemmProblem{};
  p.xq = xq;
  p.wqt = wq_t;
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.M = (int)m64;
  p.K = k;
  p.N = (int)n;
  p.tiles_m = (p.M + kGT - 1) / kGT;
  p.tiles_n = (p.N + kGT - 1) / kGT;
  p.qe = QkEpilogue{cos, sin, table_row_stride, q_scale, k_scale, q_gain, length, num_heads,
                    {static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out)},
                    out_length, out_offset};
  return FLK_OK;
}

int launch_qk(const GemmGroup& g, int64_t blocks, int scale_is_f32, void* stream) {
  return scale_is_f32 ? launch_group<false, true, true>(g, blocks, stream)
                      : launch_group<false, true, false>(g, blocks, stream);
}

}  // namespace

extern "C" int flk_w8a8_gemm(const int8_t* xq, const int8_t* wq_t, const float* a_scale, const float* w_scale,
                             int m, int k, int n, void* y, int64_t y_row_stride, int32_t* acc_or_null,
                             void* stream) {
  if (m < 0 || k < 0 || n < 0 || y_row_stride < n) return FLK_E_INVALID;
  if (m == 0 || n == 0) return FLK_OK;
  if (m > kMaxDim || n > kMaxDim) return FLK_E_INVALID;
  if (!xq || !wq_t || !a_scale || !w_scale || !y || k == 0) return FLK_E_INVALID;
  if (k % 128 || n % 4) return FLK_E_UNSUPPORTED;
  if ((int64_t)k * 127 * 127 > INT32_MAX) return FLK_E_UNSUPPORTED;   // int32 accumulation must be exact
  if (!flk_host_aligned(xq, 16) || !flk_host_aligned(wq_t, 16) || !flk_host_aligned(w_scale, 16) ||
      !flk_host_aligned(a_scale, 4) || !flk_host_aligned(y, 8) || y_row_stride % 4 ||
      (acc_or_null && !flk_host_aligned(acc_or_null, 16)))
    return FLK_E_ALIGN;
  GemmGroup g{};
  GemmProblem& p = g.p[0];
  p.xq = xq;
  p.wqt = wq_t;
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.y = static_cast<uint16_t*>(y);
  p.y_stride = y_row_stride;
  p.acc_out = acc_or_null;
  p.M = m;
  p.K = k;
  p.N = n;
  p.tiles_m = (m + kGT - 1) / kGT;
  p.tiles_n = (n + kGT - 1) / kGT;
  g.p[1] = p;
  g.first_blocks = (int)std::min<int64_t>(problem_blocks(p), INT32_MAX);
  const int64_t blocks = plan_group(g, problem_blocks(p));
  return acc_or_null ? launch_group<true, false, false>(g, blocks, stream)
                     : launch_group<false, false, false>(g, blocks, stream);
}

extern "C" int flk_w8a8_qk_prep(const int8_t* xq, const int8_t* wq_t, const float* a_scale, const float* w_scale,
                                int k, const float* cos, const float* sin, int64_t table_row_stride,
                                const void* q_scale, const void* k_scale, int scale_is_f32, float q_gain, int batch,
                                int length, int num_heads, int head_dim, void* q_out, void* k_out, void* v_out,
                                int64_t out_length, int64_t out_offset, void* stream) {
  GemmGroup g{};
  const int st = qk_problem(xq, wq_t, a_scale, w_scale, k, cos, sin, table_row_stride, q_scale, k_scale, q_gain,
                            batch, length, num_heads, head_dim, q_out, k_out, v_out, out_length, out_offset, g.p[0]);
  if (st != FLK_OK) return st == kNoWork ? FLK_OK : st;
  g.p[1] = g.p[0];
  g.first_blocks = (int)std::min<int64_t>(problem_blocks(g.p[0]), INT32_MAX);
  const int64_t blocks = plan_group(g, problem_blocks(g.p[0]));
  return launch_qk(g, blocks, scale_is_f32, stream);
}

extern "C" int flk_w8a8_qk_prep_pair(
    const int8_t* xq0, const int8_t* wq_t0, const float* a_scale0, const float* w_scale0, const float* cos0,
    const float* sin0, const void* q_scale0, const void* k_scale0, int length0, int64_t out_offset0,
    const int8_t* xq1, const int8_t* wq_t1, const float* a_scale1, const float* w_scale1, const float* cos1,
    const float* sin1, const void* q_scale1, const void* k_scale1, int length1, int64_t out_offset1, int k,
    int64_t table_row_stride, int scale_is_f32, float q_gain, int batch, int num_heads, int head_dim, void* q_out,
    void* k_out, void* v_out, int64_t out_length, void* stream) {
  GemmGroup g{};
  const int st0 = qk_problem(xq0, wq_t0, a_scale0, w_scale0, k, cos0, sin0, table_row_stride, q_scale0, k_scale0,
                             q_gain, batch, length0, num_heads, head_dim, q_out, k_out, v_out, out_length,
                             out_offset0, g.p[0]);
  if (st0 != FLK_OK && st0 != kNoWork) return st0;
  const int st1 = qk_problem(xq1, wq_t1, a_scale1, w_scale1, k, cos1, sin1, table_row_stride, q_scale1, k_scale1,
                             q_gain, batch, length1, num_heads, head_dim, q_out, k_out, v_out, out_length,
                             out_offset1, g.p[1]);
  if (st1 != FLK_OK && st1 != kNoWork) return st1;
  if (st0 == kNoWork && st1 == kNoWork) return FLK_OK;
  // An empty problem gives its place to the other one, which then takes every block.
  if (st0 == kNoWork) g.p[0] = g.p[1];
  if (st1 == kNoWork) g.p[1] = g.p[0];
  const bool both = st0 == FLK_OK && st1 == FLK_OK;
  const int64_t b0 = problem_blocks(g.p[0]);
  g.first_blocks = (int)std::min<int64_t>(b0, INT32_MAX);
  const int64_t blocks = plan_group(g, both ? b0 + problem_blocks(g.p[1]) : b0);
  return launch_qk(g, blocks, scale_is_f32, stream);
}
