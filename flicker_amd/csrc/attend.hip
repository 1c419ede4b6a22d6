// attend: bounded flash attention on gfx950 bf16 MFMA.
//
// Semantics follow the reference kernel (src/flicker/kernels.py:105-145): for each
// (b, h) and query i, over key tiles in order,
//   S = q_i . k_j  (bf16 operands, f32 accumulate)     -- q arrives scaled by 1/sqrt(D)
//   P = bf16(exp(S))                                  -- no running max: QK-norm bounds S
//   l += f32(P);  acc += P * v_j                       (f32)
//   o_i = bf16(acc / l)
//
// Formulation.  Each wave owns 64 queries (two 32-query column blocks) and computes the
// transposed score tile S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = K rows from LDS,
// B = Q^T held in registers for the whole kernel).  In the 32x32 accumulator layout a
// lane owns one query column and 16 key rows, so
//   * exp / bf16 rounding / the row sum l are lane-local (l is reduced across the two
//     lane halves once, in the epilogue), and
//   * the rounded P registers are directly the B operand (keys x queries) of the second
//     product O^T += V^T P^T -- no shuffle of P through LDS.
// Every LDS operand read feeds two MFMAs (one per query block).  V stays row-major in
// LDS; its transposed operand (d rows x 8 keys per lane) is fetched with two
// ds_read_b64_tr_b16, whose 16-lane transpose hands lane 4a+b element b of source lanes
// a, a+4, a+8, a+12 -- so source lane s points at key K0 + s/4, columns D0 + 4(s%4).
// The 8 keys a lane receives follow the accumulator-row order of S^T, so the P
// registers of lane half g line up with the V^T k-slots of the same half.
//
// Staging.  K and V tiles (64 keys x 256 B each) go from global memory straight into
// LDS with global_load_lds_dwordx4 (no registers): lane i of a wave instruction lands
// at base + 16 i, so the XOR swizzle is applied by choosing which global chunk each
// lane fetches.  Both tiles use chunk' = chunk ^ swz(row), swz = ((row&3)<<1)|((row>>2)&1),
// which keeps every 8 consecutive K rows (b128 operand reads) and every group of 4 V
// rows x 2 chunks (transpose reads) on distinct banks of the 32-bank LDS.
//
// Pipeline.  A block of 8 waves (two per SIMD, 32 queries each) streams 64-key tiles,
// two 32-key units per tile.  In the phase of unit u the wave
// first issues all 16 LDS operand reads, then alternates each QK^T MFMA of unit u+1
// with the exp / bf16 / row-sum VALU work of two elements of unit u (explicit schedule
// fences keep that interleave), then runs the 16 PV MFMAs of unit u.  Tiles stream
// through a 4-buffer ring: the copy of tile t+3 starts with tile t and is waited on two
// tiles later.
// Blocks are renumbered so that all query tiles of one head run on the same XCD
// (hardware deals blocks round-robin over the 8 XCDs), keeping the head's K/V in one L2.

#include "common.h"

namespace {

constexpr int kD = 128;                 // head dim
#ifndef FLK_ATTEND_WAVES
#define FLK_ATTEND_WAVES 8
#endif
#ifndef FLK_ATTEND_QB
#define FLK_ATTEND_QB 1
#endif
constexpr int kWaves = FLK_ATTEND_WAVES;   // waves per block (two per SIMD at 8)
constexpr int kQB = FLK_ATTEND_QB;         // 32-query column blocks per wave
constexpr int kWavesPerSimd = kWaves / 4;
constexpr int kRowsPerWave = 64 / kWaves;  // tile rows each wave copies
constexpr int kBM = kWaves * kQB * 32;  // queries per block
constexpr int kBN = 64;                 // keys per LDS tile (two 32-key units)
constexpr int kStages = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRowBytes = kD * 2;       // one K or V row: 256 B = 16 chunks of 16 B
constexpr int kTileBytes = kBN * kRowBytes;
constexpr int kBufBytes = 2 * kTileBytes;  // K tile then V tile
constexpr int kUnitBytes = 32 * kRowBytes;
constexpr int kXcds = 8;
constexpr float kLog2e = 1.4426950408889634f;

using flk::bf16x2;
using flk::bf16x8;
using flk::f32x16;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ int swz(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

// Copy one 64-key tile of K and V (rows kv0..kv0+63, clamped to the last row) into `buf`.
// Each wave moves 64/kWaves rows of K and of V, 4 rows (64 lanes x 16 B) per instruction:
// lane i of global_load_lds_dwordx4 lands at M0 + 16 i.  The instruction is issued from
// inline asm so that the compiler does not order every later LDS read behind it (it cannot
// prove the ring buffers disjoint); completion is awaited explicitly with vmcnt.
constexpr int kDmaPerTile = 2 * (kRowsPerWave / 4);  // per wave: K and V instructions of one tile

__device__ __forceinline__ void copy_tile(uint8_t* buf, const uint16_t* __restrict__ kh,
                                          const uint16_t* __restrict__ vh, int kv0, int length,
                                          int wave, int lane) {
#pragma unroll
  for (int i = 0; i < kRowsPerWave / 4; ++i) {
    const int row0 = wave * kRowsPerWave + i * 4;               // wave-uniform first row
    const int row = row0 + (lane >> 4);                          // tile row this lane fills
    const int chunk = (lane & 15) ^ swz(row);                    // logical chunk for its slot
    const int key = min(kv0 + row, length - 1);
    const int64_t src = (int64_t)key * kD + chunk * 8;
    flk::dma16(kh + src, buf + row0 * kRowBytes);
    flk::dma16(vh + src, buf + kTileBytes + row0 * kRowBytes);
  }
}

struct WaveState {
  bf16x8 qreg[kQB][8];
  f32x16 oacc[kQB][4];
  f32x16 sA[kQB];
  f32x16 sB[kQB];
  float lsum[kQB];
  int k_off[8];   // K operand byte offsets within a unit (d step st)
  int v_off[4];   // V^T transpose-read byte offsets within a tile (d block m), key step 0
};

__device__ __forceinline__ bf16x8 v_operand(const uint8_t* vtile, int off) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vtile + off));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vtile + off + 8 * kRowBytes));
  const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, both);
}

// exp / bf16 / row-sum of one element pair (two keys of one query).
template <bool kMask>
__device__ __forceinline__ uint32_t exp_pair(float s0, float s1, float& lsum, int key0, int length) {
  float e0 = __builtin_amdgcn_exp2f(s0 * kLog2e);
  float e1 = __builtin_amdgcn_exp2f(s1 * kLog2e);
  if constexpr (kMask) {
    e0 = key0 < length ? e0 : 0.0f;
    e1 = key0 + 1 < length ? e1 : 0.0f;
  }
  const uint32_t w = flk::pack_bf16x2(e0, e1);
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), ones, lsum, false);
  return w;
}

// Unit phase: P(u) = exp(S(u)) interleaved with S(u+1) = K(u+1) Q^T, then O^T += V(u)^T P(u)^T.
template <bool kMask>
__device__ __forceinline__ void unit_phase(WaveState& w, const f32x16 (&s_cur)[kQB],
                                           f32x16 (&s_next)[kQB], const uint8_t* k_next,
                                           const uint8_t* v_tile, int ks0, int key_base,
                                           int length, int g) {
  bf16x8 kop[8], vop[2][4];
#pragma unroll
  for (int st = 0; st < 8; ++st) kop[st] = *reinterpret_cast<const bf16x8*>(k_next + w.k_off[st]);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int m = 0; m < 4; ++m) vop[ks][m] = v_operand(v_tile, w.v_off[m] + (ks0 + ks) * 16 * kRowBytes);
  // S(u) may sit in accumulation registers (the MFMA wrote it there); moving it to VGPRs
  // once here, with an empty asm that must see it in VGPRs, keeps the exp work below from
  // reading accumulation registers element by element while the next MFMAs are in flight,
  // which serialises each read behind the matrix pipe.
  f32x16 sv[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    sv[qb] = s_cur[qb];
    asm volatile("" : "+v"(sv[qb]));
  }
  __builtin_amdgcn_sched_barrier(0);

  // The exp work of the 8*kQB element pairs is software-pipelined across the MFMA slots:
  // slot n carries the log2(e) multiplies of pair n+2, the exps of pair n+1 and the bf16
  // pack + row sum of pair n, so no VALU op waits on the one just issued before it.
  constexpr int kPairs = 8 * kQB;                     // pair n: query block n % kQB, elements 2*(n/kQB), +1
  uint32_t p[kQB][8];
  float t[kPairs][2], e[kPairs][2];
  auto stage_mul = [&](int n) {
    const int qb = n % kQB, i = 2 * (n / kQB);
    t[n][0] = sv[qb][i] * kLog2e;
    t[n][1] = sv[qb][i + 1] * kLog2e;
  };
  auto stage_exp = [&](int n) {
    e[n][0] = __builtin_amdgcn_exp2f(t[n][0]);
    e[n][1] = __builtin_amdgcn_exp2f(t[n][1]);
  };
  auto stage_pack = [&](int n) {
    const int qb = n % kQB, i = 2 * (n / kQB);
    float e0 = e[n][0], e1 = e[n][1];
    if constexpr (kMask) {
      const int key0 = key_base + (i >> 2) * 8 + g * 4 + (i & 3);
      e0 = key0 < length ? e0 : 0.0f;
      e1 = key0 + 1 < length ? e1 : 0.0f;
    }
    const uint32_t wv = flk::pack_bf16x2(e0, e1);
    p[qb][i >> 1] = wv;
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    w.lsum[qb] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wv), ones, w.lsum[qb], false);
  };
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) s_next[qb] = f32x16{};
  stage_mul(0);
  stage_mul(1);
  stage_exp(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int n = 0; n < kPairs; ++n) {
    const int st = n / kQB, qb = n % kQB;              // the MFMA of this slot
    s_next[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[st], w.qreg[qb][st], s_next[qb], 0, 0, 0);
    if (n + 2 < kPairs) stage_mul(n + 2);
    if (n + 1 < kPairs) stage_exp(n + 1);
    stage_pack(n);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    bf16x8 b[kQB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
      b[qb] = __builtin_bit_cast(bf16x8, make_uint4(p[qb][ks * 4], p[qb][ks * 4 + 1],
                                                    p[qb][ks * 4 + 2], p[qb][ks * 4 + 3]));
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb)
        w.oacc[qb][m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[ks][m], b[qb], w.oacc[qb][m], 0, 0, 0);
  }
}

// One 64-key tile = two unit phases.  The second phase computes S of the next tile's first
// unit (on the last tile it reads a stale buffer; that result is unused).
template <bool kMask>
__device__ __forceinline__ void tile_step(WaveState& w, const uint8_t* cur, const uint8_t* nxt,
                                          int kv0, int length, int g) {
  unit_phase<kMask>(w, w.sA, w.sB, cur + kUnitBytes, cur + kTileBytes, 0, kv0, length, g);
  __builtin_amdgcn_sched_barrier(0);
  unit_phase<kMask>(w, w.sB, w.sA, nxt, cur + kTileBytes, 2, kv0 + 32, length, g);
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void qk_first(WaveState& w, const uint8_t* kunit) {
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) w.sA[qb] = f32x16{};
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(kunit + w.k_off[st]);
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
      w.sA[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, w.qreg[qb][st], w.sA[qb], 0, 0, 0);
  }
}

__global__ __launch_bounds__(kThreads, kWavesPerSimd) void attend_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int length, int q_blocks,
    int total_blocks) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kBufBytes];

  // XCD-aware renumbering: hardware block id p runs on XCD p % 8; give each XCD a
  // contiguous range of logical ids (head-major), so a head's query tiles share an L2.
  const int p = blockIdx.x;
  const int xcd = p % kXcds, local = p / kXcds;
  const int per = total_blocks / kXcds, extra = total_blocks % kXcds;
  const int logical = xcd * per + min(xcd, extra) + local;
  const int bh = logical / q_blocks;
  const int qblk = logical - bh * q_blocks;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 5;   // lane half: selects k-slots 8g..8g+7 and accumulator rows 4g..
  const int c = lane & 31;   // query column (S^T, O^T) / operand row (K, V^T)

  const int64_t head_off = (int64_t)bh * length * kD;
  const uint16_t* qh = q + head_off;
  const uint16_t* kh = k + head_off;
  const uint16_t* vh = v + head_off;

  const int ntiles = (length + kBN - 1) / kBN;
  const int full_tiles = length / kBN;
  copy_tile(smem, kh, vh, 0, length, wave, lane);
  copy_tile(smem + kBufBytes, kh, vh, kBN, length, wave, lane);
  copy_tile(smem + 2 * kBufBytes, kh, vh, 2 * kBN, length, wave, lane);

  WaveState w;
  const int q0 = qblk * kBM + wave * (kQB * 32);
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int qi = q0 + qb * 32 + c;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      w.qreg[qb][s] = qi < length
                          ? *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * kD + s * 16 + g * 8)
                          : bf16x8{};
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) w.oacc[qb][m] = f32x16{};
    w.lsum[qb] = 0.0f;
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) w.k_off[s] = c * kRowBytes + ((((s << 1) | g) ^ swz(c)) << 4);
  {
    // Transpose-read source lane: 16-lane block h, lane sl in it -> key g*4 + sl/4 (+16 ks,
    // +8 for the upper four k-slots), columns m*32 + 16*(h&1) + 4*(sl&3) .. +3.
    const int h = lane >> 4, sl = lane & 15;
    const int key = g * 4 + (sl >> 2);
    const int half = sl & 1;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int chunk = 4 * m + 2 * (h & 1) + ((sl & 3) >> 1);
      w.v_off[m] = key * kRowBytes + ((chunk ^ swz(key)) << 4) + half * 8;
    }
  }

  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kDmaPerTile) : "memory");  // tiles 0 and 1 landed
  __syncthreads();
  qk_first(w, smem);

  // Full tiles, then the partial tail tile (if any) with key masking.  Tile t lives in
  // buffer t % 4.  Iteration t starts the copy of tile t + 3 (into the buffer tile t - 1 has
  // left) and ends by waiting for all but that copy -- i.e. for tile t + 2, which the next
  // iteration's second phase reads -- so each copy has two iterations to land.  Copies past
  // the end re-read the last row into a buffer nobody reads.
  for (int t = 0; t < full_tiles; ++t) {
    copy_tile(smem + ((t + 3) & 3) * kBufBytes, kh, vh, (t + 3) * kBN, length, wave, lane);
    tile_step<false>(w, smem + (t & 3) * kBufBytes, smem + ((t + 1) & 3) * kBufBytes, t * kBN, length, g);
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(kDmaPerTile) : "memory");
    __syncthreads();
  }
  if (full_tiles < ntiles) {
    const int t = full_tiles;
    tile_step<true>(w, smem + (t & 3) * kBufBytes, smem + ((t + 1) & 3) * kBufBytes, t * kBN, length, g);
  }
  // No copy may still be writing this block's LDS when the block ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: l over both lane halves, O = bf16(acc / l), 4 d values per 8-byte store.
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const float l = w.lsum[qb] + __shfl_xor(w.lsum[qb], 32);
    const int qi = q0 + qb * 32 + c;
    if (qi < length) {
      uint16_t* orow = o + head_off + (int64_t)qi * kD;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d0 = m * 32 + r * 8 + g * 4;
          uint2 val;
          val.x = flk::pack_bf16x2(w.oacc[qb][m][r * 4 + 0] / l, w.oacc[qb][m][r * 4 + 1] / l);
          val.y = flk::pack_bf16x2(w.oacc[qb][m][r * 4 + 2] / l, w.oacc[qb][m][r * 4 + 3] / l);
          *reinterpret_cast<uint2*>(orow + d0) = val;
        }
      }
    }
  }
}

}  // namespace

extern "C" int flk_attend(const void* q, const void* k, const void* v, void* o, int batch,
                          int heads, int length, int head_dim, void* stream) {
  if (head_dim != kD) return FLK_E_UNSUPPORTED;
  if (batch < 0 || heads < 0 || length < 0) return FLK_E_INVALID;
  if (batch == 0 || heads == 0 || length == 0) return FLK_OK;
  if (!q || !k || !v || !o) return FLK_E_INVALID;
  if (!flk_host_aligned(q, 16) || !flk_host_aligned(k, 16) || !flk_host_aligned(v, 16) ||
      !flk_host_aligned(o, 16))
    return FLK_E_ALIGN;
  const int64_t q_blocks = (length + kBM - 1) / kBM;
  const int64_t total = q_blocks * batch * heads;
  if (total > INT32_MAX) return FLK_E_INVALID;
  hipLaunchKernelGGL(attend_kernel, dim3((unsigned)total), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(o), length, (int)q_blocks, (int)total);
  return flk_launch_status();
}
