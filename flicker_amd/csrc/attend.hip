// attend: bounded flash attention on gfx950 bf16 MFMA.
//
// Semantics follow the reference kernel (src/flicker/kernels.py:105-145): for each
// (b, h) and query i, over key tiles in order,
//   S = q_i . k_j  (bf16 operands, f32 accumulate)     -- q arrives scaled by 1/sqrt(D)
//   P = bf16(exp(S))                                  -- no running max: QK-norm bounds S
//   l += f32(P);  acc += P * v_j                       (f32)
//   o_i = bf16(acc / l)
//
// Formulation.  Each wave owns 32 queries and computes the transposed score tile
// S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q^T held in
// registers for the whole kernel).  In the 32x32 accumulator layout a lane owns one
// query column and 16 key rows, so
//   * exp / bf16 rounding / the row sum l are lane-local (l is reduced across the two
//     lane halves once, in the epilogue), and
//   * the rounded P registers are directly the B operand (keys x queries) of the second
//     product O^T += V^T P^T -- no shuffle of P through LDS.
// V^T is the A operand of that product, so V tiles are written to LDS transposed
// (d-major) during staging, with the key order inside each 16-key group permuted to
// match the accumulator-row order of S^T, so one ds_read_b128 fetches an operand.
//
// Staging: a 256-thread block (4 waves, 128 queries) streams 64-key K and V tiles
// through two LDS buffers: the next tile's global loads are issued before the current
// tile's MFMAs and written to the other buffer after them (one barrier per tile).
// LDS rows are XOR-swizzled in 16-byte chunks so the operand reads of 16 consecutive
// lanes hit distinct banks.  Blocks are renumbered so that all query tiles of one head
// run on the same XCD (hardware deals blocks round-robin over the 8 XCDs), keeping
// that head's K/V resident in one L2.

#include "common.h"

namespace {

constexpr int kD = 128;                 // head dim
constexpr int kWaves = 4;
constexpr int kQW = 32;                 // queries per wave
constexpr int kBM = kWaves * kQW;       // queries per block
constexpr int kBN = 64;                 // keys per tile
constexpr int kThreads = kWaves * 64;
constexpr int kKBytes = kBN * kD * 2;   // K tile: kBN rows x 256 B
constexpr int kVBytes = kD * kBN * 2;   // V^T tile: kD rows x 128 B
constexpr int kBufBytes = kKBytes + kVBytes;
constexpr int kXcds = 8;
constexpr float kLog2e = 1.4426950408889634f;

using flk::bf16x8;
using flk::f32x16;

// Chunk swizzle of a 128-byte V^T row (8 chunks of 16 B): conflict-free for 16 consecutive
// rows on 64 banks and for 8 consecutive rows on 32 banks.
__device__ __forceinline__ int vt_swizzle(int d) { return (d & 7) ^ ((d >> 3) & 1); }

// Position of tile key `kappa` (0..63) inside its V^T row: chunk (before swizzle) and
// byte offset inside the chunk.  Slot (g, j) of the PV operand at key step ks holds key
// ks*16 + (j/4)*8 + g*4 + j%4, the key that S^T accumulator register 8*(ks%2)+j of lane
// half g holds.
__device__ __forceinline__ void vt_slot(int kappa, int& chunk, int& byte_in_chunk) {
  const int ks = kappa >> 4, r = kappa & 15;
  chunk = ks * 2 + ((r >> 2) & 1);
  byte_in_chunk = (((r >> 3) << 2) + (r & 3)) * 2;
}

struct Tile {
  uint4 k[4];
  uint4 v[4];
};

__device__ __forceinline__ void load_tile(Tile& tl, const uint16_t* __restrict__ kh,
                                          const uint16_t* __restrict__ vh, int kv0, int length,
                                          int kg, int ch) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int key = kv0 + kg * 4 + r;
    if (key < length) {
      const int64_t off = (int64_t)key * kD + ch * 8;
      tl.k[r] = *reinterpret_cast<const uint4*>(kh + off);
      tl.v[r] = *reinterpret_cast<const uint4*>(vh + off);
    } else {
      tl.k[r] = make_uint4(0, 0, 0, 0);
      tl.v[r] = make_uint4(0, 0, 0, 0);
    }
  }
}

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) {
  return (a & 0xFFFFu) | (b << 16);
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xFFFF0000u);
}

__device__ __forceinline__ void store_tile(const Tile& tl, uint8_t* buf, int kg, int ch) {
  uint8_t* ks = buf;
  uint8_t* vt = buf + kKBytes;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int key = kg * 4 + r;
    *reinterpret_cast<uint4*>(ks + key * 256 + ((ch ^ (key & 15)) << 4)) = tl.k[r];
  }
  // Transpose: 4 keys (kg*4 .. +3, contiguous in the permuted slot order) x 8 d values.
  int chunk, byte_in_chunk;
  vt_slot(kg * 4, chunk, byte_in_chunk);
  const uint32_t w0[4] = {tl.v[0].x, tl.v[0].y, tl.v[0].z, tl.v[0].w};
  const uint32_t w1[4] = {tl.v[1].x, tl.v[1].y, tl.v[1].z, tl.v[1].w};
  const uint32_t w2[4] = {tl.v[2].x, tl.v[2].y, tl.v[2].z, tl.v[2].w};
  const uint32_t w3[4] = {tl.v[3].x, tl.v[3].y, tl.v[3].z, tl.v[3].w};
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int d = ch * 8 + jj;
    const int w = jj >> 1;
    uint2 val;
    if (jj & 1) {
      val.x = hi_pair(w0[w], w1[w]);
      val.y = hi_pair(w2[w], w3[w]);
    } else {
      val.x = lo_pair(w0[w], w1[w]);
      val.y = lo_pair(w2[w], w3[w]);
    }
    *reinterpret_cast<uint2*>(vt + d * 128 + ((chunk ^ vt_swizzle(d)) << 4) + byte_in_chunk) = val;
  }
}

__global__ __launch_bounds__(kThreads, 2) void attend_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int length, int q_blocks,
    int total_blocks) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kBufBytes];

  // XCD-aware renumbering: hardware block id p runs on XCD p % 8; give each XCD a
  // contiguous range of logical ids (head-major), so a head's query tiles share an L2.
  const int p = blockIdx.x;
  const int xcd = p % kXcds, local = p / kXcds;
  const int per = total_blocks / kXcds, extra = total_blocks % kXcds;
  const int logical = xcd * per + min(xcd, extra) + local;
  const int bh = logical / q_blocks;
  const int qb = logical - bh * q_blocks;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 5;   // lane half: selects k-slots 8g..8g+7 and accumulator rows 4g..
  const int c = lane & 31;   // query column (S^T, O^T) / operand row (K, V^T)

  const int64_t head_off = (int64_t)bh * length * kD;
  const uint16_t* qh = q + head_off;
  const uint16_t* kh = k + head_off;
  const uint16_t* vh = v + head_off;

  // Q^T operand registers: query qi, d = 16*s + 8*g + j.
  const int qi = qb * kBM + wave * kQW + c;
  bf16x8 qreg[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    if (qi < length) {
      qreg[s] = *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * kD + s * 16 + g * 8);
    } else {
      qreg[s] = bf16x8{};
    }
  }

  f32x16 oacc[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) oacc[m] = f32x16{};
  float lsum = 0.0f;

  const int kg = tid >> 4, ch = tid & 15;  // staging role: keys kg*4..+3, 16-byte chunk ch
  const int ntiles = (length + kBN - 1) / kBN;

  // Per-lane LDS operand offsets (loop invariant).
  int k_off[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) k_off[s] = c * 256 + ((((s << 1) | g) ^ (c & 15)) << 4);
  int v_off[4];
  const int vsw = vt_swizzle(c);  // same for rows c + 32*m
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) v_off[ks] = c * 128 + (((ks << 1) | g) ^ vsw) * 16;

  Tile tl;
  load_tile(tl, kh, vh, 0, length, kg, ch);
  store_tile(tl, smem, kg, ch);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int kv0 = t * kBN;
    uint8_t* cur = smem + (t & 1) * kBufBytes;
    if (t + 1 < ntiles) load_tile(tl, kh, vh, kv0 + kBN, length, kg, ch);

    // S^T = K Q^T for two 32-key halves of the tile.
    f32x16 sacc[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(cur + kb * 32 * 256 + k_off[s]);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[s], sacc[kb], 0, 0, 0);
      }
    }

    // P = bf16(exp(S)); keys past the end contribute nothing.
    uint32_t pw[2][8];
    const bool tail = kv0 + kBN > length;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float e0 = __builtin_amdgcn_exp2f(sacc[kb][i] * kLog2e);
        float e1 = __builtin_amdgcn_exp2f(sacc[kb][i + 1] * kLog2e);
        if (tail) {
          const int key0 = kv0 + kb * 32 + (i >> 2) * 8 + g * 4 + (i & 3);
          if (key0 >= length) e0 = 0.0f;
          if (key0 + 1 >= length) e1 = 0.0f;
        }
        const uint32_t packed = flk::pack_bf16x2(e0, e1);
        pw[kb][i >> 1] = packed;
        lsum += flk::bf16_lo(packed) + flk::bf16_hi(packed);
      }
    }

    // O^T += V^T P^T, 16 keys per MFMA, 4 blocks of 32 d rows.
    const uint8_t* vt = cur + kKBytes;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const uint32_t* src = &pw[ks >> 1][(ks & 1) * 4];
      const uint4 pv = make_uint4(src[0], src[1], src[2], src[3]);
      const bf16x8 b = __builtin_bit_cast(bf16x8, pv);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(vt + m * 32 * 128 + v_off[ks]);
        oacc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, oacc[m], 0, 0, 0);
      }
    }

    if (t + 1 < ntiles) store_tile(tl, smem + ((t + 1) & 1) * kBufBytes, kg, ch);
    __syncthreads();
  }

  // Epilogue: l over both lane halves, O = bf16(acc / l), rows of 4 d values per store.
  lsum += __shfl_xor(lsum, 32);
  if (qi < length) {
    uint16_t* orow = o + head_off + (int64_t)qi * kD;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = m * 32 + r * 8 + g * 4;
        uint2 val;
        val.x = flk::pack_bf16x2(oacc[m][r * 4 + 0] / lsum, oacc[m][r * 4 + 1] / lsum);
        val.y = flk::pack_bf16x2(oacc[m][r * 4 + 2] / lsum, oacc[m][r * 4 + 3] / lsum);
        *reinterpret_cast<uint2*>(orow + d0) = val;
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
