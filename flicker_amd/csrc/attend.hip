// attend: bounded flash attention on gfx950 bf16 MFMA.
//
// Semantics follow the reference kernel (src/flicker/kernels.py:105-145): for each
// (b, h) and query i, over keys in order,
//   S = q_i . k_j  (bf16 operands, f32 accumulate)     -- q arrives scaled by 1/sqrt(D)
//   P = bf16(exp(S))                                  -- no running max: QK-norm bounds S
//   l += f32(P);  acc += P * v_j                       (f32)
//   o_i = bf16(acc / l)
//
// Formulation.  Each wave owns 32 queries and computes the transposed score tile
// S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q^T held in
// registers for the whole kernel).  In the 32x32 accumulator layout a lane owns one query
// column and 16 key rows, so
//   * exp / bf16 rounding / the row sum l are lane-local (l is reduced across the two
//     lane halves once, in the epilogue), and
//   * the rounded P registers are directly the B operand (keys x queries) of the second
//     product O^T += V^T P^T -- no shuffle of P through LDS.
// V stays row-major in LDS; its transposed operand (d rows x 8 keys per lane) is fetched
// with two ds_read_b64_tr_b16, whose 16-lane transpose hands lane 4a+b element b of source
// lanes a, a+4, a+8, a+12 -- so source lane s points at key K0 + s/4, columns D0 + 4(s%4).
// The 8 keys a lane receives follow the accumulator-row order of S^T, so the P registers
// of lane half g line up with the V^T k-slots of the same half.
//
// Schedule.  Keys are processed in units of 32 (one S^T accumulator).  Phase u issues 16
// MFMAs -- the 8 of S(u+1) = K(u+1) Q^T, then the 8 of O^T += V(u-1)^T P(u-1)^T -- and
// spreads the exp work of unit u over them, one element per MFMA (log2(e) multiply of
// element n+2, exp of n+1, and on every second slot the bf16 pack of a pair); the row sum
// of the unit's packed pairs follows the phase's last MFMA as one run of v_dot2.  At two
// waves per SIMD that VALU load mostly hides under the matrix pipe.  Each MFMA's LDS
// operand is read kLead slots ahead into an 8-deep register ring, and the packed P values
// are tied to their slots so the compiler cannot batch them elsewhere.
//
// Staging.  K and V live in separate 4-deep rings of 64-key tiles (16 KiB each).
// Iteration t (the exp work of units 2t, 2t+1) reads K tiles t, t+1 and V tiles t-1, t,
// starts the copies of K tile t+3 and V tile t+2, and ends by waiting for the copies it
// started one iteration earlier, then a block barrier.  Copies go from global memory straight into LDS with
// global_load_lds_dwordx4 (no registers), issued from inline asm so the compiler does not
// order later LDS reads behind them: lane i of a wave instruction lands at M0 + 16 i, so
// the XOR swizzle chunk' = chunk ^ swz(row), swz = ((row&3)<<1)|((row>>2)&1), is applied by
// choosing which global chunk each lane fetches.  It keeps every 8 consecutive K rows (b128
// operand reads) and every group of 4 V rows x 2 chunks (transpose reads) on distinct banks.
// The main loop is unrolled over the four ring positions, so every LDS address is a
// per-lane constant plus an immediate offset.
//
// Blocks of 8 waves (two per SIMD) take 256 queries of one (b, h).  Blocks are renumbered
// so that all query tiles of one head run on the same XCD (hardware deals blocks
// round-robin over the 8 XCDs), keeping the head's K/V in one L2.
//
// Small grids (few heads, short sequences) leave CUs idle for the whole launch.  For them
// the keys are cut into ranges (flk_attend_split_to): each block sums one range into
// unnormalised (acc, l) partials, and attend_merge_kernel adds the ranges in order and
// divides.  With no running max the partial sums need no rescaling.

#include <algorithm>
#include <mutex>

#include "common.h"

// Fixed partials buffer of flk_attend_split_static_to (device memory beyond its inputs and
// outputs, so that callers which cannot allocate can still take the key-split path).  Each
// GPU the library runs on holds its own copy until the process ends.  In host code this name
// is only a stand-in for the symbol: its device address is looked up per device with
// hipGetSymbolAddress (static_scratch below) and only that address reaches a kernel.
static __device__ __align__(256) uint8_t scratch[FLK_ATTEND_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kD = 128;                  // head dim
constexpr int kWaves = 8;                // waves per block, two per SIMD
constexpr int kBM = kWaves * 32;         // queries per block
constexpr int kBN = 64;                  // keys per LDS tile (two 32-key units)
constexpr int kRing = 4;                 // tiles per ring (K and V each)
constexpr int kThreads = kWaves * 64;
constexpr int kRowBytes = kD * 2;        // one K or V row: 256 B = 16 chunks of 16 B
constexpr int kUnitBytes = 32 * kRowBytes;
constexpr int kTileBytes = kBN * kRowBytes;
constexpr int kVRing = kRing * kTileBytes;     // byte offset of the V ring
constexpr int kSmemBytes = 2 * kRing * kTileBytes;
constexpr int kRowsPerWave = kBN / kWaves;     // tile rows each wave copies (8)
constexpr int kDmaPerTensor = kRowsPerWave / 4;  // copy instructions per wave per tile (2)
constexpr int kDmaPerIter = 2 * kDmaPerTensor;   // K and V
constexpr int kXcds = 8;
constexpr int kLead = 4;                 // slots between an operand's LDS read and its MFMA
constexpr int kOpRing = 8;               // operand registers in flight (> kLead)
// Slot n of every phase uses ops[n % kOpRing], and the next phase's first operands are read
// into the same places, so the ring must divide the 16 slots of a phase.
static_assert(16 % kOpRing == 0 && kOpRing > kLead, "operand ring must divide 16 and exceed kLead");
constexpr float kLog2e = 1.4426950408889634f;

using flk::bf16x2;
using flk::bf16x8;
using flk::f32x16;
using flk::f32x4;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ int swz(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }

struct WaveState {
  bf16x8 qreg[8];      // Q^T operand, d step st
  f32x16 oacc[4];      // O^T, d block m
  f32x16 sA, sB;       // S^T of consecutive units
  uint32_t pA[8], pB[8];  // bf16x2-packed P of consecutive units
  bf16x8 ops[kOpRing]; // operand ring: the A operand of MFMA slot n sits in ops[n % kOpRing]
  float lsum;
  int k_off[4];        // K operand byte offsets within a unit, d steps 0-3 (step st + 4 is
                       // 8 chunks = 128 B further: the swizzle only permutes the low 3 chunk bits)
  int v_off[4];        // V^T transpose-read byte offsets within a unit (d block m), key step 0
};

__device__ __forceinline__ bf16x8 v_operand(const uint8_t* vunit, int off) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vunit + off));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vunit + off + 8 * kRowBytes));
  const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, both);
}

// Slot n of a phase issues one MFMA: n < 8 is step n of S = K Q^T (A = K row operand of
// d step n), n >= 8 is step i = n - 8 of O^T += V^T P^T (A = V^T operand of key step i / 4,
// d block i % 4).  Its A operand is read from LDS kLead slots earlier.
__device__ __forceinline__ bf16x8 load_operand(const WaveState& w, int n, const uint8_t* k_unit,
                                               const uint8_t* v_unit) {
  if (n < 8) return *reinterpret_cast<const bf16x8*>(k_unit + w.k_off[n & 3] + (n >> 2) * 128);
  const int i = n - 8;
  return v_operand(v_unit, w.v_off[i & 3] + (i >> 2) * 16 * kRowBytes);
}

// Phase u: S(u+1) = K(u+1) Q^T and O^T += V(u-1)^T P(u-1)^T on the MFMA pipe, while the VALU
// turns S(u) into P(u) and l.  k_cur / v_cur hold K(u+1) and V(u-1); k_next holds K(u+2),
// whose first kLead operands (those of the next phase) are read at the end of this one.
template <bool kMask>
__device__ __forceinline__ void phase(WaveState& w, const f32x16& s_cur, f32x16& s_next,
                                      const uint32_t (&p_prev)[8], uint32_t (&p_cur)[8],
                                      const uint8_t* k_cur, const uint8_t* v_cur, const uint8_t* k_next,
                                      int key_base, int length, int g) {
  f32x16 sv = s_cur;
  asm volatile("" : "+v"(sv));
  float t[16], e[16];
  auto mul = [&](int n) { t[n] = sv[n] * kLog2e; };
  auto ex = [&](int n) { e[n] = __builtin_amdgcn_exp2f(t[n]); };
  auto pack = [&](int n) {  // elements n, n+1 -> p_cur[n/2]
    float e0 = e[n], e1 = e[n + 1];
    if constexpr (kMask) {
      const int key0 = key_base + (n >> 2) * 8 + g * 4 + (n & 3);
      e0 = key0 < length ? e0 : 0.0f;
      e1 = key0 + 1 < length ? e1 : 0.0f;
    }
    p_cur[n >> 1] = flk::pack_bf16x2(e0, e1);
    asm volatile("" : "+v"(p_cur[n >> 1]));   // keep the pack in its MFMA slot
  };
  auto rowsum = [&](int j) {  // l += both halves of p_cur[j]
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    w.lsum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p_cur[j]), ones, w.lsum, false);
    asm volatile("" : "+v"(w.lsum));   // pinned here: l feeds only the epilogue, so it would sink
  };
  const bf16x8 pb0 = __builtin_bit_cast(bf16x8, make_uint4(p_prev[0], p_prev[1], p_prev[2], p_prev[3]));
  const bf16x8 pb1 = __builtin_bit_cast(bf16x8, make_uint4(p_prev[4], p_prev[5], p_prev[6], p_prev[7]));

  mul(0);
  mul(1);
  ex(0);
  s_next = f32x16{};
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    bf16x8& a = w.ops[n % kOpRing];
    if (n < 8) {
      s_next = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, w.qreg[n], s_next, 0, 0, 0);
    } else {
      const int i = n - 8;
      w.oacc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, (i >> 2) ? pb1 : pb0, w.oacc[i & 3], 0, 0, 0);
    }
    const int nl = n + kLead;   // slot whose operand is read now
    if (nl < 16) w.ops[nl % kOpRing] = load_operand(w, nl, k_cur, v_cur);
    else w.ops[(nl - 16) % kOpRing] = load_operand(w, nl - 16, k_next, v_cur);
    if (n + 2 < 16) mul(n + 2);
    if (n + 1 < 16) ex(n + 1);
    if (n & 1) pack(n - 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  // The row sum of the unit's 8 packed pairs, in pair order, after the phase's last MFMA:
  // v_dot2 stalls the matrix pipe when it issues between MFMAs, and one run of eight here
  // measured 2% faster than one dot2 per slot pair (same operations, same order, same bits).
#pragma unroll
  for (int j = 0; j < 8; ++j) rowsum(j);
}

// Copy 64-key tile `tile` (clamped to the last one) of K or V into an LDS ring slot.
// Rows past the end of the sequence repeat the last row; those keys are masked.
struct CopyPlan {
  uint32_t voff[kDmaPerTensor];       // per-lane source offsets of a full tile
  uint32_t voff_last[kDmaPerTensor];  // ... of the last tile (rows past the end repeat the last row)
  int last_tile;                      // index of the last tile
  int lds_wave_off;                   // this wave's rows within a tile (bytes, wave-uniform)
};

__device__ __forceinline__ void copy_tile(uint8_t* dst, const uint16_t* __restrict__ head, int tile,
                                          const CopyPlan& cp) {
  tile = min(tile, cp.last_tile);
  const uint16_t* base = head + (int64_t)tile * kBN * kD;
  if (tile < cp.last_tile) {
#pragma unroll
    for (int i = 0; i < kDmaPerTensor; ++i) flk::dma16_at(base, cp.voff[i], dst + cp.lds_wave_off + i * 4 * kRowBytes);
  } else {
#pragma unroll
    for (int i = 0; i < kDmaPerTensor; ++i)
      flk::dma16_at(base, cp.voff_last[i], dst + cp.lds_wave_off + i * 4 * kRowBytes);
  }
}

struct Ctx {
  uint8_t* smem;
  const uint16_t* kh;
  const uint16_t* vh;
  int length, ntiles, g;
  CopyPlan cp;
};

// Iteration t at ring position r = (t - t_begin) % 4: the exp work of units 2t and 2t+1.  It reads K
// tiles t and t+1 and V tiles t-1 and t, and starts the copies of K tile t+3 and V tile
// t+2 into the slots of K tile t-1 and V tile t-2, which no read of this iteration touches.
// Called with a literal r in the unrolled main loop, so every LDS address folds to a
// per-lane constant plus an immediate offset.
template <bool kMask>
__device__ __forceinline__ void iteration(WaveState& w, const Ctx& c, int t, int r) {
  copy_tile(c.smem + ((r + 3) & 3) * kTileBytes, c.kh, t + 3, c.cp);
  copy_tile(c.smem + kVRing + ((r + 2) & 3) * kTileBytes, c.vh, t + 2, c.cp);
  const uint8_t* k_t = c.smem + r * kTileBytes;                          // K tile t
  const uint8_t* k_t1 = c.smem + ((r + 1) & 3) * kTileBytes;             // K tile t+1
  const uint8_t* v_t = c.smem + kVRing + r * kTileBytes;                 // V tile t
  const uint8_t* v_tm1 = c.smem + kVRing + ((r + 3) & 3) * kTileBytes;   // V tile t-1
  const int key0 = t * kBN;
  // phase 2t: K(2t+1), V(2t-1), next K(2t+2); phase 2t+1: K(2t+2), V(2t), next K(2t+3)
  phase<kMask>(w, w.sA, w.sB, w.pB, w.pA, k_t + kUnitBytes, v_tm1 + kUnitBytes, k_t1, key0, c.length, c.g);
  phase<kMask>(w, w.sB, w.sA, w.pA, w.pB, k_t1, v_t, k_t1 + kUnitBytes, key0 + 32, c.length, c.g);
  // Wait for the copies started one iteration ago, then a plain s_barrier: the LDS reads
  // still in flight touch no buffer the next copies write, so no lgkmcnt wait is needed.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(kDmaPerIter) : "memory");
}

// kSplit = false: the block takes every key of its 256 queries and writes O.
// kSplit = true: the key tiles are cut into `splits` ranges of equal length (+-1 tile); the
// block takes one range and writes its unnormalised acc and l to part_acc / part_l, which
// attend_merge_kernel sums.  Ring slots count from the block's first tile, so the unrolled
// loop keeps literal ring positions wherever the range starts.  Without a
// running max the partial sums of different key ranges add as they are.
template <bool kSplit>
__global__ __launch_bounds__(kThreads, 2) void attend_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int length, int q_blocks,
    int total_blocks, int heads, int splits, int64_t o_batch_stride, int64_t o_head_stride,
    int64_t o_row_stride, float* __restrict__ part_acc, float* __restrict__ part_l) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];

  // XCD-aware renumbering: hardware block id p runs on XCD p % 8; give each XCD a
  // contiguous range of logical ids (head-major, then query tile, then key range), so the
  // blocks that read one head's keys share an L2, and so do the key ranges of one query
  // tile, whose partials attend_merge_kernel then reads on the same XCD.
  const int p = blockIdx.x;
  const int xcd = p % kXcds, local = p / kXcds;
  const int per = total_blocks / kXcds, extra = total_blocks % kXcds;
  const int logical = xcd * per + min(xcd, extra) + local;
  const int split = kSplit ? logical % splits : 0;
  const int rest = kSplit ? logical / splits : logical;
  const int qblk = rest % q_blocks;
  const int bh = rest / q_blocks;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  Ctx c;
  c.smem = smem;
  c.g = lane >> 5;            // lane half: selects k-slots 8g..8g+7 and accumulator rows 4g..
  const int col = lane & 31;  // query column (S^T, O^T) / operand row (K, V^T)
  c.length = length;
  c.ntiles = (length + kBN - 1) / kBN;
  c.cp.last_tile = c.ntiles - 1;
  int t_begin = 0, t_end = c.ntiles;   // this block's key tiles
  if constexpr (kSplit) {
    t_begin = split * c.ntiles / splits;
    t_end = (split + 1) * c.ntiles / splits;
  }
  c.cp.lds_wave_off = __builtin_amdgcn_readfirstlane(wave * kRowsPerWave * kRowBytes);
  {
    const int rows_last = length - c.cp.last_tile * kBN;   // 1..64 valid rows in the last tile
#pragma unroll
    for (int i = 0; i < kDmaPerTensor; ++i) {
      const int row = wave * kRowsPerWave + i * 4 + (lane >> 4);
      const uint32_t chunk_off = ((lane & 15) ^ swz(row)) << 4;   // slot (lane & 15) holds this chunk
      c.cp.voff[i] = (uint32_t)(row * kRowBytes) + chunk_off;
      c.cp.voff_last[i] = (uint32_t)(min(row, rows_last - 1) * kRowBytes) + chunk_off;
    }
  }

  const int64_t head_off = (int64_t)bh * length * kD;
  const uint16_t* qh = q + head_off;
  c.kh = k + head_off;
  c.vh = v + head_off;

  // Prologue copies: K tiles t_begin .. +2, V tiles t_begin .. +1 into ring slots 0-2 and 0-1
  // (tile t sits in slot (t - t_begin) % 4).
  for (int tl = 0; tl < 3; ++tl) copy_tile(smem + tl * kTileBytes, c.kh, t_begin + tl, c.cp);
  for (int tl = 0; tl < 2; ++tl) copy_tile(smem + kVRing + tl * kTileBytes, c.vh, t_begin + tl, c.cp);

  WaveState w;
  const int q0 = qblk * kBM + wave * 32;
  const int qi = q0 + col;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    w.qreg[s] = qi < length ? *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * kD + s * 16 + c.g * 8)
                            : bf16x8{};
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) w.oacc[m] = f32x16{};
  w.lsum = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    w.k_off[s] = col * kRowBytes + ((((s << 1) | c.g) ^ swz(col)) << 4);
    asm volatile("" : "+v"(w.k_off[s]));
  }
  {
    // Transpose-read source lane: 16-lane block h, lane sl in it -> key g*4 + sl/4 (+16 ks,
    // +8 for the upper four k-slots), columns m*32 + 16*(h&1) + 4*(sl&3) .. +3.
    const int h = lane >> 4, sl = lane & 15;
    const int key = c.g * 4 + (sl >> 2);
    const int half = sl & 1;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int chunk = 4 * m + 2 * (h & 1) + ((sl & 3) >> 1);
      w.v_off[m] = key * kRowBytes + ((chunk ^ swz(key)) << 4) + half * 8;
      // Opaque to the compiler: it then adds the (immediate) unit offsets with the DS
      // instruction's offset field instead of a v_or per read.
      asm volatile("" : "+v"(w.v_off[m]));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) w.pB[i] = 0u;   // P(-1) = 0: phase 0's PV MFMAs add nothing
  // ... and the V(-1) operand they read (V ring slot 3, unit 1) is zeroed, so 0 * V = 0.
  reinterpret_cast<uint4*>(smem + kVRing + 3 * kTileBytes + kUnitBytes)[tid] = make_uint4(0, 0, 0, 0);

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // S(0) from K unit 0; operands of phase 0: K(1) and a placeholder V (multiplied by P(-1) = 0).
  w.sA = f32x16{};
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(smem + w.k_off[st & 3] + (st >> 2) * 128);
    w.sA = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, w.qreg[st], w.sA, 0, 0, 0);
  }
#pragma unroll
  for (int n = 0; n < kLead; ++n) w.ops[n % kOpRing] = load_operand(w, n, smem + kUnitBytes, smem);

  // Unrolled main loop over full tiles, then the remaining (at most 3 full and one partial)
  // tiles with key masking and a computed ring position.
  const int full_end = min(length / kBN, t_end);
  int t = t_begin;
  for (; t + 4 <= full_end; t += 4) {
    iteration<false>(w, c, t, 0);
    iteration<false>(w, c, t + 1, 1);
    iteration<false>(w, c, t + 2, 2);
    iteration<false>(w, c, t + 3, 3);
  }
  for (; t < t_end; ++t) iteration<true>(w, c, t, (t - t_begin) & 3);
  // No copy may still be writing this block's LDS when the block ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Drain: O^T += V(U-1)^T P(U-1)^T for the last unit (unit 1 of the last tile).
  {
    const uint8_t* v_last = smem + kVRing + ((t_end - 1 - t_begin) & 3) * kTileBytes + kUnitBytes;
    const bf16x8 pb0 = __builtin_bit_cast(bf16x8, make_uint4(w.pB[0], w.pB[1], w.pB[2], w.pB[3]));
    const bf16x8 pb1 = __builtin_bit_cast(bf16x8, make_uint4(w.pB[4], w.pB[5], w.pB[6], w.pB[7]));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w.oacc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load_operand(w, 8 + i, v_last, v_last),
                                                              (i >> 2) ? pb1 : pb0, w.oacc[i & 3], 0, 0, 0);
  }

  // Epilogue: l over both lane halves, O = bf16(acc / l), 4 d values per 8-byte store.
  const float l = w.lsum + __shfl_xor(w.lsum, 32);
  if constexpr (kSplit) {
    // Partials in the accumulator's own lane order, so each store is 64 lanes x 16 bytes
    // contiguous: with unit = bh * q_blocks + qblk, register group i = 4m + r holds
    // acc[d = 32m + 8r + 4g .. +3] of query qi at float4 index
    //   ((split * units + unit) * 8 + wave) * 1024 + i * 64 + lane,
    // and l at ((split * units + unit) * 8 + wave) * 64 + lane.
    const int64_t units = total_blocks / splits;
    const int64_t slot = ((int64_t)split * units + (int64_t)bh * q_blocks + qblk) * kWaves + wave;
    f32x4* dst = reinterpret_cast<f32x4*>(part_acc) + slot * 1024 + lane;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dst[(m * 4 + r) * 64] = f32x4{w.oacc[m][r * 4 + 0], w.oacc[m][r * 4 + 1], w.oacc[m][r * 4 + 2],
                                      w.oacc[m][r * 4 + 3]};
    part_l[slot * 64 + lane] = l;
  } else if (qi < length) {
    const int b = bh / heads, h = bh - b * heads;
    uint16_t* orow = o + b * o_batch_stride + h * o_head_stride + (int64_t)qi * o_row_stride;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d0 = m * 32 + r * 8 + c.g * 4;
        uint2 val;
        val.x = flk::pack_bf16x2(w.oacc[m][r * 4 + 0] / l, w.oacc[m][r * 4 + 1] / l);
        val.y = flk::pack_bf16x2(w.oacc[m][r * 4 + 2] / l, w.oacc[m][r * 4 + 3] / l);
        *reinterpret_cast<uint2*>(orow + d0) = val;
      }
    }
  }
}

// Sums the split partials in split order and writes O = bf16(acc / l) with attend_kernel's
// own epilogue arithmetic.  Thread id = ((unit * 8 + wave) * 16 + i) * 64 + lane takes one
// register group of one lane, so split s's value is float4 s * units * 8192 + id: every
// split is one contiguous 16-byte load per thread.  Blocks are renumbered like
// attend_kernel's, so unit u is merged on the XCD whose L2 holds its partials.
constexpr int kMergeThreads = 256;

__global__ __launch_bounds__(kMergeThreads) void attend_merge_kernel(
    const float* __restrict__ part_acc, const float* __restrict__ part_l, uint16_t* __restrict__ o,
    int length, int q_blocks, int64_t units, int heads, int splits, int64_t o_batch_stride,
    int64_t o_head_stride, int64_t o_row_stride) {
  const int p = blockIdx.x;
  const int xcd = p % kXcds, local = p / kXcds;
  const int per = gridDim.x / kXcds, extra = gridDim.x % kXcds;
  const int64_t id = (int64_t)(xcd * per + min(xcd, extra) + local) * kMergeThreads + threadIdx.x;
  const int lane = (int)(id & 63);
  const int i = (int)((id >> 6) & 15);
  const int64_t wave_slot = id >> 10;            // unit * 8 + wave
  const int wave = (int)(wave_slot & 7);
  const int64_t unit = wave_slot >> 3;
  if (unit >= units) return;
  const int64_t bh = unit / q_blocks;
  const int qblk = (int)(unit - bh * q_blocks);
  const int qi = qblk * kBM + wave * 32 + (lane & 31);
  if (qi >= length) return;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
#pragma unroll 4
  for (int s = 0; s < splits; ++s) {
    acc += reinterpret_cast<const f32x4*>(part_acc)[s * units * 8192 + id];
    l += part_l[(s * units + unit) * 512 + wave * 64 + lane];
  }
  const int64_t b = bh / heads, h = bh - b * heads;
  const int d0 = (i >> 2) * 32 + (i & 3) * 8 + (lane >> 5) * 4;
  uint2 val;
  val.x = flk::pack_bf16x2(acc.x / l, acc.y / l);
  val.y = flk::pack_bf16x2(acc.z / l, acc.w / l);
  *reinterpret_cast<uint2*>(o + b * o_batch_stride + h * o_head_stride + (int64_t)qi * o_row_stride + d0) = val;
}

}  // namespace

namespace {

// Blocks per launch below which the key range is split: a grid this small leaves CUs idle
// for the whole launch (256 CUs, one block each).
constexpr int kSplitBelow = 192;
constexpr int kCUs = 256;

// Argument checks shared by the entry points: FLK_OK = launch, kNothing = empty input (nothing
// to do), else an error status.
constexpr int kNothing = 1;

int check_attend(const void* q, const void* k, const void* v, void* o, int batch, int heads, int length,
                 int head_dim, int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride) {
  if (head_dim != kD) return FLK_E_UNSUPPORTED;
  if (batch < 0 || heads < 0 || length < 0) return FLK_E_INVALID;
  if (batch == 0 || heads == 0 || length == 0) return kNothing;
  if (!q || !k || !v || !o) return FLK_E_INVALID;
  if (!flk_host_aligned(q, 16) || !flk_host_aligned(k, 16) || !flk_host_aligned(v, 16) ||
      !flk_host_aligned(o, 8) || o_batch_stride % 4 || o_head_stride % 4 || o_row_stride % 4)
    return FLK_E_ALIGN;
  if (o_batch_stride < 0 || o_head_stride < 0 || o_row_stride < kD) return FLK_E_INVALID;
  if ((int64_t)((length + kBM - 1) / kBM) * batch * heads > INT32_MAX) return FLK_E_INVALID;
  return FLK_OK;
}

int64_t q_tiles(int length) { return (length + kBM - 1) / kBM; }
int key_groups(int length) { return ((length + kBN - 1) / kBN + 3) / 4; }

// Workspace of a split launch: per split and (b, h, 256-query tile), 512 lanes x (64 acc + 1 l)
// floats.
int64_t split_workspace_bytes(int batch, int heads, int length, int splits) {
  return (int64_t)splits * batch * heads * q_tiles(length) * kThreads * 65 * (int64_t)sizeof(float);
}

int launch_attend(const void* q, const void* k, const void* v, void* o, int batch, int heads, int length,
                  int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride, void* stream) {
  const int64_t total = q_tiles(length) * batch * heads;
  hipLaunchKernelGGL(attend_kernel<false>, dim3((unsigned)total), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(o), length, (int)q_tiles(length), (int)total, heads, 1,
                     o_batch_stride, o_head_stride, o_row_stride, nullptr, nullptr);
  return flk_launch_status();
}

}  // namespace

extern "C" int flk_attend(const void* q, const void* k, const void* v, void* o, int batch,
                          int heads, int length, int head_dim, void* stream) {
  const int64_t row = kD, head = (int64_t)length * kD, bstride = (int64_t)heads * head;
  const int st = check_attend(q, k, v, o, batch, heads, length, head_dim, bstride, head, row);
  if (st != FLK_OK) return st == kNothing ? FLK_OK : st;
  return launch_attend(q, k, v, o, batch, heads, length, bstride, head, row, stream);
}

extern "C" int flk_attend_to(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                             int length, int head_dim, int64_t o_batch_stride, int64_t o_head_stride,
                             int64_t o_row_stride, void* stream) {
  const int st = check_attend(q, k, v, o, batch, heads, length, head_dim, o_batch_stride, o_head_stride,
                              o_row_stride);
  if (st != FLK_OK) return st == kNothing ? FLK_OK : st;
  return launch_attend(q, k, v, o, batch, heads, length, o_batch_stride, o_head_stride, o_row_stride, stream);
}

extern "C" int flk_attend_plan(int batch, int heads, int length, int* splits, int64_t* workspace_bytes) {
  if (batch < 0 || heads < 0 || length < 0 || !splits || !workspace_bytes) return FLK_E_INVALID;
  int s = 1;
  const int64_t blocks = q_tiles(length) * batch * heads;
  if (blocks > 0 && blocks < kSplitBelow) {
    // As many splits as fill the CUs once, each keeping at least two 4-tile key groups.
    s = (int)std::min<int64_t>(kCUs / blocks, key_groups(length) / 2);
    s = std::max(s, 1);
  }
  *splits = s;
  *workspace_bytes = s > 1 ? split_workspace_bytes(batch, heads, length, s) : 0;
  return FLK_OK;
}

namespace {

// Grid sizes of a split launch, checked before anything is launched.
int check_split_grid(int batch, int heads, int length, int splits) {
  const int64_t units = q_tiles(length) * batch * heads;
  const int64_t total = units * splits;
  const int64_t merge_blocks = units * kWaves * 16 * 64 / kMergeThreads;
  return total > INT32_MAX || merge_blocks > INT32_MAX ? FLK_E_INVALID : FLK_OK;
}

// The split kernel into `workspace` (at least split_workspace_bytes), then the merge.
int launch_split(const void* q, const void* k, const void* v, void* o, int batch, int heads, int length,
                 int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride, int splits,
                 void* workspace, void* stream) {
  const int64_t units = q_tiles(length) * batch * heads;
  const int64_t total = units * splits;
  const int64_t merge_blocks = units * kWaves * 16 * 64 / kMergeThreads;
  float* part_acc = static_cast<float*>(workspace);
  float* part_l = part_acc + total * kThreads * 64;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(attend_kernel<true>, dim3((unsigned)total), dim3(kThreads), 0, hs,
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                     static_cast<const uint16_t*>(v), static_cast<uint16_t*>(o), length, (int)q_tiles(length),
                     (int)total, heads, splits, o_batch_stride, o_head_stride, o_row_stride, part_acc, part_l);
  const int launched = flk_launch_status();
  if (launched != FLK_OK) return launched;
  hipLaunchKernelGGL(attend_merge_kernel, dim3((unsigned)merge_blocks), dim3(kMergeThreads), 0, hs, part_acc,
                     part_l, static_cast<uint16_t*>(o), length, (int)q_tiles(length), units, heads, splits,
                     o_batch_stride, o_head_stride, o_row_stride);
  return flk_launch_status();
}

// Device address of `scratch` on the GPU that runs `stream`, looked up once per device with
// that device current and kept for the life of the process.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_addr[kMaxDevices] = {};

int static_scratch(void* stream, void** addr) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return (int)e;
  hipDevice_t dev = cur;
  if (stream) {
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev);
    if (e != hipSuccess) return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) return FLK_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return (int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (e == hipSuccess && back != hipSuccess) e = back;
    }
    if (e != hipSuccess) return (int)e;
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return FLK_OK;
}

}  // namespace

extern "C" int flk_attend_split_to(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                                   int length, int head_dim, int64_t o_batch_stride, int64_t o_head_stride,
                                   int64_t o_row_stride, int splits, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  const int st = check_attend(q, k, v, o, batch, heads, length, head_dim, o_batch_stride, o_head_stride,
                              o_row_stride);
  if (st != FLK_OK) return st == kNothing ? FLK_OK : st;
  if (splits < 1 || splits > key_groups(length)) return FLK_E_INVALID;
  if (splits == 1) return launch_attend(q, k, v, o, batch, heads, length, o_batch_stride, o_head_stride,
                                        o_row_stride, stream);
  const int64_t need = split_workspace_bytes(batch, heads, length, splits);
  if (!workspace || workspace_bytes < need) return FLK_E_INVALID;
  if (!flk_host_aligned(workspace, 16)) return FLK_E_ALIGN;
  const int grid = check_split_grid(batch, heads, length, splits);
  if (grid != FLK_OK) return grid;
  return launch_split(q, k, v, o, batch, heads, length, o_batch_stride, o_head_stride, o_row_stride, splits,
                      workspace, stream);
}

extern "C" int flk_attend_split_static_to(const void* q, const void* k, const void* v, void* o, int batch,
                                          int heads, int length, int head_dim, int64_t o_batch_stride,
                                          int64_t o_head_stride, int64_t o_row_stride, int splits, void* stream) {
  const int st = check_attend(q, k, v, o, batch, heads, length, head_dim, o_batch_stride, o_head_stride,
                              o_row_stride);
  if (st != FLK_OK) return st == kNothing ? FLK_OK : st;
  if (splits < 1 || splits > key_groups(length)) return FLK_E_INVALID;
  if (splits == 1) return launch_attend(q, k, v, o, batch, heads, length, o_batch_stride, o_head_stride,
                                        o_row_stride, stream);
  if (split_workspace_bytes(batch, heads, length, splits) > (int64_t)FLK_ATTEND_STATIC_SCRATCH_BYTES)
    return FLK_E_SCRATCH;
  const int grid = check_split_grid(batch, heads, length, splits);
  if (grid != FLK_OK) return grid;
  void* ws = nullptr;
  const int found = static_scratch(stream, &ws);
  if (found != FLK_OK) return found;
  return launch_split(q, k, v, o, batch, heads, length, o_batch_stride, o_head_stride, o_row_stride, splits,
                      ws, stream);
}
