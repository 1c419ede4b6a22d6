// attend: bounded flash attention on gfx950 bf16 MFMA.
//
// Semantics follow the reference kernel (src/flicker/kernels.py:105-145): for each
// (b, h) and query i, over keys in order,
//   S = q_i . k_j  (bf16 operands, f32 accumulate)     -- q arrives scaled by 1/sqrt(D)
//   P = bf16(exp(S))                                  -- no running max: QK-norm bounds S
//   l += f32(P);  acc += P * v_j                       (f32)
//   o_i = bf16(acc / l)
//
// Formulation.  Each wave owns 32 queries, as two groups of 16, and computes the transposed
// score tile S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = 16 K rows x 32 d from LDS, B =
// Q^T of one query group, held in registers for the whole kernel).  Under random bf16 data the
// chip runs at its power limit, and at that limit the 16x16x32 form does the same flops on
// less energy than 32x32x16 (a quarter of the accumulator traffic per instruction): with this
// kernel's softmax mix it issues ~7% more flops per second (microbenchmark).  Each K operand
// feeds the MFMAs of both query groups, so LDS traffic per flop is that of a 32-query 32x32
// tile.  In the 16x16 accumulator layout lane l owns query l % 16 of its group and keys
// 4(l/16) .. +3 of a 16-key tile, so
//   * exp / bf16 rounding are lane-local, and
//   * the rounded P of the unit's two 16-key tiles are directly the B operand (32 keys x 16
//     queries) of O^T += V^T P^T, with k-slots 0-3 = keys 4(l/16) .. +3 and 4-7 = the same
//     keys + 16 -- no shuffle of P through LDS.
// The row sum l = sum f32(P) is one more MFMA per query group and unit: O^T's d tiles get a
// ninth, whose A operand is a register constant with ones in row 0 and zeros elsewhere, so
// its row 0 accumulates sum_k 1 * P[k] (exact products, f32 sums on the matrix pipe).  That
// replaces 8 v_dot2 per phase: 2 cheap MFMAs (mostly-zero operand, no LDS read) in place of
// a fifth of the VALU work, measured 3.6% faster.
// V stays row-major in LDS; its transposed operand (16 d rows x 8 keys per lane) is fetched
// with two ds_read_b64_tr_b16, whose 16-lane transpose hands lane 4a+b element b of source
// lanes a, a+4, a+8, a+12 -- so source lane s of lane group h points at key 4h + s/4 (then
// 16 more), columns D0 + 4(s%4): the k-slots line up with those of P.
//
// Schedule.  Keys are processed in units of 32 (two 16-key tiles).  Phase u issues 32 MFMAs
// in 16 operand slots of two (one per query group) -- slots 0-7 the 16 of S(u+1) = K(u+1)
// Q^T, slots 8-15 the 16 of O^T += V(u-1)^T P(u-1)^T -- and spreads the exp work of unit u
// over the slots, one element per slot (log2(e) multiply of element n+2, exp of n+1, and on
// every second slot the bf16 pack of a pair), and the two row-sum MFMAs follow the last d
// tile.  At two waves per SIMD that VALU load mostly hides under the matrix pipe.  Each slot's LDS operand is read kLead slots ahead into an
// 8-deep register ring, and the packed P values are tied to their slots so the compiler cannot
// batch them elsewhere.
//
// Staging.  K and V live in separate 4-deep rings of 64-key tiles (16 KiB each).
// Iteration t (the exp work of units 2t, 2t+1) reads K tiles t, t+1 and V tiles t-1, t,
// starts the copies of K tile t+3 and V tile t+2, and ends by waiting for the copies it
// started one iteration earlier, then a block barrier.  Copies go from global memory straight into LDS with
// global_load_lds_dwordx4 (no registers), issued from inline asm so the compiler does not
// order later LDS reads behind them: lane i of a wave instruction lands at M0 + 16 i, so
// the XOR swizzle chunk' = chunk ^ swz(row), swz = ((row&7)<<1)|((row>>3)&1), is applied by
// choosing which global chunk each lane fetches.  gfx950's LDS serves 256 B per clock from 64
// banks, i.e. one whole 256-byte row: a b128 read is served 16 lanes at a time and a b64
// transpose read 32 lanes at a time.  The swizzle puts the 16 K rows of a b128 operand read
// (one chunk each) and the 8 V rows x 2 chunks of 32 lanes of a transpose read on 16 distinct
// chunk positions, so neither read conflicts.  (A 3-bit swizzle, distinct over 8 rows only,
// left both 2-way conflicted: SQ_LDS_BANK_CONFLICT counted exactly the predicted 2x.)
// The main loop is unrolled over the four ring positions, so every LDS address is a
// per-lane constant plus an immediate offset.
//
// Blocks of 8 waves (two per SIMD) take 256 queries of one (b, h).  Blocks are renumbered
// so that all query tiles of one head run on the same XCD (hardware deals blocks
// round-robin over the 8 XCDs), keeping the head's K/V in one L2.  A grid that fits the
// 256 CUs in one round either way takes 192-query tiles instead (attend_tile192_kernel):
// waves 4-7 then hold one query group of 16, so each SIMD holds 48 queries instead of 64
// and the one round is 3/4 as long (measured 16-20% faster, e.g. 512^2: 144 -> 192 blocks).
//
// Small grids (few heads, short sequences) leave CUs idle for the whole launch.  For them
// the keys are cut into ranges (flk_attend_split_to): each block sums one range into
// unnormalised (acc, l) partials, and attend_merge_kernel adds the ranges in order and
// divides.  With no running max the partial sums need no rescaling.

#include <algorithm>
#include <atomic>
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
// The V ring sits at LDS offset 0 and the K ring above it.  K operand pointers leave out the
// K ring's base, which the per-lane offsets k_off carry, so that every LDS address is a
// per-lane register plus an immediate below 64 KiB (the DS offset field is 16 bits).
constexpr int kVRing = 0;                      // byte offset of the V ring
constexpr int kKRing = kRing * kTileBytes;     // byte offset of the K ring
constexpr int kSmemBytes = 2 * kRing * kTileBytes;
constexpr int kRowsPerWave = kBN / kWaves;     // tile rows each wave copies (8)
constexpr int kDmaPerTensor = kRowsPerWave / 4;  // copy instructions per wave per tile (2)
constexpr int kDmaPerIter = 2 * kDmaPerTensor;   // K and V
constexpr int kXcds = 8;
constexpr int kCUs = 256;                // MI355X compute units (one balanced block each)
constexpr int kLead = 4;                 // slots between an operand's LDS read and its MFMA
constexpr int kOpRing = 8;               // operand registers in flight (> kLead)
// Slot n of every phase uses ops[n % kOpRing], and the next phase's first operands are read
// into the same places, so the ring must divide the 16 slots of a phase.
static_assert(16 % kOpRing == 0 && kOpRing > kLead, "operand ring must divide 16 and exceed kLead");
constexpr float kLog2e = 1.4426950408889634f;

using flk::bf16x8;
using flk::f32x4;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ int swz(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }

// A wave's registers for G query groups of 16 (G = 2: 32 queries; G = 1: 16).
template <int G>
struct WaveState {
  bf16x8 qreg[4][G];   // Q^T operand: d step s (32 d), query group g (16 queries)
  f32x4 oacc[8][G];    // O^T: d tile dt (16 d), query group g
  f32x4 sA[2 * G], sB[2 * G];  // S^T of consecutive units, accumulator g * 2 + kt (16-key tile kt)
  uint32_t pA[4 * G], pB[4 * G];  // bf16x2-packed P of consecutive units: word g * 4 + kt * 2 + pair
  bf16x8 ops[kOpRing]; // operand ring: the A operand of slot n sits in ops[n % kOpRing]
  f32x4 lacc[G];       // row sums l of the query groups (register 0 of lanes 0-15)
  bf16x8 ones;         // A operand of the row-sum MFMA: row 0 all ones, rows 1-15 zero
  int k_off[4];        // K operand byte offsets within a unit, d steps 0-3 (key tile 1 is 16 rows
                       // further, with the same swizzle)
  int v_off[8];        // V^T transpose-read byte offsets within a unit, d tiles 0-7
};

// The V^T operand of one 16-row d tile: keys 4h + (0..3) from the first transpose read and
// keys 16 + 4h + (0..3) from the second (h = lane / 16).
__device__ __forceinline__ bf16x8 v_operand(const uint8_t* vunit, int off) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vunit + off));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vunit + off + 16 * kRowBytes));
  const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, both);
}

// Slot n of a phase issues one MFMA per query group, sharing its A operand: n < 8 is
// d step n / 2 of S = K Q^T for 16-key tile n % 2 (A = K rows of that tile and d step), n >= 8
// is d tile n - 8 of O^T += V^T P^T (A = V^T operand of the tile).  The operand is read from
// LDS kLead slots earlier.
template <int G>
__device__ __forceinline__ bf16x8 load_operand(const WaveState<G>& w, int n, const uint8_t* k_unit,
                                               const uint8_t* v_unit) {
  if (n < 8) {
    const int st = n >> 1, kt = n & 1;
    return *reinterpret_cast<const bf16x8*>(k_unit + w.k_off[st] + kt * 16 * kRowBytes);
  }
  const int dt = n - 8;
  return v_operand(v_unit, w.v_off[dt]);
}

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// P^T of query group g as the B operand of O^T += V^T P^T: k-slots 0-3 from 16-key tile 0,
// 4-7 from tile 1 -- the group's four packed words, in order.
template <int G>
__device__ __forceinline__ bf16x8 p_operand(const uint32_t (&p)[4 * G], int g) {
  return __builtin_bit_cast(bf16x8, make_uint4(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3]));
}

// Phase u: S(u+1) = K(u+1) Q^T and O^T += V(u-1)^T P(u-1)^T on the MFMA pipe, while the VALU
// turns S(u) into P(u) and l.  k_cur / v_cur hold K(u+1) and V(u-1); k_next holds K(u+2),
// whose first kLead operands (those of the next phase) are read at the end of this one.
// Element n of a unit is register n % 4 of accumulator n / 4 = g * 2 + kt.  The unit's 8 G
// softmax elements are spread over the 16 slots: one per slot for G = 2, one every other
// slot for G = 1.
template <bool kMask, int G, typename SlotHook>
__device__ __forceinline__ void phase(WaveState<G>& w, const f32x4 (&s_cur)[2 * G], f32x4 (&s_next)[2 * G],
                                      const uint32_t (&p_prev)[4 * G], uint32_t (&p_cur)[4 * G],
                                      const uint8_t* k_cur, const uint8_t* v_cur, const uint8_t* k_next,
                                      int key_base, int length, int h, SlotHook&& hook) {
  static_assert(G == 1 || G == 2, "one or two query groups per wave");
  constexpr int E = 8 * G;   // softmax elements per lane per unit
  f32x4 sv[2 * G];
#pragma unroll
  for (int i = 0; i < 2 * G; ++i) {
    sv[i] = s_cur[i];
    asm volatile("" : "+v"(sv[i]));
  }
  float t[E], e[E];
  auto mul = [&](int n) { t[n] = sv[n >> 2][n & 3] * kLog2e; };
  auto ex = [&](int n) { e[n] = __builtin_amdgcn_exp2f(t[n]); };
  auto pack = [&](int n) {  // elements n, n+1 -> p_cur[n/2]
    float e0 = e[n], e1 = e[n + 1];
    if constexpr (kMask) {
      const int key0 = key_base + ((n >> 2) & 1) * 16 + h * 4 + (n & 3);
      e0 = key0 < length ? e0 : 0.0f;
      e1 = key0 + 1 < length ? e1 : 0.0f;
    }
    p_cur[n >> 1] = flk::pack_bf16x2(e0, e1);
    asm volatile("" : "+v"(p_cur[n >> 1]));   // keep the pack in its MFMA slot
  };
  bf16x8 pb[G];
#pragma unroll
  for (int g = 0; g < G; ++g) pb[g] = p_operand<G>(p_prev, g);

  mul(0);
  mul(1);
  ex(0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    bf16x8& a = w.ops[n % kOpRing];
    if (n < 8) {
      const int st = n >> 1, kt = n & 1;
      // each S chain starts from the MFMA's inline zero accumulator
#pragma unroll
      for (int g = 0; g < G; ++g)
        s_next[2 * g + kt] = mfma16(a, w.qreg[st][g], st == 0 ? f32x4{} : s_next[2 * g + kt]);
    } else {
      const int dt = n - 8;
#pragma unroll
      for (int g = 0; g < G; ++g) w.oacc[dt][g] = mfma16(a, pb[g], w.oacc[dt][g]);
      if (dt == 7) {
#pragma unroll
        for (int g = 0; g < G; ++g) w.lacc[g] = mfma16(w.ones, pb[g], w.lacc[g]);
      }
    }
    const int nl = n + kLead;   // slot whose operand is read now
    if (nl < 16) w.ops[nl % kOpRing] = load_operand(w, nl, k_cur, v_cur);
    else w.ops[(nl - 16) % kOpRing] = load_operand(w, nl - 16, k_next, v_cur);
    if constexpr (G == 2) {
      if (n + 2 < E) mul(n + 2);
      if (n + 1 < E) ex(n + 1);
      if (n & 1) pack(n - 1);
    } else {
      const int m = n >> 1;
      if ((n & 1) == 0) {
        if (m + 1 < E) ex(m + 1);
        if (m + 2 < E) mul(m + 2);
      } else if (m & 1) {
        pack(m - 1);
      }
    }
    hook(n);   // the iteration's tile copies, one instruction on some slots
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Copy 64-key tile `tile` (clamped to the last one) of K or V into an LDS ring slot.
// Rows past the end of the sequence repeat the last row; those keys are masked.
struct CopyPlan {
  uint32_t voff[kDmaPerTensor];       // per-lane source offsets of a full tile
  uint32_t voff_last[kDmaPerTensor];  // ... of the last tile (rows past the end repeat the last row)
  int last_tile;                      // index of the last tile
  int lds_wave_off;                   // this wave's rows within a tile (bytes, wave-uniform)
};

// One tile copy, planned once and issued as kDmaPerTensor instructions (each 4 rows of the
// wave's 8).  The last tile's offsets are chosen per lane by a select, not a branch.
struct TileCopy {
  const uint16_t* base;
  uint8_t* dst;
  uint32_t off[kDmaPerTensor];
};

__device__ __forceinline__ TileCopy plan_copy(uint8_t* dst, const uint16_t* __restrict__ head, int tile,
                                              const CopyPlan& cp) {
  tile = min(tile, cp.last_tile);
  TileCopy tc;
  tc.base = head + (int64_t)tile * kBN * kD;
  tc.dst = dst + cp.lds_wave_off;
  const bool last = tile == cp.last_tile;
#pragma unroll
  for (int i = 0; i < kDmaPerTensor; ++i) tc.off[i] = last ? cp.voff_last[i] : cp.voff[i];
  return tc;
}

__device__ __forceinline__ void issue_copy(const TileCopy& tc, int i) {
  flk::dma16_at(tc.base, tc.off[i], tc.dst + i * 4 * kRowBytes);
}

// Copy 64-key tile `tile` (clamped to the last one) of K or V into an LDS ring slot at once.
__device__ __forceinline__ void copy_tile(uint8_t* dst, const uint16_t* __restrict__ head, int tile,
                                          const CopyPlan& cp) {
  const TileCopy tc = plan_copy(dst, head, tile, cp);
#pragma unroll
  for (int i = 0; i < kDmaPerTensor; ++i) issue_copy(tc, i);
}

struct Ctx {
  uint8_t* smem;
  const uint16_t* kh;
  const uint16_t* vh;
  int length, ntiles, h;
  CopyPlan cp;
};

// Iteration t at ring position r = (t - t_begin) % 4: the exp work of units 2t and 2t+1.  It reads K
// tiles t and t+1 and V tiles t-1 and t, and starts the copies of K tile t+3 and V tile
// t+2 into the slots of K tile t-1 and V tile t-2, which no read of this iteration touches.
// Called with a literal r in the unrolled main loop, so every LDS address folds to a
// per-lane constant plus an immediate offset.
// Slots at which the copy instructions of iteration t issue (K's, then V's; 0-15 in phase
// 2t, 16-31 in phase 2t+1): one at a time between MFMAs rather than all four at the top of
// the iteration (1.3% faster at 4608 keys than the block of four, measured).
constexpr int kDmaSlot[kDmaPerIter] = {1, 3, 17, 19};

template <bool kMask, int G>
__device__ __forceinline__ void iteration(WaveState<G>& w, const Ctx& c, int t, int r) {
  const TileCopy kc = plan_copy(c.smem + kKRing + ((r + 3) & 3) * kTileBytes, c.kh, t + 3, c.cp);
  const TileCopy vc = plan_copy(c.smem + kVRing + ((r + 2) & 3) * kTileBytes, c.vh, t + 2, c.cp);
  auto hook_a = [&](int n) {
#pragma unroll
    for (int i = 0; i < kDmaPerIter; ++i)
      if (kDmaSlot[i] == n) {
        if (i < kDmaPerTensor) issue_copy(kc, i);
        else issue_copy(vc, i - kDmaPerTensor);
      }
  };
  auto hook_b = [&](int n) {
#pragma unroll
    for (int i = 0; i < kDmaPerIter; ++i)
      if (kDmaSlot[i] == n + 16) {
        if (i < kDmaPerTensor) issue_copy(kc, i);
        else issue_copy(vc, i - kDmaPerTensor);
      }
  };
  const uint8_t* k_t = c.smem + r * kTileBytes;                          // K tile t (less kKRing)
  const uint8_t* k_t1 = c.smem + ((r + 1) & 3) * kTileBytes;             // K tile t+1 (less kKRing)
  const uint8_t* v_t = c.smem + kVRing + r * kTileBytes;                 // V tile t
  const uint8_t* v_tm1 = c.smem + kVRing + ((r + 3) & 3) * kTileBytes;   // V tile t-1
  const int key0 = t * kBN;
  // phase 2t: K(2t+1), V(2t-1), next K(2t+2); phase 2t+1: K(2t+2), V(2t), next K(2t+3)
  phase<kMask, G>(w, w.sA, w.sB, w.pB, w.pA, k_t + kUnitBytes, v_tm1 + kUnitBytes, k_t1, key0, c.length, c.h, hook_a);
  phase<kMask, G>(w, w.sB, w.sA, w.pA, w.pB, k_t1, v_t, k_t1 + kUnitBytes, key0 + 32, c.length, c.h, hook_b);
  // Wait for the copies started one iteration ago, then a plain s_barrier: the LDS reads
  // still in flight touch no buffer the next copies write, so no lgkmcnt wait is needed.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(kDmaPerIter) : "memory");
}

// One segment of work for a block: head bh (batch-major), key tiles [t_begin, t_end), and
// for this wave the 16 G queries from q0.  On return w holds the segment's unnormalised O^T accumulators and row
// sums (lacc), and every LDS read and copy of the segment has completed.  Ring slots count from
// the segment's first tile, so the unrolled loop keeps literal ring positions wherever the
// range starts.
template <int G>
__device__ __forceinline__ void attend_segment(WaveState<G>& w, uint8_t* smem, const uint16_t* __restrict__ q,
                                               const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                               int length, int bh, int q0, int t_begin, int t_end) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  Ctx c;
  c.smem = smem;
  c.h = lane >> 4;            // lane group: k-slots 8h..8h+7 and accumulator rows 4h..4h+3
  const int col = lane & 15;  // query column (S^T, O^T) / operand row (K, V^T) in a 16-tile
  c.length = length;
  c.ntiles = (length + kBN - 1) / kBN;
  c.cp.last_tile = c.ntiles - 1;
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
  for (int tl = 0; tl < 3; ++tl) copy_tile(smem + kKRing + tl * kTileBytes, c.kh, t_begin + tl, c.cp);
  for (int tl = 0; tl < 2; ++tl) copy_tile(smem + kVRing + tl * kTileBytes, c.vh, t_begin + tl, c.cp);

  // k-slots 8h..8h+7 of the S MFMAs take d chunk dperm = 4 st + perm(h) of the K and Q rows,
  // perm(h) = 0, 2, 1, 3: lanes l and l + 32 then read neighbouring chunks (c, c ^ 1), which
  // the swizzle keeps on distinct banks whether a b128 read is served as 16 consecutive lanes
  // or as 8 lanes from each half of the wave.
  const int hperm = ((c.h & 1) << 1) | (c.h >> 1);
#pragma unroll
  for (int g = 0; g < G; ++g) {   // query group g of this wave: q0 + 16 g .. + 15
    const int qi = q0 + g * 16 + col;
#pragma unroll
    for (int st = 0; st < 4; ++st)
      w.qreg[st][g] = qi < length
                          ? *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * kD + st * 32 + hperm * 8)
                          : bf16x8{};
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int g = 0; g < G; ++g) w.oacc[dt][g] = f32x4{};
#pragma unroll
  for (int g = 0; g < G; ++g) w.lacc[g] = f32x4{};
  {
    const __bf16 one = (lane & 15) == 0 ? (__bf16)1.0f : (__bf16)0.0f;
    w.ones = bf16x8{one, one, one, one, one, one, one, one};
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    // K operand of d step st: row col of the 16-key tile, d = 32 st + 8 perm(h) .. +7
    w.k_off[st] = kKRing + col * kRowBytes + ((((st << 2) | hperm) ^ swz(col)) << 4);
    asm volatile("" : "+v"(w.k_off[st]));
  }
  {
    // Transpose-read source lane sl of lane group h -> key 4h + sl/4 (+16 for k-slots 4-7),
    // columns 16 dt + 4 (sl % 4) .. +3: chunk 2 dt + (sl % 4) / 2, half sl % 2.
    const int sl = lane & 15;
    const int key = c.h * 4 + (sl >> 2);
    const int half = sl & 1;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int chunk = 2 * dt + ((sl & 3) >> 1);
      w.v_off[dt] = key * kRowBytes + ((chunk ^ swz(key)) << 4) + half * 8;
      // Opaque to the compiler: it then adds the (immediate) unit offsets with the DS
      // instruction's offset field instead of a v_or per read.
      asm volatile("" : "+v"(w.v_off[dt]));
    }
  }
#pragma unroll
  for (int i = 0; i < 4 * G; ++i) w.pB[i] = 0u;   // P(-1) = 0: phase 0's PV MFMAs add nothing
  // ... and the V(-1) operand they read (V ring slot 3, unit 1) is zeroed, so 0 * V = 0.
  reinterpret_cast<uint4*>(smem + kVRing + 3 * kTileBytes + kUnitBytes)[tid] = make_uint4(0, 0, 0, 0);

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // S(0) from K unit 0; operands of phase 0: K(1) and a placeholder V (multiplied by P(-1) = 0).
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int st = n >> 1, kt = n & 1;
    const bf16x8 a = load_operand(w, n, smem, smem);
#pragma unroll
    for (int g = 0; g < G; ++g) w.sA[2 * g + kt] = mfma16(a, w.qreg[st][g], st == 0 ? f32x4{} : w.sA[2 * g + kt]);
  }
#pragma unroll
  for (int n = 0; n < kLead; ++n) w.ops[n % kOpRing] = load_operand(w, n, smem + kUnitBytes, smem);

  // Unrolled main loop over full tiles, then the remaining (at most 3 full and one partial)
  // tiles with key masking and a computed ring position.
  const int full_end = min(length / kBN, t_end);
  int t = t_begin;
  for (; t + 4 <= full_end; t += 4) {
    iteration<false, G>(w, c, t, 0);
    iteration<false, G>(w, c, t + 1, 1);
    iteration<false, G>(w, c, t + 2, 2);
    iteration<false, G>(w, c, t + 3, 3);
  }
  for (; t < t_end; ++t) iteration<true, G>(w, c, t, (t - t_begin) & 3);
  // No copy may still be writing this block's LDS when the segment ends.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Drain: O^T += V(U-1)^T P(U-1)^T for the last unit (unit 1 of the last tile).
  {
    const uint8_t* v_last = smem + kVRing + ((t_end - 1 - t_begin) & 3) * kTileBytes + kUnitBytes;
    bf16x8 pb[G];
#pragma unroll
    for (int g = 0; g < G; ++g) pb[g] = p_operand<G>(w.pB, g);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const bf16x8 a = load_operand(w, 8 + dt, v_last, v_last);
#pragma unroll
      for (int g = 0; g < G; ++g) w.oacc[dt][g] = mfma16(a, pb[g], w.oacc[dt][g]);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) w.lacc[g] = mfma16(w.ones, pb[g], w.lacc[g]);
  }
}

// l of each query group from lanes 0-15 (row 0 of the row-sum tile) to the lanes of every
// lane group.
template <int G>
__device__ __forceinline__ void row_sums(const WaveState<G>& w, float (&l)[G]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int g = 0; g < G; ++g) l[g] = __shfl(w.lacc[g][0], lane & 15);
}

// O = bf16(acc / l) of the wave's 16 G queries from q0, 4 d values per 8-byte store.
template <int G>
__device__ __forceinline__ void store_o(const WaveState<G>& w, const float (&l)[G], uint16_t* __restrict__ o, int bh,
                                        int heads, int q0, int length, int64_t o_batch_stride,
                                        int64_t o_head_stride, int64_t o_row_stride) {
  const int lane = threadIdx.x & 63;
  const int h4 = lane >> 4, col = lane & 15;
  const int b = bh / heads, hd = bh - b * heads;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int qi = q0 + g * 16 + col;
    if (qi >= length) continue;
    uint16_t* orow = o + b * o_batch_stride + hd * o_head_stride + (int64_t)qi * o_row_stride;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d0 = dt * 16 + h4 * 4;
      uint2 val;
      val.x = flk::pack_bf16x2(w.oacc[dt][g][0] / l[g], w.oacc[dt][g][1] / l[g]);
      val.y = flk::pack_bf16x2(w.oacc[dt][g][2] / l[g], w.oacc[dt][g][3] / l[g]);
      *reinterpret_cast<uint2*>(orow + d0) = val;
    }
  }
}

// Partials of one 256-query tile in the accumulator's own lane order, so each store is 64
// lanes x 16 bytes contiguous: register group i = 2 dt + g of wave w holds acc[d = 16 dt +
// 4h .. +3] of query q0 + 16 g + col at float4 index (slot * 8 + w) * 1024 + i * 64 + lane,
// and the l of wave query j (= 16 g + col) at (slot * 8 + w) * 64 + j.
// kCoherent: every word is written by a relaxed device-scope atomic store (a store that
// is coherent across the device on its own, so a reader on any CU that loads it the same
// way after the writer's stores have completed sees it; no cache-wide write-back needed).
template <bool kCoherent = false>
__device__ __forceinline__ void store_partial(const WaveState<2>& w, const float (&l)[2], float* __restrict__ part_acc,
                                              float* __restrict__ part_l, int64_t slot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ws = slot * kWaves + wave;
  f32x4* dst = reinterpret_cast<f32x4*>(part_acc) + ws * 1024 + lane;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if constexpr (kCoherent) {
        union { f32x4 f; uint64_t u[2]; } x;
        x.f = w.oacc[dt][g];
        uint64_t* d = reinterpret_cast<uint64_t*>(dst + (dt * 2 + g) * 64);
        __hip_atomic_store(d, x.u[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(d + 1, x.u[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        dst[(dt * 2 + g) * 64] = w.oacc[dt][g];
      }
    }
  if ((lane >> 4) < 2) {   // lanes 0-15: group 0, 16-31: group 1
    if constexpr (kCoherent)
      __hip_atomic_store(part_l + ws * 64 + lane, l[lane >> 4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      part_l[ws * 64 + lane] = l[lane >> 4];
  }
}

// kSplit = false: the block takes every key of its 256 queries and writes O.
// kSplit = true: the key tiles are cut into `splits` ranges of equal length (+-1 tile); the
// block takes one range and writes its unnormalised acc and l to part_acc / part_l, which
// attend_merge_kernel sums.  Without a running max the partial sums of different key ranges
// add as they are.
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
  const int ntiles = (length + kBN - 1) / kBN;
  int t_begin = 0, t_end = ntiles;   // this block's key tiles
  if constexpr (kSplit) {
    t_begin = split * ntiles / splits;
    t_end = (split + 1) * ntiles / splits;
  }

  const int q0 = qblk * kBM + (threadIdx.x >> 6) * 32;   // this wave's 32 queries
  WaveState<2> w;
  attend_segment(w, smem, q, k, v, length, bh, q0, t_begin, t_end);
  float l[2];
  row_sums(w, l);
  if constexpr (kSplit) {
    const int64_t units = total_blocks / splits;
    store_partial(w, l, part_acc, part_l, (int64_t)split * units + (int64_t)bh * q_blocks + qblk);
  } else {
    store_o(w, l, o, bh, heads, q0, length, o_batch_stride, o_head_stride, o_row_stride);
  }
}

constexpr int kBM192 = 192;   // queries per block of the 192-query tiles

// One block of 256 queries from q_start (every wave two query groups) or, with tile192, of
// 192 (waves 4-7 one group each); queries at or past q_limit (<= length) are not stored.
__device__ __forceinline__ void query_tile(uint8_t* smem, const uint16_t* __restrict__ q,
                                           const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                           uint16_t* __restrict__ o, int length, int bh, int q_start, int q_limit,
                                           bool tile192, int heads, int64_t o_batch_stride, int64_t o_head_stride,
                                           int64_t o_row_stride) {
  const int ntiles = (length + kBN - 1) / kBN;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform branch below
  if (!tile192 || wave < 4) {
    const int q0 = q_start + wave * 32;
    WaveState<2> w;
    attend_segment(w, smem, q, k, v, length, bh, q0, 0, ntiles);
    float l[2];
    row_sums(w, l);
    store_o(w, l, o, bh, heads, q0, q_limit, o_batch_stride, o_head_stride, o_row_stride);
  } else {
    const int q0 = q_start + 128 + (wave - 4) * 16;
    WaveState<1> w;
    attend_segment(w, smem, q, k, v, length, bh, q0, 0, ntiles);
    float l[1];
    row_sums(w, l);
    store_o(w, l, o, bh, heads, q0, q_limit, o_batch_stride, o_head_stride, o_row_stride);
  }
}

// attend_kernel<false> with 192-query tiles, for grids that fit the CUs in one round either
// way: waves 0-3 take 32 queries each (two groups) and waves 4-7 16 each (one group), so
// every SIMD still holds one wave of each kind and 48 queries instead of 64.  Every query's
// arithmetic is attend_kernel's, so the output is the same, bit for bit.
__global__ __launch_bounds__(kThreads, 2) void attend_tile192_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ o, int length, int q_blocks, int total_blocks, int heads, int64_t o_batch_stride,
    int64_t o_head_stride, int64_t o_row_stride) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];
  const int p = blockIdx.x;
  const int xcd = p % kXcds, local = p / kXcds;
  const int per = total_blocks / kXcds, extra = total_blocks % kXcds;
  const int logical = xcd * per + min(xcd, extra) + local;
  const int qblk = logical % q_blocks;
  const int bh = logical / q_blocks;
  query_tile(smem, q, k, v, o, length, bh, qblk * kBM192, length, true, heads, o_batch_stride, o_head_stride,
             o_row_stride);
}

// Rounds launch, for grids of more than one round: each XCD takes a contiguous range of the
// 256-query tiles (b, h, tile), as the balanced launch deals them, runs whole rounds of 32
// of them, and cuts the queries of the tiles left over into 192-query tiles, head by head,
// so that the last round has up to 4/3 as many blocks with 3/4 of the work each.

// The j-th 192-query tile of the queries of 256-query tiles [first, end): head segment by
// head segment, the last tile of a segment cut short at its end (q_end).  False past the last.
__device__ __forceinline__ bool leftover_tile(int first, int end, int q_blocks, int length, int j, int& bh,
                                              int& q_start, int& q_end) {
  for (int u = first; u < end;) {
    const int b = u / q_blocks, t0 = u - b * q_blocks;
    const int t1 = min(q_blocks, t0 + (end - u));
    const int s = t0 * kBM, e = min(t1 * kBM, length);
    const int count = (e - s + kBM192 - 1) / kBM192;
    if (j < count) {
      bh = b;
      q_start = s + j * kBM192;
      q_end = min(q_start + kBM192, e);
      return true;
    }
    j -= count;
    u += t1 - t0;
  }
  return false;
}

__global__ __launch_bounds__(kThreads, 2) void attend_rounds_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ o, int length, int q_blocks, int units, int heads, int64_t o_batch_stride,
    int64_t o_head_stride, int64_t o_row_stride) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];
  constexpr int C = kCUs / kXcds;
  const int x = blockIdx.x % kXcds, l = blockIdx.x / kXcds;   // hardware deals blocks round-robin over XCDs
  const int ux0 = (int)((int64_t)x * units / kXcds);
  const int n = (int)((int64_t)(x + 1) * units / kXcds) - ux0;
  const int full = n / C * C;
  if (l < full) {
    const int unit = ux0 + l;
    const int bh = unit / q_blocks, qblk = unit - bh * q_blocks;
    query_tile(smem, q, k, v, o, length, bh, qblk * kBM, length, false, heads, o_batch_stride, o_head_stride,
               o_row_stride);
    return;
  }
  int bh, q_start, q_end;
  if (!leftover_tile(ux0 + full, ux0 + n, q_blocks, length, l - full, bh, q_start, q_end)) return;
  query_tile(smem, q, k, v, o, length, bh, q_start, q_end, true, heads, o_batch_stride, o_head_stride,
             o_row_stride);
}

// Balanced attend: one persistent block per CU (256), so that the last, partial round of
// tiles is shared by all the CUs.  Tiles (b, h, 256-query tile) are dealt to the 8 XCDs in
// contiguous ranges (keeping each head's K/V in one L2).  On an XCD with n tiles and C = 32
// CUs, CU l first takes tiles l, l + C, ... whole for R = floor(n / C) rounds -- the plain
// kernel's rounds, every CU streaming the keys from tile 0 together, so that K/V tiles are
// shared in the L2 as they arrive.  The r = n - R C tiles left over are W = r * ntiles key
// tiles of work, laid end to end and cut into P = min(C, W) equal ranges, one per CU l < P
// (floor(W l / P) to floor(W (l + 1) / P)): every range is shorter than a tile, so it spans
// at most two segments, and a leftover tile is covered by the ranges of CUs cf .. cl.
//
// A tile covered by one range is written directly.  Otherwise each of its pieces, when its
// segment ends, either finds the tile's counter at pieces - 1 arrivals (every other piece
// published) or publishes its (acc, l) partial: coherent stores to its slot, a wait until they
// have completed, then its arrival on the counter -- whose previous count says whether it was
// the last.  The last piece sums all the pieces in CU order, ((p0 + p1) + p2) + ..., so the
// result does not depend on the order of arrival (its own piece from registers when it is p0
// or p1, whose sum is the same either way; otherwise it publishes too and reads its own back)
// and writes O.  No block ever waits for another.
//
// A counter holds (epoch << 8) | arrivals, the epoch a tag the host gives each call.  A value
// with another epoch, or a count that is already complete (arrivals >= pieces: the previous
// replay of the same captured launch), counts as no arrival, so the counters are never reset:
// a workspace left in any state by an earlier call -- even by two calls that overlapped on it
// -- is valid again for the next call that has it to itself.  A device-scope fence here would write back and
// invalidate the whole L2 of the XCD for every piece, which stalls every block streaming
// keys through that L2 (tens of microseconds per fence).
struct XcdSplit {
  int ux0, R, r, P;
  int W;   // leftover key tiles (< 32 ntiles; the host keeps 1024 ntiles below 2^31)
};

constexpr unsigned kEpochMask = 0xFFFFFFu;   // 24-bit call tags, 8-bit arrival counts (<= 32 pieces)

// Arrivals a counter value records for this call's tile of `pieces` pieces.
__device__ __forceinline__ int arrivals_of(unsigned c, unsigned epoch, int pieces) {
  const int n = (int)(c & 0xFFu);
  return ((c >> 8) == epoch && n < pieces) ? n : 0;
}

// This piece's arrival: the counter becomes (epoch << 8) | (arrivals + 1); returns the arrivals
// before it (pieces - 1: this piece is the last).  `old` is the value last read from the counter:
// the compare-and-swap succeeds at once unless another piece arrived since, and each retry
// starts from the value the failed swap returned.
__device__ __forceinline__ int arrive(int* counter, unsigned epoch, int pieces, unsigned old) {
  for (;;) {
    const int prior = arrivals_of(old, epoch, pieces);
    const unsigned want = (epoch << 8) | (unsigned)(prior + 1);
    const unsigned seen = (unsigned)atomicCAS(counter, (int)old, (int)want);
    if (seen == old) return prior;
    old = seen;
  }
}

__device__ __forceinline__ XcdSplit xcd_split(int units, int ntiles, int x) {
  constexpr int C = kCUs / kXcds;
  XcdSplit xs;
  xs.ux0 = (int)((int64_t)x * units / kXcds);
  const int n = (int)((int64_t)(x + 1) * units / kXcds) - xs.ux0;
  xs.R = n / C;
  xs.r = n - xs.R * C;
  xs.W = xs.r * ntiles;
  xs.P = min(C, xs.W);
  return xs;
}

// Start of leftover range c (key tiles), c = 0 .. P.
__device__ __forceinline__ int range_start(const XcdSplit& xs, int c) { return xs.W * c / xs.P; }

// The range that holds leftover key tile u: the largest c with range_start(c) <= u.
__device__ __forceinline__ int range_of(const XcdSplit& xs, int u) { return (xs.P * (u + 1) - 1) / xs.W; }

// Adds (or, first, assigns) the partial in `slot` to res / rl: res + p in f32, the order of
// the fold.  Read with relaxed device-scope atomic loads (coherent with store_partial<true>).
__device__ __forceinline__ void gather_partial(f32x4 (&res)[8][2], float (&rl)[2], bool first,
                                               const float* __restrict__ part_acc,
                                               const float* __restrict__ part_l, int64_t slot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t ws = slot * kWaves + wave;
  const f32x4* src = reinterpret_cast<const f32x4*>(part_acc) + ws * 1024 + lane;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const uint64_t* s = reinterpret_cast<const uint64_t*>(src + (dt * 2 + g) * 64);
      union { f32x4 f; uint64_t u[2]; } x;
      x.u[0] = __hip_atomic_load(s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      x.u[1] = __hip_atomic_load(s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      res[dt][g] = first ? x.f : res[dt][g] + x.f;
    }
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float v = __hip_atomic_load(part_l + ws * 64 + g * 16 + (lane & 15), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    rl[g] = first ? v : rl[g] + v;
  }
}

__global__ __launch_bounds__(kThreads, 2) void attend_balanced_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, int length, int q_blocks, int units,
    int heads, int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride,
    float* __restrict__ part_acc, float* __restrict__ part_l, int* __restrict__ counters, unsigned epoch) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kSmemBytes];
  __shared__ int arrival;
  __shared__ unsigned counter_seen;   // the counter's value when this piece checked it
  constexpr int C = kCUs / kXcds;
  const int x = blockIdx.x % kXcds, l = blockIdx.x / kXcds;   // hardware deals blocks round-robin over XCDs
  const int ntiles = (length + kBN - 1) / kBN;
  const XcdSplit xs = xcd_split(units, ntiles, x);
  const int left0 = xs.ux0 + xs.R * C;   // first leftover tile of this XCD

  // Segments: the whole tiles of the full rounds, then this CU's leftover range, one
  // segment per tile it touches (i = the leftover tile, -1 for a whole tile).
  int u = l < xs.P ? range_start(xs, l) : 0;
  const int u_end = l < xs.P ? range_start(xs, l + 1) : 0;
  for (int sg = 0;; ++sg) {
    int unit, t0 = 0, t1 = ntiles, i = -1;
    if (sg < xs.R) {
      unit = xs.ux0 + sg * C + l;
    } else {
      if (u >= u_end) break;
      i = u / ntiles;
      t0 = u - i * ntiles;
      t1 = min(ntiles, t0 + (u_end - u));
      u += t1 - t0;
      unit = left0 + i;
    }
    const int bh = unit / q_blocks, qblk = unit - bh * q_blocks;
    __syncthreads();   // every wave is done with the previous segment's LDS
    const int q0 = qblk * kBM + (threadIdx.x >> 6) * 32;
    WaveState<2> w;
    attend_segment(w, smem, q, k, v, length, bh, q0, t0, t1);
    float ls[2];
    row_sums(w, ls);
    const int cf = i < 0 ? 0 : range_of(xs, i * ntiles);
    const int cl = i < 0 ? 0 : range_of(xs, (i + 1) * ntiles - 1);
    if (cf == cl) {   // a whole tile of one range
      store_o(w, ls, o, bh, heads, q0, length, o_batch_stride, o_head_stride, o_row_stride);
      continue;
    }
    const int others = cl - cf, pos = l - cf;
    auto slot_of = [&](int c) {
      return (int64_t)(x * C + c) * 2 + (i - range_start(xs, c) / ntiles);
    };
    int* counter = &counters[x * C + i];
    const int pieces = others + 1;
    if (threadIdx.x == 0) {
      counter_seen = (unsigned)__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      arrival = arrivals_of(counter_seen, epoch, pieces);
    }
    __syncthreads();
    // Publish unless every other piece already has and this piece is one of the first two
    // (whose sum is the same in either order, so it can start from its registers).
    if (arrival < others || pos >= 2) {
      store_partial<true>(w, ls, part_acc, part_l, slot_of(l));
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();   // every wave's stores have completed before the arrival
      if (threadIdx.x == 0) arrival = arrive(counter, epoch, pieces, counter_seen);
      __syncthreads();
      if (arrival < others) continue;   // a later piece writes O
    } else if (threadIdx.x == 0) {
      arrive(counter, epoch, pieces, counter_seen);   // the count completes: a replay with this epoch starts afresh
    }
    // Last piece: O = ((p_cf + p_cf+1) + p_cf+2) + ..., the pieces in CU order.
    if (pos <= 1) {
      gather_partial(w.oacc, ls, false, part_acc, part_l, slot_of(pos == 0 ? cf + 1 : cf));
      for (int c = cf + 2; c <= cl; ++c) gather_partial(w.oacc, ls, false, part_acc, part_l, slot_of(c));
    } else {
      for (int c = cf; c <= cl; ++c) gather_partial(w.oacc, ls, c == cf, part_acc, part_l, slot_of(c));
    }
    store_o(w, ls, o, bh, heads, q0, length, o_batch_stride, o_head_stride, o_row_stride);
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
  const int qw = (i & 1) * 16 + (lane & 15);   // query within the wave: group i % 2, column lane % 16
  const int qi = qblk * kBM + wave * 32 + qw;
  if (qi >= length) return;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
#pragma unroll 4
  for (int s = 0; s < splits; ++s) {
    acc += reinterpret_cast<const f32x4*>(part_acc)[s * units * 8192 + id];
    l += part_l[(s * units + unit) * 512 + wave * 64 + qw];
  }
  const int64_t b = bh / heads, h = bh - b * heads;
  const int d0 = (i >> 1) * 16 + (lane >> 4) * 4;
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
  // Query and key positions up to a tile past the end stay within int in the kernels.
  if (length > INT32_MAX - kBM) return FLK_E_INVALID;
  if (((int64_t)length + kBM - 1) / kBM * batch * heads > INT32_MAX) return FLK_E_INVALID;
  return FLK_OK;
}

int64_t q_tiles(int length) { return ((int64_t)length + kBM - 1) / kBM; }
int key_groups(int length) { return (int)((((int64_t)length + kBN - 1) / kBN + 3) / 4); }

// Workspace of a split launch: per split and (b, h, 256-query tile), 512 lanes x (64 acc + 1 l)
// floats.
int64_t split_workspace_bytes(int batch, int heads, int length, int splits) {
  return (int64_t)splits * batch * heads * q_tiles(length) * kThreads * 65 * (int64_t)sizeof(float);
}

// 192-query tiles when the grid fits the CUs in one round with them as with 256-query tiles:
// the launch then takes the time of one block, and a 192-query block does 3/4 of the work.
int64_t q_tiles192(int length) { return ((int64_t)length + kBM192 - 1) / kBM192; }

bool tile192_preferred(int batch, int heads, int length) {
  const int64_t bh = (int64_t)batch * heads;
  return q_tiles(length) * bh <= kCUs && q_tiles192(length) * bh <= kCUs;
}

// Grid of the rounds launch (attend_rounds_kernel), or 0 when it is not the choice: it needs
// a full round of 256-query tiles on every XCD, tiles left over, and at most one round (32
// per XCD) of 192-query tiles for them.
int64_t rounds_grid(int batch, int heads, int length) {
  constexpr int C = kCUs / kXcds;
  const int64_t units = q_tiles(length) * batch * heads;
  if (units < kCUs || units > INT32_MAX) return 0;
  const int64_t qb = q_tiles(length);
  int64_t most = 0, left_max = 0;
  for (int x = 0; x < kXcds; ++x) {
    const int64_t ux0 = x * units / kXcds, n = (x + 1) * units / kXcds - ux0;
    const int64_t full = n / C * C;
    int64_t count = 0;
    for (int64_t u = ux0 + full; u < ux0 + n;) {   // as leftover_tile walks them
      const int64_t b = u / qb, t0 = u - b * qb, t1 = std::min(qb, t0 + (ux0 + n - u));
      const int64_t e = std::min<int64_t>(t1 * kBM, length);
      count += (e - t0 * kBM + kBM192 - 1) / kBM192;
      u += t1 - t0;
    }
    if (count > C) return 0;
    left_max = std::max(left_max, n - full);
    most = std::max(most, full + count);
  }
  return left_max > 0 ? most * kXcds : 0;
}

int launch_attend(const void* q, const void* k, const void* v, void* o, int batch, int heads, int length,
                  int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride, void* stream) {
  if (const int64_t grid = rounds_grid(batch, heads, length)) {
    hipLaunchKernelGGL(attend_rounds_kernel, dim3((unsigned)grid), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<uint16_t*>(o), length, (int)q_tiles(length),
                       (int)(q_tiles(length) * batch * heads), heads, o_batch_stride, o_head_stride,
                       o_row_stride);
    return flk_launch_status();
  }
  if (tile192_preferred(batch, heads, length)) {
    const int64_t total = q_tiles192(length) * batch * heads;
    hipLaunchKernelGGL(attend_tile192_kernel, dim3((unsigned)total), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<uint16_t*>(o), length, (int)q_tiles192(length), (int)total, heads,
                       o_batch_stride, o_head_stride, o_row_stride);
    return flk_launch_status();
  }
  const int64_t total = q_tiles(length) * batch * heads;
  hipLaunchKernelGGL(attend_kernel<false>, dim3((unsigned)total), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(o), length, (int)q_tiles(length), (int)total, heads, 1,
                     o_batch_stride, o_head_stride, o_row_stride, nullptr, nullptr);
  return flk_launch_status();
}

}  // namespace

extern "C" const char* flk_attend_kernel(int batch, int heads, int length) {
  if (batch <= 0 || heads <= 0 || length <= 0) return "";
  if (rounds_grid(batch, heads, length)) return "attend_rounds_kernel";
  if (tile192_preferred(batch, heads, length)) return "attend_tile192_kernel";
  return "attend_kernel";
}

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

namespace {

// Workspace of a balanced launch on `grid` blocks: two partial slots per block, one per
// leftover segment (acc: 8 waves x 1024 float4; l: 8 waves x 64 floats), then one int counter
// per leftover tile (fewer than 32 per XCD, so `grid` counters).
constexpr int64_t kSlotAccBytes = (int64_t)kWaves * 1024 * 16;
constexpr int64_t kSlotLBytes = (int64_t)kWaves * 64 * 4;

int64_t balanced_counters_offset(int grid) { return 2 * (int64_t)grid * (kSlotAccBytes + kSlotLBytes); }
int64_t balanced_workspace_bytes(int grid) { return balanced_counters_offset(grid) + 4 * (int64_t)grid; }

// Whether the balanced launch beats the rounds launch (one block per 256-query tile, the
// tiles an XCD has left after its full rounds of 32 re-tiled by 192 queries), by those
// leftover tiles of the fullest XCD: it does when every XCD has at least one full round, at
// most 16 tiles are left over and each CU's share of their keys is at least 16 key tiles
// (measured against the rounds launch: 6% at 8 left over, 2-5% at 11-12, 1% at 13; the
// rounds launch 2% faster at 19 left over, and 20% at 4 left over of 24 key tiles each,
// whose shares of 3 key tiles spend more on hand-offs than on keys).
bool balanced_preferred(int batch, int heads, int length) {
  const int64_t units = q_tiles(length) * batch * heads;
  constexpr int C = kCUs / kXcds;
  const int64_t key_tiles = ((int64_t)length + kBN - 1) / kBN;
  if (units < kCUs || units > INT32_MAX || key_tiles * 1024 > INT32_MAX) return false;
  const int64_t left = ((units + kXcds - 1) / kXcds) % C;   // leftover tiles of the fullest XCD
  return left > 0 && left <= 16 && left * key_tiles >= 16 * C;
}

}  // namespace

extern "C" int flk_attend_balanced_plan(int batch, int heads, int length, int* grid, int64_t* workspace_bytes,
                                        int64_t* counters_offset) {
  if (batch < 0 || heads < 0 || length < 0 || !grid || !workspace_bytes || !counters_offset) return FLK_E_INVALID;
  *grid = balanced_preferred(batch, heads, length) ? kCUs : 0;
  *workspace_bytes = balanced_workspace_bytes(kCUs);
  *counters_offset = balanced_counters_offset(kCUs);
  return FLK_OK;
}

extern "C" int flk_attend_balanced_to(const void* q, const void* k, const void* v, void* o, int batch, int heads,
                                      int length, int head_dim, int64_t o_batch_stride, int64_t o_head_stride,
                                      int64_t o_row_stride, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  const int st = check_attend(q, k, v, o, batch, heads, length, head_dim, o_batch_stride, o_head_stride,
                              o_row_stride);
  if (st != FLK_OK) return st == kNothing ? FLK_OK : st;
  const int64_t units = q_tiles(length) * batch * heads;   // <= INT32_MAX (check_attend)
  if (((int64_t)length + kBN - 1) / kBN * 1024 > INT32_MAX) return FLK_E_UNSUPPORTED;   // 32-bit split math
  constexpr int grid = kCUs;
  if (!workspace || workspace_bytes < balanced_workspace_bytes(grid)) return FLK_E_INVALID;
  if (!flk_host_aligned(workspace, 16)) return FLK_E_ALIGN;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* part_acc = reinterpret_cast<float*>(ws);
  float* part_l = reinterpret_cast<float*>(ws + 2 * (int64_t)grid * kSlotAccBytes);
  int* counters = reinterpret_cast<int*>(ws + balanced_counters_offset(grid));
  // This call's counter tag: 1 .. 2^24 - 1 in turn (0 is what a zeroed workspace holds).
  static std::atomic<unsigned> next_epoch{0};
  const unsigned epoch = next_epoch.fetch_add(1, std::memory_order_relaxed) % kEpochMask + 1;
  hipLaunchKernelGGL(attend_balanced_kernel, dim3((unsigned)grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(o), length, (int)q_tiles(length), (int)units, heads, o_batch_stride,
                     o_head_stride, o_row_stride, part_acc, part_l, counters, epoch);
  return flk_launch_status();
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
