// Shared device helpers for the gfx950 (MI355X, CDNA4) kernels of flicker_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flicker_hip.h"

namespace flk {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// bf16 bit pattern <-> float32 (exact widening).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Two float32 -> packed bf16x2 (round to nearest even; v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 p = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, p);
}

// float32 -> nearest bf16 value, widened back to float32.
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

// Butterfly sum over one 16-lane DPP row.  Every lane of the row ends with the same bit
// pattern (each step adds two commuted partial sums).
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)); // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
  return v;
}

// Copy 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane i of the wave lands at lds_dst + 16 i, where lds_dst must be wave-uniform.  Issued
// from inline asm so the compiler does not order later LDS reads behind it (it cannot
// prove the destination disjoint from them); callers wait with s_waitcnt vmcnt.  The LDS
// address is an M0 operand ("{m0}"), so the compiler writes M0 itself and knows it is in use;
// the s_nop is the wait state an M0 write needs before an LDS DMA reads it.
__device__ __forceinline__ void dma16(const void* src, const uint8_t* lds_dst) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" :: "{m0}"(lds), "v"(src) : "memory");
}

// The same copy from a wave-uniform base (scalar registers) plus a 32-bit per-lane byte
// offset: one VGPR per source instead of a 64-bit address.
__device__ __forceinline__ void dma16_at(const void* base, uint32_t voff, const uint8_t* lds_dst) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_dst);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" :: "{m0}"(lds), "v"(voff), "s"(base) : "memory");
}

__device__ __forceinline__ bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace flk

// Host-side helpers shared by the C-ABI launchers.
static inline bool flk_host_aligned(const void* p, unsigned bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

static inline int flk_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FLK_OK : (int)e;
}
