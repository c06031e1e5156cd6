// gfx950 MFMA operand types and the LDS tile layout shared by the grouped
// GEMM kernels (forward gemm.hip, backward gemm_xm.hip).
#pragma once

#include "common.h"

namespace dsmoe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));  // native vector: stays in registers
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// 16-byte load through a global-address-space pointer.  Pointers read from
// device tables are generic to the compiler, which would emit flat loads;
// flat loads also count against the LDS wait counter, so a wait for LDS
// fragments would wait for the next slab's prefetch as well.
typedef __attribute__((address_space(1))) const u32x4_t gu32x4_t;
__device__ __forceinline__ u32x4_t ldg16(const bf16_t* p) { return *(gu32x4_t*)(p); }

constexpr int MF_K = 64;  // K slab per pipeline stage (8 chunks of 16 bytes per row)

// LDS tile row = 64 bf16 of K = 128 bytes = 8 chunks of 16 bytes.  gfx950
// serves a ds_read_b128 16 lanes (256 bytes, two rows) per cycle; chunk c of
// row r is stored at c ^ ((r >> 1) & 7), so the 16 rows read at one logical
// chunk by a fragment load land on 16 distinct 16-byte bank groups.
// Returns the element offset of chunk c of row r.
__device__ __forceinline__ int swz(int row, int chunk) { return row * MF_K + ((chunk ^ ((row >> 1) & 7)) << 3); }

// s_waitcnt immediate (gfx9 encoding) waiting until at most n vector-memory
// operations of this wave are outstanding; lgkm/exp counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Waits until every LDS (and scalar-memory) operation of this wave has
// completed; vector-memory and export counters unconstrained.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }

// Workgroup barrier without the memory fences of __syncthreads(): those would
// wait for every in-flight direct load.  Ordering is explicit instead: each
// wave waits for its own loads of the slab (wait_vm), then all waves meet
// here; the asm memory clobber keeps the compiler from moving LDS accesses
// across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Direct global -> LDS load of 16 bytes per lane (gfx950
// global_load_lds_dwordx4): lane i's 16 bytes land at LDS byte address
// lds_base + 16 i; lds_base must be wave-uniform (it is passed in M0).
// Issued as inline asm: the compiler models the builtin's LDS write as an
// out-of-order LDS event and then turns every wait for an ordinary LDS read
// into a full drain.  The caller tracks completion with explicit vmcnt waits
// (wait_vm) instead; the s_nop is the wait state the hardware needs between
// writing M0 and an LDS-DMA load that reads it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "{m0}"(lds_base) : "memory");
}

// The same load addressed as a wave-uniform 64-bit base (SGPRs) plus a
// 32-bit per-lane byte offset: no 64-bit address arithmetic in VGPRs, and the
// per-lane offsets stay 32-bit registers.
__device__ __forceinline__ void dma16s(const char* base, uint32_t off, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(lds_base) : "memory");
}

// Two fp32 values rounded to nearest-even bf16 and packed (lo = a), one
// v_cvt_pk_bf16_f32 on gfx950.
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// LDS byte address of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

}  // namespace dsmoe
