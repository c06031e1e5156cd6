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

}  // namespace dsmoe
