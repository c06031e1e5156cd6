// Grouped NT GEMM with direct global->LDS loads (gfx950 global_load_lds_dwordx4).
//
// Same contract and tile enumeration as gemm_mfma_kernel (gemm.hip).  Block
// tile 256 x 256 (SwiGLU: 256 rows x 128 columns of W1 and of W3), 4 waves in
// a 2 x 2 grid, each wave 128 x 128 outputs (16 MFMA 32x32x16 tiles, 256 fp32
// accumulators).  K advances in slabs of 32; slabs stream straight from global
// memory into a 4-deep LDS ring (no staging registers), issued three slabs
// ahead of the one being multiplied.  One barrier per slab; LDS fragment
// reads run one MFMA group ahead of their use.
//
// LDS rows are 64 bytes (4 chunks of 16 bytes); chunk c of row r is stored at
// chunk c ^ ((r >> 2) & 3).  gfx950 serves a ds_read_b128 16 lanes (256 bytes,
// four rows) per cycle, and the 16 rows read at one logical chunk then land on
// 16 different 16-byte bank groups.  A direct load writes 64
// consecutive 16-byte LDS chunks per wave instruction, lane i to chunk i, so
// each lane fetches the global chunk that belongs at its LDS position.
#include <cstdlib>

#include "gemm_tile.h"

namespace dsmoe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 dl_bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float dl_f32x16_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

constexpr int DL_BM = 256;
constexpr int DL_BK = 32;
constexpr int DL_STAGES = 4;
constexpr int DL_MAX_SEG = 2;            // K segments of B (shared experts summed in one GEMM)
constexpr int DL_ROWB = DL_BK * 2;            // bytes per LDS row
constexpr int DL_TILE_B = 256 * DL_ROWB;      // bytes of one 256-row operand slab
constexpr int DL_STAGE_B = 2 * DL_TILE_B;     // A slab + B slab
constexpr size_t DL_LDS = (size_t)DL_STAGES * DL_STAGE_B;

// s_waitcnt immediate (gfx9 encoding) waiting until at most n vector-memory
// operations of this wave are outstanding; lgkm/exp counters unconstrained.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without the memory fences of __syncthreads(): those would
// wait for every in-flight direct load.  Ordering is explicit instead: each
// wave waits for its own loads of the slab (wait_vm), then all waves meet
// here; the asm memory clobber keeps the compiler from moving LDS accesses
// across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ int dl_swz_byte(int r, int c) { return r * DL_ROWB + ((c ^ ((r >> 2) & 3)) << 4); }

template <int EPI>
__global__ __launch_bounds__(256) void gemm_dl_kernel(const GemmDesc g, const float* __restrict__ row_scale) {
  constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int TM = 4;
  constexpr int TN = (EPI == EPI_SWIGLU) ? 2 : 4;   // per B operand
  constexpr int BN = 2 * TN * 32;                    // output columns per block
  extern __shared__ __attribute__((aligned(16))) char dl_smem[];

  const int n_tiles = (int)cdiv(g.N, BN);
  int grp, row0, rows, n_tile;
  if (!tile_for_block<DL_BM>(g, n_tiles, grp, row0, rows, n_tile)) return;
  // wave-uniform from here on: lets the B pointer tables load through the
  // scalar cache (lgkm counter) instead of the vector path
  grp = __builtin_amdgcn_readfirstlane(grp);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rows = __builtin_amdgcn_readfirstlane(rows);
  n_tile = __builtin_amdgcn_readfirstlane(n_tile);
  const int n0 = n_tile * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- per-lane sources of the 4 A and 4 B direct loads of every slab.
  // Instruction i of wave w fills LDS chunks p = (4w + i) * 64 + lane, i.e.
  // row r = p >> 2 at physical chunk p & 3 (logical chunk (p & 3) ^ ((r >> 2) & 3)).
  // Offsets are 32-bit element offsets from uniform base pointers (the host
  // checks that every operand spans fewer than 2^31 elements).
  const bf16_t* __restrict__ A = static_cast<const bf16_t*>(g.A);
  uint32_t a_off[4];
  uint32_t b_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = (wave * 4 + i) * 64 + lane;
    const int r = p >> 2;
    const int c = (p & 3) ^ ((r >> 2) & 3);
    const int ra = min(r, rows - 1);
    const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + ra] : (int64_t)(row0 + ra);
    a_off[i] = (uint32_t)(arow * g.lda + c * 8);
    const int bn = (NB == 2) ? n0 + (r & 127) : n0 + r;   // SwiGLU: rows 0..127 W1, 128..255 W3
    b_off[i] = (uint32_t)((int64_t)min(bn, g.N - 1) * g.ldb + c * 8);
  }
  // B base pointers of the (at most two) K segments, read before the first
  // direct load so that no table read waits behind them.  Kept as separate
  // scalars: an array here would be indexed from memory.
  const void* const* tab0 = g.B0 + (int64_t)grp * g.nseg;
  const void* const* tab1 = (NB == 2) ? g.B1 + (int64_t)grp * g.nseg : tab0;
  const int last = g.nseg - 1;
  const bf16_t* const b0s0 = static_cast<const bf16_t*>(tab0[0]);
  const bf16_t* const b0s1 = static_cast<const bf16_t*>(tab0[last]);
  const bf16_t* const b1s0 = static_cast<const bf16_t*>(tab1[0]);
  const bf16_t* const b1s1 = static_cast<const bf16_t*>(tab1[last]);
  const int nk = g.K / DL_BK;

  auto issue = [&](int kb) {
    const int k0 = kb * DL_BK;
    const bool hi = k0 >= g.kseg;
    const int kin = hi ? k0 - g.kseg : k0;
    char* st = dl_smem + (kb & (DL_STAGES - 1)) * DL_STAGE_B;
    const bf16_t* b0 = hi ? b0s1 : b0s0;
    const bf16_t* b1 = hi ? b1s1 : b1s0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds((const glb_void_t*)(A + a_off[i] + k0),
                                       (lds_void_t*)(st + (wave * 4 + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // instruction i of wave w covers B rows 64w + 16i .. +15: W3 when >= 128
      const bf16_t* bb = (NB == 2 && (wave * 4 + i) >= 8) ? b1 : b0;
      __builtin_amdgcn_global_load_lds((const glb_void_t*)(bb + b_off[i] + kin),
                                       (lds_void_t*)(st + DL_TILE_B + (wave * 4 + i) * 1024), 16, 0, 0);
    }
  };

  dl_f32x16_t acc[NB][TM][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int ni = 0; ni < TN; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[b][mi][ni][r] = 0.0f;

  // Fragment reads of one 16-wide K step (kk) of slab kb into (fa, fb).
  auto read_frags = [&](int kb, int kk, dl_bf16x8_t (&fa)[TM], dl_bf16x8_t (&fb)[NB][TN]) {
    const char* sA = dl_smem + (kb & (DL_STAGES - 1)) * DL_STAGE_B;
    const char* sB = sA + DL_TILE_B;
    const int c = kk * 2 + (lane >> 5);
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
      fa[mi] = *reinterpret_cast<const dl_bf16x8_t*>(sA + dl_swz_byte(wm * 128 + mi * 32 + (lane & 31), c));
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int ni = 0; ni < TN; ++ni) {
        const int r = (NB == 2 ? b * 128 + wn * 64 : wn * 128) + ni * 32 + (lane & 31);
        fb[b][ni] = *reinterpret_cast<const dl_bf16x8_t*>(sB + dl_swz_byte(r, c));
      }
  };
  auto mma = [&](const dl_bf16x8_t (&fa)[TM], const dl_bf16x8_t (&fb)[NB][TN]) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int mi = 0; mi < TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < TN; ++ni)
          acc[b][mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][ni], fa[mi], acc[b][mi][ni], 0, 0, 0);
  };

  // Pipeline (per slab kb, two K steps kk0 / kk1 held in register sets F0 / F1):
  //   read F1(kb); MMA F0(kb); [wait slab kb+1; barrier; DMA slab kb+3; read F0(kb+1)]; MMA F1(kb)
  // LDS reads are always issued one MFMA group ahead.  The DMA of slab kb+3
  // reuses the buffer of slab kb-1, whose last reads completed before every
  // wave passed this slab's barrier (they fed MMA F1(kb-1)).
  dl_bf16x8_t fa0[TM], fa1[TM];
  dl_bf16x8_t fb0[NB][TN], fb1[NB][TN];
  issue(0);
  if (nk > 1) issue(1);
  if (nk > 2) issue(2);
  if (nk > 2)
    wait_vm<16>();
  else if (nk > 1)
    wait_vm<8>();
  else
    wait_vm<0>();
  lds_barrier();
  read_frags(0, 0, fa0, fb0);
  for (int kb = 0; kb < nk; ++kb) {
    read_frags(kb, 1, fa1, fb1);
    mma(fa0, fb0);
    if (kb + 1 < nk) {
      if (kb + 2 < nk)
        wait_vm<8>();
      else
        wait_vm<0>();
      lds_barrier();
      if (kb + 3 < nk) issue(kb + 3);
      read_frags(kb + 1, 0, fa0, fb0);
    }
    mma(fa1, fb1);
  }

  // ---- epilogue (same register layout as gemm_mfma_kernel)
  bf16_t* C = static_cast<bf16_t*>(g.C);
  const int64_t ccol = (int64_t)grp * g.c_group_col;
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) {
    const int m = wm * 128 + mi * 32 + (lane & 31);
    if (m >= rows) continue;
    const int64_t crow = g.c_map ? (int64_t)g.c_map[row0 + m] : (int64_t)(row0 + m);
    float scale = 1.0f;
    if (EPI == EPI_STORE && row_scale) scale = row_scale[row0 + m];
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + (NB == 2 ? wn * 64 : wn * 128) + ni * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        const int64_t o = crow * g.ldc + ccol + n;
        uint32_t packed[2];
        if (EPI == EPI_SWIGLU) {
          uint32_t pg[2], pu[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float g0 = acc[0][mi][ni][q * 4 + 2 * h], g1 = acc[0][mi][ni][q * 4 + 2 * h + 1];
            const float u0 = acc[NB - 1][mi][ni][q * 4 + 2 * h], u1 = acc[NB - 1][mi][ni][q * 4 + 2 * h + 1];
            packed[h] = (uint32_t)f2bf(silu_f(g0) * u0) | ((uint32_t)f2bf(silu_f(g1) * u1) << 16);
            pg[h] = (uint32_t)f2bf(g0) | ((uint32_t)f2bf(g1) << 16);
            pu[h] = (uint32_t)f2bf(u0) | ((uint32_t)f2bf(u1) << 16);
          }
          if (g.Gs) *reinterpret_cast<uint2*>(static_cast<bf16_t*>(g.Gs) + o) = make_uint2(pg[0], pg[1]);
          if (g.Us) *reinterpret_cast<uint2*>(static_cast<bf16_t*>(g.Us) + o) = make_uint2(pu[0], pu[1]);
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float v0 = acc[0][mi][ni][q * 4 + 2 * h] * scale, v1 = acc[0][mi][ni][q * 4 + 2 * h + 1] * scale;
            packed[h] = (uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16);
          }
        }
        *reinterpret_cast<uint2*>(C + o) = make_uint2(packed[0], packed[1]);
      }
    }
  }
}

// Requirements beyond the register-staged kernel: at most DL_MAX_SEG K
// segments; K and the K segment are multiples of 32 (implied by the 64 the
// caller checks).
bool gemm_dl_ok(const GemmDesc& g, int64_t a_rows) {
  const int64_t lim = int64_t(1) << 31;
  return g.nseg >= 1 && g.nseg <= DL_MAX_SEG && a_rows * g.lda < lim && (int64_t)g.N * g.ldb < lim;
}

int launch_gemm_dl(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st) {
  const int bn = (epi == EPI_SWIGLU) ? 128 : 256;
  const int64_t m_bound = g.sched ? g.m_tiles_bound : cdiv(g.dense_rows, DL_BM) * g.groups;
  const int64_t grid = 8 * cdiv(m_bound * cdiv(g.N, bn), 8);
  if (grid == 0) return DSMOE_OK;
  if (epi == EPI_SWIGLU) {
    static bool a = false;
    if (!a && hipFuncSetAttribute((const void*)gemm_dl_kernel<EPI_SWIGLU>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)DL_LDS) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "gemm_dl: cannot raise LDS limit");
    a = true;
    hipLaunchKernelGGL(gemm_dl_kernel<EPI_SWIGLU>, dim3((unsigned)grid), dim3(256), DL_LDS, st, g, row_scale);
  } else {
    static bool a = false;
    if (!a && hipFuncSetAttribute((const void*)gemm_dl_kernel<EPI_STORE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)DL_LDS) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "gemm_dl: cannot raise LDS limit");
    a = true;
    hipLaunchKernelGGL(gemm_dl_kernel<EPI_STORE>, dim3((unsigned)grid), dim3(256), DL_LDS, st, g, row_scale);
  }
  return check_launch("gemm_dl");
}

}  // namespace dsmoe
