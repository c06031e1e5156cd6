// Measurement probe (no counterpart in the reference), built into its own
// library (libdsmoe_probe.so, declared in dsmoe_probe.h): reads an exact byte
// count from global memory with the direct global -> LDS loads the grouped
// GEMMs issue (global_load_lds_dwordx4), so the per-dispatch reading of a
// traffic counter (FETCH_SIZE) can be set against the bytes actually read.
#include "dsmoe_probe.h"
#include "common.h"
#include "mfma.h"

namespace dsmoe {

constexpr int64_t PROBE_CHUNK = 1 << 20;   // bytes read by one workgroup

// Workgroup b reads bytes [b, b + 1) MiB of src once: wave w loads the 1 KB
// pieces w, w + 4, ... into a 4-slot LDS ring of its own (the values are not
// used), then one word of the ring goes to sink[b] so the loads stay live.
__global__ __launch_bounds__(256) void probe_dma_kernel(const char* __restrict__ src, uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(16))) char ring[16 * 1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const char* base = src + (int64_t)blockIdx.x * PROBE_CHUNK;
  const uint32_t slot0 = lds_addr(ring) + wave * 4096;
  int i = 0;
  for (uint32_t off = wave * 1024; off < (uint32_t)PROBE_CHUNK; off += 4096, ++i) {
    dma16s(base, off + lane * 16, slot0 + (i & 3) * 1024);
    if ((i & 7) == 7) wait_vm<8>();
  }
  wait_vm<0>();
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = *reinterpret_cast<const uint32_t*>(ring);
}

}  // namespace dsmoe

extern "C" int dsmoe_probe_dma_read(const void* src, size_t bytes, uint32_t* sink, void* stream) {
  if (!src || !sink || bytes == 0 || bytes % dsmoe::PROBE_CHUNK != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
    return -1;
  hipLaunchKernelGGL(dsmoe::probe_dma_kernel, dim3((unsigned)(bytes / dsmoe::PROBE_CHUNK)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const char*>(src), sink);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
