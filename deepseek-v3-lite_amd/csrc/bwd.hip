// Backward helpers of the MoE layer (autograd of models/moe.py:29-37,74-133).
//
//   dw_dot_kernel    d weights[t, j] = <dy[t], o[t*k+j]>  (gradient of the
//                    routed combine out * weight, models/moe.py:132)
//   gate_bwd_kernel  renormalisation and sigmoid backward (models/moe.py:32-36):
//                    w_j = s_j / Z * rs  =>  ds_i = rs (dw_i / Z - sum_j dw_j s_j / Z^2),
//                    dlogit_i = ds_i s_i (1 - s_i); only the k selected experts
//                    of a token get a gradient, the bias none.
//   dwgate_kernel    dW_gate[e] = sum over rows routed to e (ascending sorted
//                    position) of dlogit * x[token]: a deterministic segmented
//                    reduction over the sorted order.
//   dx_final_kernel  dx[t] = sum_j (ascending expert id) dx_slot[t*k+j]
//                    + dx_shared[t] + sum_j dlogit[t,j] W_gate[e_j], fp32, one rounding.
#include "common.h"

namespace dsmoe {

template <typename T>
__global__ __launch_bounds__(256) void dw_dot_kernel(const T* __restrict__ dy, const T* __restrict__ o_slots, int64_t N,
                                                     int k, int D, float* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= N) return;
  const int64_t t = s / k;
  const T* a = dy + t * D;
  const T* b = o_slots + s * D;
  float acc = 0.0f;
  for (int d = lane; d < D; d += 64) acc = fmaf(to_f<T>(a[d]), to_f<T>(b[d]), acc);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) dw[s] = acc;
}

__global__ __launch_bounds__(256) void gate_bwd_kernel(const float* __restrict__ dw, const float* __restrict__ sel,
                                                       int T, int k, float route_scale, float* __restrict__ dlog) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float* dwt = dw + (int64_t)t * k;
  const float* st = sel + (int64_t)t * k;
  float z = 0.0f, c = 0.0f;
  for (int j = 0; j < k; ++j) z += st[j];
  for (int j = 0; j < k; ++j) c = fmaf(dwt[j], st[j], c);
  const bool clamped = z < 1e-10f;
  const float den = clamped ? 1e-10f : z;
  for (int j = 0; j < k; ++j) {
    const float ds = clamped ? route_scale * dwt[j] / den : route_scale * (dwt[j] / den - c / (den * den));
    dlog[(int64_t)t * k + j] = ds * st[j] * (1.0f - st[j]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void dwgate_kernel(const T* __restrict__ x, const float* __restrict__ dlog,
                                                     const int32_t* __restrict__ sorted_slot,
                                                     const int32_t* __restrict__ sorted_token,
                                                     const int32_t* __restrict__ offsets, int D,
                                                     float* __restrict__ dgw) {
  const int e = blockIdx.y;
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= D) return;
  const int p0 = offsets[e], p1 = offsets[e + 1];
  float acc = 0.0f;
  for (int p = p0; p < p1; ++p) acc = fmaf(dlog[sorted_slot[p]], to_f<T>(x[(int64_t)sorted_token[p] * D + d]), acc);
  dgw[(int64_t)e * D + d] = acc;
}

template <typename T>
__global__ __launch_bounds__(256) void dx_final_kernel(const T* __restrict__ dx_slots, const T* __restrict__ dx_shared,
                                                       const float* __restrict__ dlog, const int32_t* __restrict__ idx,
                                                       const float* __restrict__ gw, int Tn, int D, int k,
                                                       T* __restrict__ dx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)Tn * D) return;
  const int64_t t = i / D;
  const int d = (int)(i - t * D);
  int ord[MAX_TOPK], ev[MAX_TOPK];
  for (int j = 0; j < k; ++j) {  // ascending expert id (insertion sort, k <= 16)
    const int e = idx[t * k + j];
    int p = j;
    while (p > 0 && ev[p - 1] > e) {
      ev[p] = ev[p - 1];
      ord[p] = ord[p - 1];
      --p;
    }
    ev[p] = e;
    ord[p] = j;
  }
  float acc = 0.0f;
  for (int q = 0; q < k; ++q) acc += to_f<T>(dx_slots[(t * k + ord[q]) * (int64_t)D + d]);
  if (dx_shared) acc += to_f<T>(dx_shared[t * (int64_t)D + d]);
  for (int q = 0; q < k; ++q) acc = fmaf(dlog[t * k + ord[q]], gw[(int64_t)ev[q] * D + d], acc);
  dx[t * (int64_t)D + d] = from_f<T>(acc);
}

// ---------------------------------------------------------------- launchers
int launch_dw_dot(const void* dy, const void* o_slots, int64_t N, int k, int D, int dtype, float* dw,
                  hipStream_t st) {
  if (N == 0) return DSMOE_OK;
  const unsigned grid = (unsigned)cdiv(N, 4);
  if (dtype == DSMOE_BF16)
    hipLaunchKernelGGL(dw_dot_kernel<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(dy),
                       static_cast<const bf16_t*>(o_slots), N, k, D, dw);
  else
    hipLaunchKernelGGL(dw_dot_kernel<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(dy),
                       static_cast<const float*>(o_slots), N, k, D, dw);
  return check_launch("dw_dot");
}

int launch_gate_bwd(const float* dw, const float* sel, int T, int k, float rs, float* dlog, hipStream_t st) {
  if (T == 0) return DSMOE_OK;
  hipLaunchKernelGGL(gate_bwd_kernel, dim3((unsigned)cdiv(T, 256)), dim3(256), 0, st, dw, sel, T, k, rs, dlog);
  return check_launch("gate_bwd");
}

int launch_dwgate(const void* x, const float* dlog, const int32_t* sorted_slot, const int32_t* sorted_token,
                  const int32_t* offsets, int E, int D, int dtype, float* dgw, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(D, 256), (unsigned)E);
  if (dtype == DSMOE_BF16)
    hipLaunchKernelGGL(dwgate_kernel<bf16_t>, grid, dim3(256), 0, st, static_cast<const bf16_t*>(x), dlog, sorted_slot,
                       sorted_token, offsets, D, dgw);
  else
    hipLaunchKernelGGL(dwgate_kernel<float>, grid, dim3(256), 0, st, static_cast<const float*>(x), dlog, sorted_slot,
                       sorted_token, offsets, D, dgw);
  return check_launch("dwgate");
}

int launch_dx_final(const void* dx_slots, const void* dx_shared, const float* dlog, const int32_t* idx, const float* gw,
                    int T, int D, int k, int dtype, void* dx, hipStream_t st) {
  if (T == 0) return DSMOE_OK;
  const unsigned grid = (unsigned)cdiv((int64_t)T * D, 256);
  if (dtype == DSMOE_BF16)
    hipLaunchKernelGGL(dx_final_kernel<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(dx_slots),
                       static_cast<const bf16_t*>(dx_shared), dlog, idx, gw, T, D, k, static_cast<bf16_t*>(dx));
  else
    hipLaunchKernelGGL(dx_final_kernel<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(dx_slots),
                       static_cast<const float*>(dx_shared), dlog, idx, gw, T, D, k, static_cast<float*>(dx));
  return check_launch("dx_final");
}

// Schedule of height bm from int32 offsets (E + 1) already in device memory.
__global__ __launch_bounds__(256) void sched32_kernel(const int32_t* __restrict__ offsets, int E, int bm,
                                                      MTile* __restrict__ sched, int32_t* __restrict__ sched_count) {
  extern __shared__ int32_t til32[];
  if (threadIdx.x == 0) {
    int32_t tl = 0;
    for (int e = 0; e < E; ++e) {
      til32[e] = tl;
      tl += (offsets[e + 1] - offsets[e] + bm - 1) / bm;
    }
    *sched_count = tl;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const int32_t o = offsets[e], c = offsets[e + 1] - offsets[e];
    for (int i = 0; i * bm < c; ++i) {
      MTile m;
      m.group = e;
      m.row0 = o + i * bm;
      m.rows = min(bm, c - i * bm);
      m.pad = 0;
      sched[til32[e] + i] = m;
    }
  }
}

int launch_sched32(const int32_t* offsets, int E, int bm, MTile* sched, int32_t* sched_count, hipStream_t st) {
  hipLaunchKernelGGL(sched32_kernel, dim3(1), dim3(256), sizeof(int32_t) * E, st, offsets, E, bm, sched, sched_count);
  return check_launch("sched32");
}

}  // namespace dsmoe
