// (d) Weighted combine + shared add, and the f1 bias update.
//
// combine:  y[t] = sum_{j by ascending expert id} w[t,j] * o_slots[t*k+j] + shared[t]
// restates the out-of-place index_add loop of models/moe.py:118-133 (the
// reference adds expert outputs in ascending expert id) and the shared add of
// models/moe.py:100-102.  Accumulation is fp32 with one final rounding; the k
// rows of a token are contiguous (slot order), so every access is a coalesced
// 16-byte vector.  A token's slot order is computed once, by k threads.
#include "common.h"

namespace dsmoe {

constexpr int CMB_MAX_K = 16;

template <typename T, int VEC>
struct Vec;
template <>
struct Vec<uint16_t, 8> {
  using type = uint4;
  static __device__ __forceinline__ void to_f(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf2f((uint16_t)(w[i] & 0xffffu));
      f[2 * i + 1] = bf2f((uint16_t)(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ uint4 from_f(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f2bf(f[2 * i]) | ((uint32_t)f2bf(f[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <>
struct Vec<float, 4> {
  using type = float4;
  static __device__ __forceinline__ void to_f(const float4& v, float* f) {
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
  static __device__ __forceinline__ float4 from_f(const float* f) { return make_float4(f[0], f[1], f[2], f[3]); }
};

// Sort a token's k (expert, slot j) pairs by expert id (insertion sort, k <= 16).
__device__ __forceinline__ void order_by_expert(const int32_t* idx_row, int k, int* ord) {
  int ev[CMB_MAX_K];
  for (int j = 0; j < k; ++j) {
    const int e = idx_row[j];
    int p = j;
    while (p > 0 && ev[p - 1] > e) {
      ev[p] = ev[p - 1];
      ord[p] = ord[p - 1];
      --p;
    }
    ev[p] = e;
    ord[p] = j;
  }
}

// One block per token.  Threads j < k put slot j at its ascending-expert
// position q (stable for equal ids) with its weight and the row of o that
// holds it, in LDS; then each thread takes VEC-wide column chunks c,
// c + blockDim, ... and issues the loads of the token's k rows before the fp32
// accumulation in q order.  Slot s's output is row row_of[s] of o (the layer
// keeps them in expert-sorted order, row_of = slot_pos) or row s (row_of null).
// KE > 0: k == KE at compile time (k <= 8), so every load and sum is
// unconditional and the loads stay in flight together (a load the compiler
// can sink into a k-guarded use is waited for there, one at a time).
template <typename T, int VEC, int KB, int KE>
__global__ __launch_bounds__(256) void combine_kernel(const T* __restrict__ o_slots, const int32_t* __restrict__ row_of,
                                                      const float* __restrict__ w, const int32_t* __restrict__ idx,
                                                      const T* __restrict__ shared, int T_, int D, int k_,
                                                      T* __restrict__ y) {
  const int k = KE > 0 ? KE : k_;
  using V = Vec<T, VEC>;
  using VT = typename V::type;
  __shared__ int row_s[KB];
  __shared__ float w_s[KB];
  const int64_t t = blockIdx.x;
  if ((int)threadIdx.x < k) {
    const int j = threadIdx.x;
    const int e = idx[t * k + j];
    int q = 0;
    for (int jj = 0; jj < k; ++jj) {
      const int ee = idx[t * k + jj];
      q += (ee < e) || (ee == e && jj < j);
    }
    row_s[q] = row_of ? row_of[t * k + j] : (int)(t * k + j);
    w_s[q] = w[t * k + j];
  }
  __syncthreads();
  const int cpr = D / VEC;
  for (int c = threadIdx.x; c < cpr; c += blockDim.x) {
    // every load unconditional (slots past k re-read slot k - 1, a missing
    // shared row reads slot 0; neither is added): a guarded load would make
    // the compiler wait for each in turn
    VT ov[KB];
#pragma unroll
    for (int q = 0; q < KB; ++q) ov[q] = reinterpret_cast<const VT*>(o_slots + (int64_t)row_s[min(q, k - 1)] * D)[c];
    const VT sv = reinterpret_cast<const VT*>(shared ? shared + t * (int64_t)D : o_slots + (int64_t)row_s[0] * D)[c];
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      if (q >= k) break;
      const float wj = w_s[q];
      float f[VEC];
      V::to_f(ov[q], f);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = fmaf(wj, f[v], acc[v]);
    }
    if (shared) {
      float f[VEC];
      V::to_f(sv, f);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] += f[v];
    }
    reinterpret_cast<VT*>(y + t * (int64_t)D)[c] = V::from_f(acc);
  }
}

template <typename T, int VEC>
static void launch_combine_vec(const void* o_slots, const int32_t* row_of, const float* w, const int32_t* idx,
                               const void* shared, const dsmoe_dims& d, void* y, hipStream_t st) {
  const int cpr = d.D / VEC;
  const int threads = cpr >= 256 ? 256 : (int)(cdiv(cpr, 64) * 64);
  auto o = static_cast<const T*>(o_slots);
  auto sh = static_cast<const T*>(shared);
  auto yy = static_cast<T*>(y);
  switch (d.k) {
#define CMB_K(n)                                                                                                    \
  case n:                                                                                                           \
    hipLaunchKernelGGL((combine_kernel<T, VEC, n, n>), dim3((unsigned)d.T), dim3(threads), 0, st, o, row_of, w, idx, \
                       sh, d.T, d.D, d.k, yy);                                                                      \
    break;
    CMB_K(1) CMB_K(2) CMB_K(3) CMB_K(4) CMB_K(5) CMB_K(6) CMB_K(7) CMB_K(8)
#undef CMB_K
    default:
      hipLaunchKernelGGL((combine_kernel<T, VEC, CMB_MAX_K, 0>), dim3((unsigned)d.T), dim3(threads), 0, st, o, row_of,
                         w, idx, sh, d.T, d.D, d.k, yy);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void combine_scalar_kernel(const T* __restrict__ o_slots,
                                                             const int32_t* __restrict__ row_of,
                                                             const float* __restrict__ w,
                                                             const int32_t* __restrict__ idx,
                                                             const T* __restrict__ shared, int T_, int D, int k,
                                                             T* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)T_ * D) return;
  const int64_t t = i / D;
  const int c = (int)(i - t * D);
  int ord[CMB_MAX_K];
  order_by_expert(idx + t * k, k, ord);
  float acc = 0.0f;
  for (int q = 0; q < k; ++q) {
    const int j = ord[q];
    const int64_t r = row_of ? (int64_t)row_of[t * k + j] : t * k + j;
    acc = fmaf(w[t * k + j], to_f<T>(o_slots[r * D + c]), acc);
  }
  if (shared) acc += to_f<T>(shared[t * (int64_t)D + c]);
  y[t * (int64_t)D + c] = from_f<T>(acc);
}

int launch_combine(const void* o_slots, const int32_t* row_of, const float* w, const int32_t* idx, const void* shared,
                   const dsmoe_dims& d, void* y, hipStream_t st) {
  if (d.T == 0) return DSMOE_OK;
  const bool al = ((reinterpret_cast<uintptr_t>(o_slots) | reinterpret_cast<uintptr_t>(y) |
                    reinterpret_cast<uintptr_t>(shared)) & 15) == 0;
  if (d.dtype == DSMOE_BF16) {
    if (d.D % 8 == 0 && al) {
      launch_combine_vec<uint16_t, 8>(o_slots, row_of, w, idx, shared, d, y, st);
    } else {
      const int64_t n = (int64_t)d.T * d.D;
      hipLaunchKernelGGL(combine_scalar_kernel<uint16_t>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st,
                         static_cast<const uint16_t*>(o_slots), row_of, w, idx, static_cast<const uint16_t*>(shared),
                         d.T, d.D, d.k, static_cast<uint16_t*>(y));
    }
  } else {
    if (d.D % 4 == 0 && al) {
      launch_combine_vec<float, 4>(o_slots, row_of, w, idx, shared, d, y, st);
    } else {
      const int64_t n = (int64_t)d.T * d.D;
      hipLaunchKernelGGL(combine_scalar_kernel<float>, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st,
                         static_cast<const float*>(o_slots), row_of, w, idx, static_cast<const float*>(shared), d.T,
                         d.D, d.k, static_cast<float*>(y));
    }
  }
  return check_launch("combine");
}

// f1: models/moe.py:21-27 on device.  One block; counts (E) int32 (the gate
// histogram) or fp32 (any caller-provided counts, fractional ones included).
// The reference's mean is counts.float().mean().  Integer counts (int32, or
// fp32 holding integers below 2^24) make every fp32 partial sum exact, so any
// summation order gives the same sum, and the fp32 division is the reference's.
// For fractional counts torch's fp32 reduction order is its own; here the sum
// is taken in fp64 and the mean rounded to fp32 once (the correctly rounded
// mean), which can differ from torch's by an ulp and so flip a decision only
// for a count within an ulp of a band edge.
template <typename C>
__global__ void update_bias_kernel(const C* __restrict__ counts, float* __restrict__ bias, int E, float speed,
                                   float upper, float lower) {
  __shared__ float s_avg;
  if (threadIdx.x == 0) {
    double s = 0.0;
    bool integral = true;
    for (int e = 0; e < E; ++e) {
      const float c = (float)counts[e];
      s += (double)c;
      integral = integral && c == truncf(c) && fabsf(c) < 16777216.0f;
    }
    // integral: the fp64 sum is the exact fp32 sum (below 2^24 per term, and
    // E terms stay exact in fp64), and fp32 division of it is the reference's
    s_avg = integral && fabs(s) < 16777216.0 ? (float)s / (float)E : (float)(s / (double)E);
  }
  __syncthreads();
  const float avg = s_avg;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const float c = (float)counts[e];
    float b = bias[e];
    if (c > avg * (1.0f + upper)) b -= speed;
    if (c < avg * (1.0f - lower)) b += speed;
    bias[e] = b;
  }
}

int launch_update_bias(const int32_t* counts, float* bias, int E, float speed, float upper, float lower,
                       hipStream_t st) {
  hipLaunchKernelGGL(update_bias_kernel<int32_t>, dim3(1), dim3(256), 0, st, counts, bias, E, speed, upper, lower);
  return check_launch("update_bias");
}

int launch_update_bias_f32(const float* counts, float* bias, int E, float speed, float upper, float lower,
                           hipStream_t st) {
  hipLaunchKernelGGL(update_bias_kernel<float>, dim3(1), dim3(256), 0, st, counts, bias, E, speed, upper, lower);
  return check_launch("update_bias_f32");
}

}  // namespace dsmoe
