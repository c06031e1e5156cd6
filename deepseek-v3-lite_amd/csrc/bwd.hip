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
#include <algorithm>

#include "common.h"

namespace dsmoe {

// Slot s's expert output is row row_of[s] of o (the layer keeps them in
// expert-sorted order, row_of = slot_pos) or row s (row_of null).
template <typename T>
__global__ __launch_bounds__(256) void dw_dot_kernel(const T* __restrict__ dy, const T* __restrict__ o_slots,
                                                     const int32_t* __restrict__ row_of, int64_t N, int k, int D,
                                                     float* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= N) return;
  const int64_t t = s / k;
  const T* a = dy + t * D;
  const T* b = o_slots + (row_of ? (int64_t)row_of[s] : s) * D;
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

// Vectorised forms (VEC consecutive columns per thread, 16-byte loads).
template <typename T>
struct Vec16;
template <>
struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ static void load(const bf16_t* p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ static void store(bf16_t* p, const float (&v)[8]) {
    uint4 u;
    u.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    u.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
    u.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
    u.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
    *reinterpret_cast<uint4*>(p) = u;
  }
};
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  __device__ static void load(const float* p, float (&v)[4]) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  }
  __device__ static void store(float* p, const float (&v)[4]) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

// dx[t] per token (one block): same order and rounding as dx_final_kernel.
// Threads j < k put slot j at its ascending-expert position q in LDS (with
// its expert and dlogit); the k slot rows of a column chunk are loaded
// together before the fp32 sums.
// KE > 0: k == KE at compile time (k <= 8): every load and sum is
// unconditional, so the loads stay in flight together.
template <typename T, int KB, int KE>
__global__ __launch_bounds__(256) void dx_final_vec_kernel(const T* __restrict__ dx_slots, const T* __restrict__ dx_shared,
                                                           const float* __restrict__ dlog, const int32_t* __restrict__ idx,
                                                           const float* __restrict__ gw, int D, int k_,
                                                           T* __restrict__ dx) {
  const int k = KE > 0 ? KE : k_;
  constexpr int V = Vec16<T>::N;
  __shared__ int ord_s[KB], ev_s[KB];
  __shared__ float dl_s[KB];
  const int64_t t = blockIdx.x;
  if ((int)threadIdx.x < k) {
    const int j = threadIdx.x;
    const int e = idx[t * k + j];
    int q = 0;
    for (int jj = 0; jj < k; ++jj) {
      const int ee = idx[t * k + jj];
      q += (ee < e) || (ee == e && jj < j);
    }
    ord_s[q] = j;
    ev_s[q] = e;
    dl_s[q] = dlog[t * k + j];
  }
  __syncthreads();
  for (int c = threadIdx.x; c * V < D; c += blockDim.x) {
    const int d = c * V;
    float acc[V], v[KB][V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int q = 0; q < KB; ++q)
      if (KE > 0 || q < k) Vec16<T>::load(dx_slots + (t * k + ord_s[q]) * (int64_t)D + d, v[q]);
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      if (q >= k) break;
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += v[q][i];
    }
    if (dx_shared) {
      float sv[V];
      Vec16<T>::load(dx_shared + t * (int64_t)D + d, sv);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += sv[i];
    }
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      if (q >= k) break;
      const float dl = dl_s[q];
      const float* grow = gw + (int64_t)ev_s[q] * D + d;
#pragma unroll
      for (int i = 0; i < V; i += 4) {
        const float4 w4 = *reinterpret_cast<const float4*>(grow + i);
        acc[i] = fmaf(dl, w4.x, acc[i]);
        acc[i + 1] = fmaf(dl, w4.y, acc[i + 1]);
        acc[i + 2] = fmaf(dl, w4.z, acc[i + 2]);
        acc[i + 3] = fmaf(dl, w4.w, acc[i + 3]);
      }
    }
    Vec16<T>::store(dx + t * (int64_t)D + d, acc);
  }
}

// dW_gate[e, cols] for one expert and 64 * VEC columns.
// NW waves per (expert, 64 V columns); wave w takes the expert's rows
// p0 + w, p0 + w + NW, ... in ascending order, U at a time: the x rows and
// dlogits of a batch are loaded together while the sorted indices of the next
// batch are already in flight (a batch waits for one round trip, not two), and
// every load of a full batch is unconditional (clamped columns; a guarded load
// is waited for at its branch).  The last, partial batch goes one row at a
// time.  The waves' sums are added in wave order: a fixed order, so the result
// does not depend on scheduling.
template <typename T, int NW>
__global__ __launch_bounds__(NW * 64) void dwgate_vec_kernel(const T* __restrict__ x, const float* __restrict__ dlog,
                                                             const int32_t* __restrict__ sorted_slot,
                                                             const int32_t* __restrict__ sorted_token,
                                                             const int32_t* __restrict__ offsets, int D,
                                                             float* __restrict__ dgw) {
  constexpr int V = Vec16<T>::N;
  constexpr int U = 8;
  __shared__ float red[NW - 1][64 * V];
  const int e = blockIdx.y;
  const int grp = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int dl = (blockIdx.x * 64 + l) * V;
  const bool live = dl < D;
  const int d = min(dl, D - V);
  const int p0 = offsets[e], p1 = offsets[e + 1];
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  int p = p0 + grp;
  if (p + NW * (U - 1) < p1) {
    int slot[U], tok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      slot[u] = sorted_slot[p + NW * u];
      tok[u] = sorted_token[p + NW * u];
    }
    for (;;) {
      float wv[U], xv[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        wv[u] = dlog[slot[u]];
        Vec16<T>::load(x + (int64_t)tok[u] * D + d, xv[u]);
      }
      const int pn = p + NW * U;
      const bool more = pn + NW * (U - 1) < p1;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = min(pn + NW * u, p1 - 1);  // in the expert's range
        slot[u] = sorted_slot[q];
        tok[u] = sorted_token[q];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = fmaf(wv[u], xv[u][i], acc[i]);
      p = pn;
      if (!more) break;
    }
  }
  for (; p < p1; p += NW) {
    float xv[V];
    const float wv = dlog[sorted_slot[p]];
    Vec16<T>::load(x + (int64_t)sorted_token[p] * D + d, xv);
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = fmaf(wv, xv[i], acc[i]);
  }
  if (grp > 0) {
#pragma unroll
    for (int i = 0; i < V; ++i) red[grp - 1][l * V + i] = acc[i];
  }
  __syncthreads();
  if (grp == 0 && live) {
#pragma unroll
    for (int gi = 0; gi < NW - 1; ++gi)
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] += red[gi][l * V + i];
    float* o = dgw + (int64_t)e * D + d;
#pragma unroll
    for (int i = 0; i < V; i += 4) *reinterpret_cast<float4*>(o + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
  }
}

// bf16, one wave per token: dy[t] is read once, 16 bytes per lane, and the
// k dot products with the token's slot rows accumulate together.
template <int KB>
__global__ __launch_bounds__(256) void dw_dot_tok_kernel(const bf16_t* __restrict__ dy, const bf16_t* __restrict__ o_slots,
                                                         const int32_t* __restrict__ row_of, int T, int k, int D,
                                                         float* __restrict__ dw) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int vpr = D / 8;
  int64_t orow[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) orow[j] = j < k ? (row_of ? (int64_t)row_of[t * k + j] : t * k + j) : 0;
  const uint4* a = reinterpret_cast<const uint4*>(dy + t * D);
  float acc[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) acc[j] = 0.0f;
  for (int c = lane; c < vpr; c += 64) {
    float af[8];
    Vec16<bf16_t>::load(reinterpret_cast<const bf16_t*>(a + c), af);
    float bv[KB][8];
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (j < k) Vec16<bf16_t>::load(o_slots + orow[j] * D + c * 8, bv[j]);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (j >= k) break;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j] = fmaf(af[i], bv[j][i], acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    if (j >= k) break;
    float v = acc[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) dw[t * k + j] = v;
  }
}

// dw and the weighted dY rows in one pass, one wave per token: dY_t is read
// once; for each slot j of the token, dw[t k + j] = <dY_t, o_slot> (the
// dw_dot_tok_kernel sums, in the same order) and dy_w[slot_pos[t k + j]] =
// bf16(w[t k + j] * dY_t) (scale_gather_kernel's rounding).
// KE > 0: k == KE at compile time (k <= 8): every load is unconditional, so
// the loads stay in flight together.
template <int KB, int KE>
__global__ __launch_bounds__(256) void prep_tok_kernel(const bf16_t* __restrict__ dy, const bf16_t* __restrict__ o_slots,
                                                       const int32_t* __restrict__ row_of, const float* __restrict__ w,
                                                       const int32_t* __restrict__ slot_pos, int T, int k_, int D,
                                                       float* __restrict__ dw, bf16_t* __restrict__ dy_w) {
  const int k = KE > 0 ? KE : k_;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int vpr = D / 8;
  float ws[KB];
  int64_t pos[KB], orow[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    ws[j] = 0.0f;
    pos[j] = 0;
    orow[j] = 0;
    if (KE > 0 || j < k) {
      ws[j] = w[t * k + j];
      pos[j] = slot_pos[t * k + j];
      orow[j] = row_of ? (int64_t)row_of[t * k + j] : t * k + j;
    }
  }
  float acc[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) acc[j] = 0.0f;
  for (int c = lane; c < vpr; c += 64) {
    float af[8];
    Vec16<bf16_t>::load(dy + t * D + c * 8, af);
    float bv[KB][8];
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (KE > 0 || j < k) Vec16<bf16_t>::load(o_slots + orow[j] * D + c * 8, bv[j]);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (j >= k) break;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j] = fmaf(af[i], bv[j][i], acc[j]);
      float sv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = af[i] * ws[j];
      Vec16<bf16_t>::store(dy_w + pos[j] * D + c * 8, sv);
    }
  }
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    if (j >= k) break;
    float v = acc[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) dw[t * k + j] = v;
  }
}

static bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int launch_prep_tok(const void* dy, const void* o_slots, const int32_t* row_of, const float* w, const int32_t* slot_pos,
                    int T, int k, int D, int dtype, float* dw, void* dy_w, hipStream_t st) {
  if (!(dtype == DSMOE_BF16 && D % 8 == 0 && k <= 8 && dy_w && al16p(dy) && al16p(o_slots) && al16p(dy_w)))
    return DSMOE_ERR_UNSUPPORTED;
  if (T == 0) return DSMOE_OK;
  switch (k) {
#define PREP_K(n)                                                                                                   \
  case n:                                                                                                           \
    hipLaunchKernelGGL((prep_tok_kernel<n, n>), dim3((unsigned)cdiv(T, 4)), dim3(256), 0, st,                       \
                       static_cast<const bf16_t*>(dy), static_cast<const bf16_t*>(o_slots), row_of, w, slot_pos, T, \
                       k, D, dw, static_cast<bf16_t*>(dy_w));                                                       \
    break;
    PREP_K(1) PREP_K(2) PREP_K(3) PREP_K(4) PREP_K(5) PREP_K(6) PREP_K(7) PREP_K(8)
#undef PREP_K
    default:
      hipLaunchKernelGGL((prep_tok_kernel<8, 0>), dim3((unsigned)cdiv(T, 4)), dim3(256), 0, st,
                         static_cast<const bf16_t*>(dy), static_cast<const bf16_t*>(o_slots), row_of, w, slot_pos, T, k,
                         D, dw, static_cast<bf16_t*>(dy_w));
  }
  return check_launch("prep_tok");
}

// ---------------------------------------------------------------- launchers
// dst[p] = bf16(w[p] * src[rows[p]]), 8 columns per thread: one fp32 product
// per element rounded once, as the backward of the routed combine's
// out * weight (models/moe.py:132) rounds it.
__global__ __launch_bounds__(256) void scale_gather_kernel(const bf16_t* __restrict__ src, const int32_t* __restrict__ rows,
                                                           const float* __restrict__ w, int64_t n, int vpr,
                                                           bf16_t* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * vpr) return;
  const int64_t p = i / vpr;
  const int c = (int)(i - p * vpr);
  const float s = w[p];
  const uint4 v = reinterpret_cast<const uint4*>(src + (int64_t)rows[p] * vpr * 8)[c];
  uint4 o;
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t out[4];
#pragma unroll
  for (int d = 0; d < 4; ++d)
    out[d] = (uint32_t)f2bf(__uint_as_float(in[d] << 16) * s) |
             ((uint32_t)f2bf(__uint_as_float(in[d] & 0xffff0000u) * s) << 16);
  o.x = out[0]; o.y = out[1]; o.z = out[2]; o.w = out[3];
  reinterpret_cast<uint4*>(dst + p * vpr * 8)[c] = o;
}

int launch_scale_gather_rows(const void* src, const int32_t* rows, const float* w, int64_t n, int D, void* dst,
                             hipStream_t st) {
  if (n == 0) return DSMOE_OK;
  if (D % 8) return fail(DSMOE_ERR_UNSUPPORTED, "scale_gather: D must be a multiple of 8");
  const int vpr = D / 8;
  hipLaunchKernelGGL(scale_gather_kernel, dim3((unsigned)cdiv(n * vpr, 256)), dim3(256), 0, st,
                     static_cast<const bf16_t*>(src), rows, w, n, vpr, static_cast<bf16_t*>(dst));
  return check_launch("scale_gather");
}

int launch_dw_dot(const void* dy, const void* o_slots, const int32_t* row_of, int64_t N, int k, int D, int dtype,
                  float* dw, hipStream_t st) {
  if (N == 0) return DSMOE_OK;
  const unsigned grid = (unsigned)cdiv(N, 4);
  if (dtype == DSMOE_BF16 && D % 8 == 0 && al16p(dy) && al16p(o_slots) && k <= 8) {
    const int T = (int)(N / k);
    hipLaunchKernelGGL(dw_dot_tok_kernel<8>, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, st,
                       static_cast<const bf16_t*>(dy), static_cast<const bf16_t*>(o_slots), row_of, T, k, D, dw);
    return check_launch("dw_dot");
  }
  if (dtype == DSMOE_BF16)
    hipLaunchKernelGGL(dw_dot_kernel<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(dy),
                       static_cast<const bf16_t*>(o_slots), row_of, N, k, D, dw);
  else
    hipLaunchKernelGGL(dw_dot_kernel<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(dy),
                       static_cast<const float*>(o_slots), row_of, N, k, D, dw);
  return check_launch("dw_dot");
}

int launch_gate_bwd(const float* dw, const float* sel, int T, int k, float rs, float* dlog, hipStream_t st) {
  if (T == 0) return DSMOE_OK;
  hipLaunchKernelGGL(gate_bwd_kernel, dim3((unsigned)cdiv(T, 256)), dim3(256), 0, st, dw, sel, T, k, rs, dlog);
  return check_launch("gate_bwd");
}

constexpr int DWG_WAVES = 16;

int launch_dwgate(const void* x, const float* dlog, const int32_t* sorted_slot, const int32_t* sorted_token,
                  const int32_t* offsets, int E, int D, int dtype, float* dgw, hipStream_t st) {
  const int V = dtype == DSMOE_BF16 ? 8 : 4;
  if (D % V == 0 && al16p(x) && al16p(dgw)) {
    const dim3 gv((unsigned)cdiv(D, 64 * V), (unsigned)E);
    if (dtype == DSMOE_BF16)
      hipLaunchKernelGGL((dwgate_vec_kernel<bf16_t, DWG_WAVES>), gv, dim3(DWG_WAVES * 64), 0, st,
                         static_cast<const bf16_t*>(x), dlog,
                         sorted_slot, sorted_token, offsets, D, dgw);
    else
      hipLaunchKernelGGL((dwgate_vec_kernel<float, DWG_WAVES>), gv, dim3(DWG_WAVES * 64), 0, st,
                         static_cast<const float*>(x), dlog,
                         sorted_slot, sorted_token, offsets, D, dgw);
    return check_launch("dwgate_vec");
  }
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
  const int V = dtype == DSMOE_BF16 ? 8 : 4;
  if (D % V == 0 && al16p(dx_slots) && al16p(dx) && al16p(gw) && (!dx_shared || al16p(dx_shared))) {
    const unsigned threads = (unsigned)std::min<int64_t>(256, cdiv(cdiv(D, V), 64) * 64);
    auto go = [&](auto tag) {
      using TT = decltype(tag);
      const TT* s = static_cast<const TT*>(dx_slots);
      const TT* sh = static_cast<const TT*>(dx_shared);
      TT* o = static_cast<TT*>(dx);
      switch (k) {
#define DXF_K(n)                                                                                                   \
  case n:                                                                                                          \
    hipLaunchKernelGGL((dx_final_vec_kernel<TT, n, n>), dim3((unsigned)T), dim3(threads), 0, st, s, sh, dlog, idx, \
                       gw, D, k, o);                                                                               \
    break;
        DXF_K(1) DXF_K(2) DXF_K(3) DXF_K(4) DXF_K(5) DXF_K(6) DXF_K(7) DXF_K(8)
#undef DXF_K
        default:
          hipLaunchKernelGGL((dx_final_vec_kernel<TT, MAX_TOPK, 0>), dim3((unsigned)T), dim3(threads), 0, st, s, sh,
                             dlog, idx, gw, D, k, o);
      }
    };
    if (dtype == DSMOE_BF16)
      go(bf16_t{});
    else
      go(float{});
    return check_launch("dx_final_vec");
  }
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
      m.seq = mtile_seq(i, (c + bm - 1) / bm);
      sched[til32[e] + i] = m;
    }
  }
}

int launch_sched32(const int32_t* offsets, int E, int bm, MTile* sched, int32_t* sched_count, hipStream_t st) {
  hipLaunchKernelGGL(sched32_kernel, dim3(1), dim3(256), sizeof(int32_t) * E, st, offsets, E, bm, sched, sched_count);
  return check_launch("sched32");
}

}  // namespace dsmoe
