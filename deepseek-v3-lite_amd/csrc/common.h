// Internal helpers shared by the dsmoe HIP sources (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "dsmoe.h"

namespace dsmoe {

using bf16_t = uint16_t;  // bf16 storage; arithmetic is done in fp32

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// fp32 -> bf16, round to nearest even (NaN kept quiet).
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<bf16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16_t>(u >> 16);
}

template <typename T>
__device__ __forceinline__ float to_f(T v);
template <>
__device__ __forceinline__ float to_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f<bf16_t>(bf16_t v) { return bf2f(v); }

template <typename T>
__device__ __forceinline__ T from_f(float v);
template <>
__device__ __forceinline__ float from_f<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16_t from_f<bf16_t>(float v) { return f2bf(v); }

// silu(g) = g * sigmoid(g), fp32.
__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }
__device__ __forceinline__ float sigmoid_f(float g) { return 1.0f / (1.0f + __expf(-g)); }

// Routing sigmoid: double evaluation, single rounding to fp32 (matches the oracle).
__device__ __forceinline__ float route_sigmoid(float x) {
  return static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(x))));
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ __forceinline__ size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

#define DSMOE_REQUIRE(cond, code, msg)                         \
  do {                                                         \
    if (!(cond)) return ::dsmoe::fail((code), std::string(msg)); \
  } while (0)

// ---------------------------------------------------------------- workspace carving
struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
  size_t used() const { return align_up(off, 256); }
};

// ---------------------------------------------------------------- grouped GEMM description
// One launch computes, for every group g and every row r of the group's row range:
//   C[cmap(r)][c_col(g) + n] = epilogue( sum_k A[amap(r)][k] * B_g(n, k) )
// where row ranges come from a device-side M-tile schedule (routed experts) or
// are dense (every group covers rows [0, dense_rows)).
enum Epi : int {
  EPI_STORE = 0,        // C = acc (rounded to C dtype)
  EPI_SWIGLU = 1,       // two B operands (W1, W3): C = silu(acc0) * acc1; optional G/U saves
};

struct MTile {  // one M tile of the routed schedule
  int32_t group;
  int32_t row0;   // first row (sorted position)
  int32_t rows;   // valid rows in this tile (<= BM)
  int32_t seq;    // mtile_seq(): this tile's index among its group's tiles and their count
};

// MTile::seq of tile i of a group of n M tiles: i << 16 | n, or 0 when the
// group has more than 65535 tiles (consumers then keep the schedule order).
__host__ __device__ inline int32_t mtile_seq(int32_t i, int32_t n) { return n < 65536 ? (i << 16) | n : 0; }

struct GemmDesc {
  // schedule
  const MTile* sched;         // routed schedule (device) or nullptr for dense
  const int32_t* sched_count; // number of valid entries in sched (device)
  int32_t dense_rows;         // dense: rows per group
  int32_t groups;             // number of groups (dense)
  int32_t m_tiles_bound;      // host upper bound of M tiles (grid sizing)
  int32_t bm;                 // rows per M tile (must equal the schedule's tile height)
  // A operand: rows of length K (K contiguous)
  const void* A;
  int64_t lda;
  int64_t a_rows;             // rows addressable through A (bounds the offset width)
  const int32_t* a_map;       // row -> A row, nullptr = identity
  // B operand(s): per group and K segment: B0[g * nseg + s] points at an (N x kseg) row-major block
  const void* const* B0;
  const void* const* B1;
  int64_t ldb;
  int32_t kseg;
  int32_t nseg;
  int32_t N, K;
  // outputs
  void* C;
  int64_t ldc;
  const int32_t* c_map;       // row -> C row, nullptr = identity
  int64_t c_group_col;        // column offset per group (dense shared GEMM1)
  void* Gs;                   // SWIGLU: optional pre-activation saves (same indexing as C)
  void* Us;
};

constexpr int TILE_M = 128;   // M tile of the SIMT fallback GEMM
constexpr int MAX_TOPK = 16;

struct GateOut {
  float* logits;
  int32_t* idx;
  int64_t* idx64;
  float* weights;
  void* weights_x;  // x dtype
  float* sel_scores;
  int32_t* counts;
};

struct PermuteScratch {
  int32_t* blockhist;
  int32_t* local_rank;
  MTile* sched;
  int32_t* sched_count;
};

// Tokens are ranked in blocks of RANK_TOKENS (one token per lane of a wave).
constexpr int RANK_TOKENS = 64;

// Outputs and scratch of the permute stage.  blockhist[b * E + e]: the count
// of expert e among the tokens of rank block b; local_rank[s]: slot s's rank
// among the earlier tokens of its rank block routed to the same expert (-1:
// the slot is not placed).
struct PermuteOut {
  int32_t* offsets;       // E + 1
  int32_t* sorted_slot;   // T * k
  int32_t* sorted_token;  // T * k
  int32_t* slot_pos;      // T * k
  int32_t* counts;        // E, optional
  const float* w;         // T * k, optional: gathered into sorted_w
  float* sorted_w;
  MTile* sched;           // M tiles of bm rows inside each expert
  int32_t* sched_count;
  int32_t bm;
  int32_t* blockhist;
  int32_t* local_rank;
};
PermuteOut permute_out(const PermuteScratch& s, int bm, int32_t* offsets, int32_t* sorted_slot, int32_t* sorted_token,
                       int32_t* slot_pos, int32_t* counts, const float* w, float* sorted_w);

// ---------------------------------------------------------------- launchers
// A chunk of a device pointer table passed by value as a kernel argument
// (within the 4 KB argument space): dst[off + i] = p[i] for i < n.
constexpr int PTR_CHUNK = 448;
struct PtrChunk {
  const void* p[PTR_CHUNK];
  int32_t n;
  int32_t off;
};

// part (optional): workspace of gate_part_floats(d) floats.  With it the
// MFMA gate writes K-split partial logits and a second launch adds them and
// routes; without it one launch computes and routes whole token tiles.
// tables (optional, MFMA gate only): a pointer table written by the gate
// launch itself (workgroup 0) into tab_dst, saving the upload launch.
// po (optional): the routing launch also ranks the routed slots for the
// permute (po's scratch), and for a call of one rank block finishes the
// permute; *ranked tells whether it did (the SIMT gate does not rank).
int launch_gate(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                const GateOut& out, hipStream_t st, float* part = nullptr, const PtrChunk* tables = nullptr,
                const void** tab_dst = nullptr, const PermuteOut* po = nullptr, bool* ranked = nullptr);
bool gate_uses_mfma(const void* x, const float* gw, const dsmoe_dims& d);
int gate_k_splits(const dsmoe_dims& d);
size_t gate_part_floats(const dsmoe_dims& d);
constexpr int GATE_KS_MAX = 8;       // K splits of the gate at most
void launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t st);
int64_t sched_bound(int64_t rows, int groups, int bm);
size_t permute_scratch_carve(Carver& c, const dsmoe_dims& d, int bm, PermuteScratch* out);
// The permute of idx into po.  ranked: the slots are already ranked (by the
// routing launch, launch_gate with po), else a rank launch runs first.
int launch_permute(const int32_t* idx, const dsmoe_dims& d, const PermuteOut& po, bool ranked, hipStream_t st);
// dst[p] = x[rows[p]] for p < nrows (rows of D elements); rows outside
// [0, src_rows) give zero rows.
// x_sorted[slot_pos[t k + j]] = x[t]: the gather of the sorted rows from the
// token side (falls back to the row gather through sorted_token when rows are
// not 16-byte vectors).
int launch_scatter_rows(const void* x, int64_t T, int k, const int32_t* slot_pos, const int32_t* sorted_token,
                        int D, int elem, void* dst, hipStream_t st);
int launch_gather_rows(const void* x, int64_t src_rows, const int32_t* rows, int64_t nrows, int D, int elem, void* dst,
                       hipStream_t st);
int launch_sched_from_offsets(const int64_t* offsets64, int E, int bm, int64_t rows, int32_t* offsets32, MTile* sched,
                              int32_t* sched_count, hipStream_t st);
// Whether launch_grouped_gemm will take the MFMA kernel for this descriptor,
// and the M-tile height of that choice; the routed schedule (and desc.bm) must
// be built with the same height.
bool gemm_mfma_eligible(const GemmDesc& g, int dtype, bool allow_mfma);
int gemm_tile_m(bool mfma);
bool gemm_qp_ok(const GemmDesc& g);
int launch_gemm_qp(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st);
int launch_gemm_qp_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, const float* row_scale, hipStream_t st);
int launch_grouped_gemm(const GemmDesc& g, int epi, int dtype, const float* row_scale, bool allow_mfma,
                        hipStream_t st);
// Few-row grouped GEMM (decode): row tiles of SK_BM rows, weights streamed
// once.  The routed schedule must be built with bm = SK_BM; no G/U saves.
constexpr int SK_BM = 64;
bool gemm_sk_ok(const GemmDesc& g);
int launch_gemm_sk(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st);
int launch_gemm_sk_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, const float* row_scale, hipStream_t st);
// gr (routed or dense) then the dense gd (same epilogue): one persistent launch
// when that kernel takes both, else two launches.  row_scale applies to gr.
int launch_grouped_gemm_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, int dtype, const float* row_scale,
                             bool allow_mfma_r, bool allow_mfma_d, hipStream_t st);
// row_of: slot s's output is row row_of[s] of o_slots (null: row s)
int launch_combine(const void* o_slots, const int32_t* row_of, const float* w, const int32_t* idx, const void* shared,
                   const dsmoe_dims& d, void* y, hipStream_t st);
int launch_update_bias(const int32_t* counts, float* bias, int E, float speed, float upper, float lower,
                       hipStream_t st);
int launch_update_bias_f32(const float* counts, float* bias, int E, float speed, float upper, float lower,
                           hipStream_t st);


// ---------------------------------------------------------------- backward GEMM description
// C(m, n) = sum_k A(m, k) * B(n, k) with the operand layouts the backward
// pass needs.  "rowspace" indices are sorted positions (routed) or token ids
// (dense / shared).
enum XAMode : int {
  XA_ROWS = 0,   // A(m, k) = A[amap(r) * lda + k], r = rowspace row of output row m
  XA_KMAJOR = 1, // A(m, k) = A[amap(p) * lda + a_col + m] * kscale(p), p = rowspace index k
};
enum XBMode : int {
  XB_W_NT = 0,     // B(n, k) = Btab[g*nseg + seg][n * ldb + kin]      (weights, K contiguous)
  XB_W_NN = 1,     // B(n, k) = Btab[g*nseg + seg][kin * ldb + n]      (weights, N contiguous)
  XB_ACT_KMAJOR = 2, // B(n, k) = Bact[bmap(p) * ldb + b_col + n], p = rowspace index k
};
enum XSched : int {
  XS_ROUTED = 0,  // M tiles from the routed schedule, full K
  XS_DENSE = 1,   // groups x dense_rows, full K
  XS_WGRAD = 2,   // groups x M x N output per group, K = rowspace range k_off[g] .. k_off[g+1] (or 0..K)
};
enum XEpi : int {
  XE_STORE = 0,       // C[cmap(r) * ldc + g * c_group_col + n] = acc
  XE_SWIGLU_BWD = 1,  // dh = row_w(r) * acc; with g, u saved: dg -> C[..+n], du -> C[..+du_off+n]
  XE_WGRAD = 2,       // per-group output pointers, rows split at msplit into Ctab0 / Ctab1
};

struct XGemm {
  int32_t sched_mode;
  const MTile* sched;
  const int32_t* sched_count;
  int32_t m_tiles_bound;
  int32_t bm;                  // schedule tile height (routed)
  int32_t dense_rows;
  int32_t groups;
  const int32_t* k_off;        // XS_WGRAD: per-group K range (groups + 1 entries), null -> [0, K)
  int32_t M, N, K;             // M: output rows per group (XS_WGRAD)
  // A
  int32_t a_mode;
  const void* A;
  int64_t lda;
  int64_t a_col;               // XA_KMAJOR: column offset per group (times group index)
  const int32_t* a_map;
  const float* a_kscale;
  // B
  int32_t b_mode;
  const void* const* Btab;
  int64_t ldb;
  int32_t kseg;
  int32_t nseg;
  const void* Bact;
  const int32_t* b_map;
  int64_t b_col;               // XB_ACT_KMAJOR: column offset per group (times group index)
  // C
  void* C;
  int64_t ldc;
  const int32_t* c_map;
  int64_t c_group_col;
  void* const* Ctab0;
  void* const* Ctab1;
  int32_t msplit;
  // SwiGLU backward
  const void* Gs;
  const void* Us;
  int64_t ld_gu;
  int64_t gu_group_col;
  const float* row_w;
  int64_t du_off;
  // XS_WGRAD split-K (MFMA path only): each group's K range is cut into
  // ksplit slab-aligned parts; part i writes fp32 partial sums to
  // part[((i * groups + grp) * M + m) * N + n] and a second kernel adds the
  // parts in ascending i and rounds once.  ksplit <= 1: direct store.
  int32_t ksplit;
  float* part;
  // XE_WGRAD: the output rows (Ctab0 / Ctab1) are fp32 (fp32 master weights
  // of a bf16 computation), written unrounded; else the compute dtype.
  int32_t c_f32;
};

// Backward grouped GEMM: MFMA kernel when dtype is bf16, allow_mfma is set
// (the caller checked the alignment of every pointer-table entry) and the
// shapes fit (xgemm_mfma_ok); fp32-FMA tiles otherwise.
int launch_xgemm(const XGemm& g, int epi, int dtype, bool allow_mfma, hipStream_t st);
bool xgemm_mfma_ok(const XGemm& g, int epi);
int launch_xgemm_mfma(const XGemm& g, int epi, hipStream_t st);
bool xgemm_q_ok(const XGemm& g, int epi);
int launch_wgrad_reduce(const XGemm& g, hipStream_t st);
int launch_xgemm_q(const XGemm& g, int epi, hipStream_t st);
// dst[p] = bf16(w[p] * src[rows[p]]) for p < n, rows of D bf16 (w * dY in sorted order)
int launch_scale_gather_rows(const void* src, const int32_t* rows, const float* w, int64_t n, int D, void* dst,
                             hipStream_t st);
int xgemm_pick_ksplit(int64_t tiles, int64_t k_len);
int64_t xgemm_tiles(int64_t M, int64_t N, int groups);
int launch_dw_dot(const void* dy, const void* o_slots, const int32_t* row_of, int64_t N, int k, int D, int dtype,
                  float* dw, hipStream_t st);
// launch_dw_dot and launch_scale_gather_rows (rows by token, slot weights) in
// one pass; DSMOE_ERR_UNSUPPORTED (nothing launched) when the shape or
// alignment does not fit (bf16, D % 8, k <= 8, 16-byte rows).
int launch_prep_tok(const void* dy, const void* o_slots, const int32_t* row_of, const float* w, const int32_t* slot_pos,
                    int T, int k, int D, int dtype, float* dw, void* dy_w, hipStream_t st);
int launch_gate_bwd(const float* dw, const float* sel, int T, int k, float rs, float* dlog, hipStream_t st);
int launch_dwgate(const void* x, const float* dlog, const int32_t* sorted_slot, const int32_t* sorted_token,
                  const int32_t* offsets, int E, int D, int dtype, float* dgw, hipStream_t st);
int launch_dx_final(const void* dx_slots, const void* dx_shared, const float* dlog, const int32_t* idx, const float* gw,
                    int T, int D, int k, int dtype, void* dx, hipStream_t st);
int launch_sched32(const int32_t* offsets, int E, int bm, MTile* sched, int32_t* sched_count, hipStream_t st);

}  // namespace dsmoe
