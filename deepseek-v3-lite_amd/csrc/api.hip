// extern "C" entry points of libdsmoe.so (declared in include/dsmoe.h).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <utility>
#include <string>
#include <vector>

#include "common.h"

namespace dsmoe {

// ---------------------------------------------------------------- errors
static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DSMOE_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return DSMOE_OK;
}

// ---------------------------------------------------------------- pointer tables

__global__ void set_ptrs_kernel(PtrChunk c, const void** dst) {
  for (int i = threadIdx.x; i < c.n; i += blockDim.x) dst[c.off + i] = c.p[i];
}

// Copies the concatenation of `lists` (host arrays of device pointers) into
// the device table dst[0..], in as few launches as the argument space allows.
static int upload_ptr_lists(std::initializer_list<std::pair<const void* const*, int>> lists, const void** dst,
                            hipStream_t st) {
  PtrChunk c;
  c.n = 0;
  c.off = 0;
  int pos = 0;
  for (const auto& l : lists) {
    for (int i = 0; i < l.second; ++i) {
      c.p[c.n++] = l.first[i];
      ++pos;
      if (c.n == PTR_CHUNK) {
        hipLaunchKernelGGL(set_ptrs_kernel, dim3(1), dim3(256), 0, st, c, dst);
        c.off = pos;
        c.n = 0;
      }
    }
  }
  if (c.n) hipLaunchKernelGGL(set_ptrs_kernel, dim3(1), dim3(256), 0, st, c, dst);
  return check_launch("upload_ptrs");
}

static bool all_aligned16(const void* const* p, int n) {
  for (int i = 0; i < n; ++i)
    if (!p[i] || (reinterpret_cast<uintptr_t>(p[i]) & 15)) return false;
  return true;
}

static int elem_size(int dtype) { return dtype == DSMOE_BF16 ? 2 : 4; }

static int validate(const dsmoe_dims* d, bool need_experts) {
  if (!d) return fail(DSMOE_ERR_INVALID, "dims is NULL");
  if (d->dtype != DSMOE_F32 && d->dtype != DSMOE_BF16)
    return fail(DSMOE_ERR_UNSUPPORTED, "dtype must be DSMOE_F32 or DSMOE_BF16");
  if (d->T < 0 || d->D <= 0 || d->E <= 0) return fail(DSMOE_ERR_INVALID, "need T >= 0, D > 0, E > 0");
  if (d->E > 256) return fail(DSMOE_ERR_UNSUPPORTED, "n_routed_experts > 256 is not supported");
  if (d->k <= 0 || d->k > d->E) return fail(DSMOE_ERR_INVALID, "need 1 <= n_activated_experts <= n_routed_experts");
  if (d->k > MAX_TOPK) return fail(DSMOE_ERR_UNSUPPORTED, "n_activated_experts > 16 is not supported");
  if ((int64_t)d->T * d->k >= (int64_t(1) << 31)) return fail(DSMOE_ERR_UNSUPPORTED, "T * k must be < 2^31");
  if (need_experts) {
    if (d->I <= 0) return fail(DSMOE_ERR_INVALID, "moe_inter_dim must be > 0");
    if (d->S < 0 || (d->S > 0 && d->I_s <= 0)) return fail(DSMOE_ERR_INVALID, "bad shared expert shape");
  }
  return DSMOE_OK;
}

// ---------------------------------------------------------------- layer workspace layout
struct FwdLayout {
  const void** ptrs;  // [w1 E][w3 E][w2 E][sw1 S][sw3 S][sw2 S]
  float* gate_part;   // partial logits of a K-split gate, or nullptr
  int32_t* idx;
  float* w;
  float* sel;
  int32_t* offsets;
  int32_t* sorted_slot;
  int32_t* sorted_token;
  int32_t* slot_pos;
  float* sorted_w;  // training: weights in sorted order
  PermuteScratch ps;
  void* h;
  void* g;
  void* u;
  void* hs;
  void* gs;
  void* us;
  void* o_sorted;   // routed expert outputs (N, D) in sorted order
  void* shared_out;
  void* x_sorted;   // training: routed rows of x in sorted order (the backward's K-major operand)
  size_t total;
};

static FwdLayout fwd_layout(const dsmoe_dims& d, int training, void* base) {
  Carver c(base);
  FwdLayout L;
  const int64_t N = (int64_t)d.T * d.k;
  const int es = elem_size(d.dtype);
  L.ptrs = c.take<const void*>(3 * d.E + 3 * d.S);
  L.idx = c.take<int32_t>(N);
  L.w = c.take<float>(N);
  L.sel = c.take<float>(N);
  L.offsets = c.take<int32_t>(d.E + 1);
  L.sorted_slot = c.take<int32_t>(N);
  L.sorted_token = c.take<int32_t>(N);
  L.slot_pos = c.take<int32_t>(N);
  L.sorted_w = training ? c.take<float>(N) : nullptr;
  L.gate_part = gate_part_floats(d) ? c.take<float>(gate_part_floats(d)) : nullptr;
  permute_scratch_carve(c, d, SK_BM, &L.ps);  // the smallest schedule tile height
  L.h = c.take<char>((size_t)N * d.I * es);
  L.g = training ? c.take<char>((size_t)N * d.I * es) : nullptr;
  L.u = training ? c.take<char>((size_t)N * d.I * es) : nullptr;
  const int64_t SIs = (int64_t)d.S * d.I_s;
  L.hs = d.S ? c.take<char>((size_t)d.T * SIs * es) : nullptr;
  L.gs = (d.S && training) ? c.take<char>((size_t)d.T * SIs * es) : nullptr;
  L.us = (d.S && training) ? c.take<char>((size_t)d.T * SIs * es) : nullptr;
  L.o_sorted = c.take<char>((size_t)N * d.D * es);
  L.shared_out = d.S ? c.take<char>((size_t)d.T * d.D * es) : nullptr;
  L.x_sorted = training ? c.take<char>((size_t)N * d.D * es) : nullptr;
  L.total = c.used();
  return L;
}

// ---------------------------------------------------------------- stage timing
enum Stage : int {
  ST_TABLES = 0, ST_GATE, ST_PERMUTE, ST_GEMM1, ST_GEMM2, ST_COMBINE,
  ST_BWD_PREP, ST_BWD_DH, ST_BWD_DH_SHARED, ST_BWD_DX, ST_BWD_DX_SHARED, ST_BWD_DW13, ST_BWD_DW2,
  ST_BWD_DW_SHARED, ST_BWD_GATE, ST_BWD_REDUCE, ST_COUNT
};
static const char* kStageNames[ST_COUNT] = {
  "tables", "gate", "permute", "gemm1", "gemm2", "combine",
  "bwd_prep", "bwd_dh_routed", "bwd_dh_shared", "bwd_dx_routed", "bwd_dx_shared", "bwd_dw13_routed",
  "bwd_dw2_routed", "bwd_dw_shared", "bwd_gate", "bwd_reduce"};

struct TimingState {
  std::mutex mu;
  bool on = false;
  struct Rec { hipEvent_t a, b; int stage; };
  std::vector<Rec> recs;
  std::vector<int> calls;
};
static TimingState g_timing;

// Records the boundary of `stage` on `st` when timing is enabled.
class StageTimer {
 public:
  explicit StageTimer(hipStream_t st) : st_(st) {
    std::lock_guard<std::mutex> lk(g_timing.mu);
    on_ = g_timing.on;
  }
  void begin(int stage) {
    if (!on_) return;
    stage_ = stage;
    (void)hipEventCreate(&a_);
    (void)hipEventRecord(a_, st_);
  }
  void end() {
    if (!on_ || stage_ < 0) return;
    hipEvent_t b;
    (void)hipEventCreate(&b);
    (void)hipEventRecord(b, st_);
    std::lock_guard<std::mutex> lk(g_timing.mu);
    g_timing.recs.push_back({a_, b, stage_});
    stage_ = -1;
  }
  bool on() const { return on_; }
  void call_done(int kind) {
    if (!on_) return;
    std::lock_guard<std::mutex> lk(g_timing.mu);
    g_timing.calls.push_back(kind);
  }

 private:
  hipStream_t st_;
  bool on_ = false;
  int stage_ = -1;
  hipEvent_t a_{};
};

// A second stream per calling thread and device, with its fork and join
// events, for backward work that does not depend on the routed chain.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
// The calling thread's second stream on the device of `st`, or null (the
// caller then keeps all its work on `st`): when `st` belongs to a device other
// than the current one, or when the stream or its events cannot be made.  A
// failed query or creation leaves no error behind for the next launch check.
static SideStream* side_stream(hipStream_t st) {
  constexpr int kDev = 16;
  thread_local SideStream ss[kDev];
  const auto none = []() -> SideStream* {
    (void)hipGetLastError();
    return nullptr;
  };
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDev) return none();
  if (st) {
    hipDevice_t sd = -1;
    if (hipStreamGetDevice(st, &sd) != hipSuccess || sd != dev) return none();
  }
  SideStream& x = ss[dev];
  if (!x.s) {
    hipStream_t s = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return none();
    if (hipEventCreateWithFlags(&a, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&b, hipEventDisableTiming) != hipSuccess) {
      if (a) (void)hipEventDestroy(a);
      (void)hipStreamDestroy(s);
      return none();
    }
    x.s = s;
    x.fork = a;
    x.join = b;
  }
  return &x;
}

static GemmDesc desc_zero() {
  GemmDesc g;
  std::memset(static_cast<void*>(&g), 0, sizeof(g));
  g.nseg = 1;
  return g;
}

// ---------------------------------------------------------------- static permute scratch
// The scratch of dsmoe_permute_noalloc: a file-scope device array, one copy
// per GPU (each at its own address), held until the process ends.  In host
// code `scratch` names a host-side stand-in, so kernels get the device
// address from hipGetSymbolAddress, fetched once per device with that device
// current and kept in g_scratch_ptr.
static __device__ __align__(256) char scratch[DSMOE_PERMUTE_NOALLOC_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

static int static_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(DSMOE_ERR_HIP, "permute_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(DSMOE_ERR_UNSUPPORTED, "permute_noalloc: device index >= 64");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(DSMOE_ERR_HIP, std::string("permute_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DSMOE_OK;
}

}  // namespace dsmoe

using namespace dsmoe;

// =============================================================== C ABI
extern "C" {

const char* dsmoe_last_error(void) { return g_last_error.c_str(); }

int dsmoe_version(void) { return 1; }

int dsmoe_gate_fwd(const void* x, const float* gate_w, const float* gate_bias, const dsmoe_dims* dims, float* logits,
                   int32_t* idx, int64_t* idx64, float* weights, void* weights_x, float* sel_scores, int32_t* counts,
                   void* stream) {
  int rc = validate(dims, false);
  if (rc) return rc;
  DSMOE_REQUIRE(x && gate_w && gate_bias && idx && weights, DSMOE_ERR_INVALID, "gate: NULL required pointer");
  GateOut o{logits, idx, idx64, weights, weights_x, sel_scores, counts};
  return launch_gate(x, nullptr, gate_w, gate_bias, *dims, o, static_cast<hipStream_t>(stream));
}

int dsmoe_route_from_logits(const float* logits, const float* gate_bias, const dsmoe_dims* dims, int32_t* idx,
                            int64_t* idx64, float* weights, void* weights_x, float* sel_scores, int32_t* counts,
                            void* stream) {
  int rc = validate(dims, false);
  if (rc) return rc;
  DSMOE_REQUIRE(logits && gate_bias && idx && weights, DSMOE_ERR_INVALID, "route: NULL required pointer");
  GateOut o{nullptr, idx, idx64, weights, weights_x, sel_scores, counts};
  return launch_gate(nullptr, logits, nullptr, gate_bias, *dims, o, static_cast<hipStream_t>(stream));
}

size_t dsmoe_permute_workspace_size(const dsmoe_dims* dims) {
  if (validate(dims, false)) return 0;
  Carver c(nullptr);
  return permute_scratch_carve(c, *dims, TILE_M, nullptr);
}

int dsmoe_permute(const int32_t* idx, const dsmoe_dims* dims, int32_t* offsets, int32_t* sorted_slot,
                  int32_t* sorted_token, int32_t* slot_pos, int32_t* counts, const void* x, void* x_sorted,
                  const float* weights, float* sorted_w, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate(dims, false);
  if (rc) return rc;
  DSMOE_REQUIRE(idx && offsets && sorted_slot && sorted_token && slot_pos, DSMOE_ERR_INVALID,
                "permute: NULL required pointer");
  DSMOE_REQUIRE((x == nullptr) == (x_sorted == nullptr), DSMOE_ERR_INVALID, "permute: x and x_sorted go together");
  DSMOE_REQUIRE((weights == nullptr) == (sorted_w == nullptr), DSMOE_ERR_INVALID,
                "permute: weights and sorted_w go together");
  const size_t need = dsmoe_permute_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "permute: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  Carver c(workspace);
  PermuteScratch ps;
  permute_scratch_carve(c, *dims, TILE_M, &ps);
  rc = launch_permute(idx, *dims,
                      permute_out(ps, TILE_M, offsets, sorted_slot, sorted_token, slot_pos, counts, weights, sorted_w),
                      false, st);
  if (rc) return rc;
  if (x)
    rc = launch_gather_rows(x, dims->T, sorted_token, (int64_t)dims->T * dims->k, dims->D, elem_size(dims->dtype),
                            x_sorted, st);
  return rc;
}

int dsmoe_permute_noalloc(const int32_t* idx, const dsmoe_dims* dims, int32_t* offsets, int32_t* sorted_slot,
                          int32_t* sorted_token, int32_t* slot_pos, int32_t* counts, const void* x, void* x_sorted,
                          const float* weights, float* sorted_w, void* stream) {
  int rc = validate(dims, false);
  if (rc) return rc;
  const size_t need = dsmoe_permute_workspace_size(dims);
  if (need > DSMOE_PERMUTE_NOALLOC_BYTES)
    return fail(DSMOE_ERR_UNSUPPORTED, "permute_noalloc: this call needs " + std::to_string(need) +
                                           " bytes of scratch, more than the static " +
                                           std::to_string((size_t)DSMOE_PERMUTE_NOALLOC_BYTES) +
                                           "; use dsmoe_permute with a workspace");
  void* ws = nullptr;
  rc = static_scratch(&ws);
  if (rc) return rc;
  // the same launches as dsmoe_permute; no scratch value is read before the
  // call writes it, so nothing needs clearing between calls
  return dsmoe_permute(idx, dims, offsets, sorted_slot, sorted_token, slot_pos, counts, x, x_sorted, weights, sorted_w,
                       ws, DSMOE_PERMUTE_NOALLOC_BYTES, stream);
}

static size_t grouped_ws(const dsmoe_dims& d, void* base, const void*** ptrs, int32_t** off32, MTile** sched,
                         int32_t** cnt, void** h) {
  Carver c(base);
  const void** p = c.take<const void*>(3 * d.E);
  int32_t* o = c.take<int32_t>(d.E + 1);
  MTile* s = c.take<MTile>(sched_bound(d.T, d.E, TILE_M));
  int32_t* n = c.take<int32_t>(1);
  void* hh = c.take<char>((size_t)d.T * d.I * elem_size(d.dtype));
  if (ptrs) {
    *ptrs = p; *off32 = o; *sched = s; *cnt = n; *h = hh;
  }
  return c.used();
}

size_t dsmoe_grouped_swiglu_workspace_size(const dsmoe_dims* dims) {
  if (!dims || dims->T < 0 || dims->E <= 0 || dims->D <= 0 || dims->I <= 0) return 0;
  return grouped_ws(*dims, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
}

int dsmoe_grouped_swiglu_fwd(const void* x_sorted, const void* const* w1, const void* const* w2, const void* const* w3,
                             const float* sorted_w, const int64_t* offsets, const dsmoe_dims* dims, void* y_sorted,
                             void* workspace, size_t workspace_bytes, void* stream) {
  DSMOE_REQUIRE(dims, DSMOE_ERR_INVALID, "dims is NULL");
  const dsmoe_dims& d = *dims;
  DSMOE_REQUIRE(d.dtype == DSMOE_F32 || d.dtype == DSMOE_BF16, DSMOE_ERR_UNSUPPORTED, "unsupported dtype");
  DSMOE_REQUIRE(d.T >= 0 && d.E > 0 && d.D > 0 && d.I > 0, DSMOE_ERR_INVALID, "grouped: bad dims");
  DSMOE_REQUIRE(x_sorted && w1 && w2 && w3 && offsets && y_sorted, DSMOE_ERR_INVALID, "grouped: NULL pointer");
  const size_t need = dsmoe_grouped_swiglu_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "grouped: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const void** ptrs;
  int32_t* off32;
  MTile* sched;
  int32_t* cnt;
  void* h;
  grouped_ws(d, workspace, &ptrs, &off32, &sched, &cnt, &h);
  int rc = upload_ptr_lists({{w1, d.E}, {w3, d.E}, {w2, d.E}}, ptrs, st);
  if (rc) return rc;
  const bool mf = all_aligned16(w1, d.E) && all_aligned16(w2, d.E) && all_aligned16(w3, d.E);
  GemmDesc g = desc_zero();
  g.A = x_sorted; g.lda = d.D; g.a_rows = d.T; g.B0 = ptrs; g.B1 = ptrs + d.E; g.ldb = d.D; g.kseg = d.D;
  g.N = d.I; g.K = d.D; g.C = h; g.ldc = d.I;
  GemmDesc g2 = desc_zero();
  g2.A = h; g2.lda = d.I; g2.a_rows = d.T; g2.B0 = ptrs + 2 * d.E; g2.ldb = d.I; g2.kseg = d.I;
  g2.N = d.D; g2.K = d.I; g2.C = y_sorted; g2.ldc = d.D;
  const bool mfr = gemm_mfma_eligible(g, d.dtype, mf) && gemm_mfma_eligible(g2, d.dtype, mf);
  const int bm = gemm_tile_m(mfr);
  rc = launch_sched_from_offsets(offsets, d.E, bm, d.T, off32, sched, cnt, st);
  if (rc) return rc;
  g.sched = g2.sched = sched;
  g.sched_count = g2.sched_count = cnt;
  g.m_tiles_bound = g2.m_tiles_bound = (int32_t)sched_bound(d.T, d.E, bm);
  g.bm = g2.bm = bm;
  rc = launch_grouped_gemm(g, EPI_SWIGLU, d.dtype, nullptr, mfr, st);
  if (rc) return rc;
  return launch_grouped_gemm(g2, EPI_STORE, d.dtype, sorted_w, mfr, st);
}

int dsmoe_combine_fwd(const void* o_slots, const float* weights, const int32_t* idx, const void* shared,
                      const dsmoe_dims* dims, void* y, void* stream) {
  int rc = validate(dims, false);
  if (rc) return rc;
  DSMOE_REQUIRE(o_slots && weights && idx && y, DSMOE_ERR_INVALID, "combine: NULL required pointer");
  return launch_combine(o_slots, nullptr, weights, idx, shared, *dims, y, static_cast<hipStream_t>(stream));
}

size_t dsmoe_moe_fwd_workspace_size(const dsmoe_dims* dims, int training) {
  if (validate(dims, true)) return 0;
  return fwd_layout(*dims, training, nullptr).total;
}

// Few-row (decode) GEMM path: tokens per inference call up to which it is taken.
constexpr int SK_MAX_T = SK_BM;

// Routed problem gr on the few-row kernel, with the dense shared problem gd
// in the same launch when that kernel takes it too (else on the general path).
static int launch_sk_pair(const GemmDesc& gr, const GemmDesc& gd, bool has_gd, int epi, int dtype, bool mf,
                          hipStream_t st) {
  if (!has_gd) return launch_gemm_sk(gr, epi, nullptr, st);
  GemmDesc d1 = gd;
  d1.bm = SK_BM;
  if (gemm_sk_ok(d1)) return launch_gemm_sk_pair(gr, d1, epi, nullptr, st);
  const int rc = launch_gemm_sk(gr, epi, nullptr, st);
  if (rc) return rc;
  return launch_grouped_gemm(gd, epi, dtype, nullptr, gemm_mfma_eligible(gd, dtype, mf), st);
}

int dsmoe_moe_fwd(const void* x, const float* gate_w, const float* gate_bias, const void* const* w1,
                  const void* const* w2, const void* const* w3, const void* const* sw1, const void* const* sw2,
                  const void* const* sw3, const dsmoe_dims* dims, int training, void* y, int64_t* idx64,
                  void* weights_x, int32_t* counts, float* logits, void* workspace, size_t workspace_bytes,
                  void* stream) {
  int rc = validate(dims, true);
  if (rc) return rc;
  const dsmoe_dims& d = *dims;
  DSMOE_REQUIRE(x && gate_w && gate_bias && w1 && w2 && w3 && y, DSMOE_ERR_INVALID, "moe_fwd: NULL required pointer");
  DSMOE_REQUIRE(d.S == 0 || (sw1 && sw2 && sw3), DSMOE_ERR_INVALID, "moe_fwd: NULL shared expert pointers");
  const size_t need = dsmoe_moe_fwd_workspace_size(dims, training);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "moe_fwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  FwdLayout L = fwd_layout(d, training, workspace);
  const int64_t N = (int64_t)d.T * d.k;
  StageTimer tm(st);

  // The weight pointer table goes to the device with the gate launch when it
  // fits one argument chunk and the MFMA gate runs, else with its own launch.
  const int ntab = 3 * d.E + 3 * d.S;
  const bool tab_in_gate = ntab <= PTR_CHUNK && gate_uses_mfma(x, gate_w, d);
  PtrChunk tabc;
  tabc.n = 0;
  tabc.off = 0;
  if (tab_in_gate) {
    for (const auto& l : {std::make_pair(w1, d.E), std::make_pair(w3, d.E), std::make_pair(w2, d.E),
                          std::make_pair(sw1, d.S), std::make_pair(sw3, d.S), std::make_pair(sw2, d.S)})
      for (int i = 0; i < l.second; ++i) tabc.p[tabc.n++] = l.first[i];
  } else {
    tm.begin(ST_TABLES);
    rc = upload_ptr_lists({{w1, d.E}, {w3, d.E}, {w2, d.E}, {sw1, d.S}, {sw3, d.S}, {sw2, d.S}}, L.ptrs, st);
    tm.end();
    if (rc) return rc;
  }
  const bool mf = all_aligned16(w1, d.E) && all_aligned16(w2, d.E) && all_aligned16(w3, d.E) &&
                  (d.S == 0 || (all_aligned16(sw1, d.S) && all_aligned16(sw2, d.S) && all_aligned16(sw3, d.S)));
  // GEMM descriptors; the routed schedule height follows the kernel choice
  GemmDesc g1 = desc_zero();
  g1.A = x; g1.lda = d.D; g1.a_rows = d.T; g1.a_map = L.sorted_token;
  g1.B0 = L.ptrs; g1.B1 = L.ptrs + d.E; g1.ldb = d.D; g1.kseg = d.D;
  g1.N = d.I; g1.K = d.D; g1.C = L.h; g1.ldc = d.I; g1.Gs = L.g; g1.Us = L.u;
  GemmDesc g2 = desc_zero();
  g2.A = L.h; g2.lda = d.I; g2.a_rows = N; g2.B0 = L.ptrs + 2 * d.E; g2.ldb = d.I; g2.kseg = d.I;
  // expert outputs stay in sorted order (rows written whole, in order); the
  // combine and the backward read slot s at row slot_pos[s]
  g2.N = d.D; g2.K = d.I; g2.C = L.o_sorted; g2.ldc = d.D;
  const bool mfr = gemm_mfma_eligible(g1, d.dtype, mf) && gemm_mfma_eligible(g2, d.dtype, mf);
  // Decode shapes (at most SK_MAX_T tokens, inference): every routed and
  // shared row tile fits the few-row kernel, which streams the weights once.
  bool sk = false;
  if (!training && d.dtype == DSMOE_BF16 && d.T <= SK_MAX_T && mf) {
    GemmDesc t1 = g1, t2 = g2;
    t1.bm = t2.bm = SK_BM;
    t1.Gs = t1.Us = nullptr;
    sk = gemm_sk_ok(t1) && gemm_sk_ok(t2);
  }
  const int bm = sk ? SK_BM : gemm_tile_m(mfr);
  // (a) gate; the MFMA gate's routing launch also ranks the slots for the
  // permute (and finishes it for a call of one rank block)
  const PermuteOut po = permute_out(L.ps, bm, L.offsets, L.sorted_slot, L.sorted_token, L.slot_pos, counts,
                                    training ? L.w : nullptr, L.sorted_w);
  GateOut go{logits, L.idx, idx64, L.w, weights_x, L.sel, nullptr};
  bool ranked = false;
  tm.begin(ST_GATE);
  rc = launch_gate(x, nullptr, gate_w, gate_bias, d, go, st, L.gate_part, tab_in_gate ? &tabc : nullptr, L.ptrs, &po,
                   &ranked);
  tm.end();
  if (rc) return rc;
  // (b) permute (counts are the exact per-expert totals, no atomics)
  tm.begin(ST_PERMUTE);
  rc = launch_permute(L.idx, d, po, ranked, st);
  if (!rc && training) {
    // the routed rows of x in sorted order, for the backward's weight
    // gradient (a K-major operand read without a row gather); gemm1 keeps
    // gathering from x, which stays cache-resident
    rc = launch_scatter_rows(x, d.T, d.k, L.slot_pos, L.sorted_token, d.D, elem_size(d.dtype), L.x_sorted, st);
  }
  tm.end();
  if (rc) return rc;
  g1.sched = g2.sched = L.ps.sched;
  g1.sched_count = g2.sched_count = L.ps.sched_count;
  g1.m_tiles_bound = g2.m_tiles_bound = (int32_t)sched_bound(N, d.E, bm);
  g1.bm = g2.bm = bm;
  // (c) gate/up + SwiGLU: routed rows gathered from x through sorted_token,
  // and the shared experts as S dense groups over all tokens (h_shared =
  // [h_0 | h_1 | ...]), in one launch when the persistent kernel takes both
  GemmDesc s1 = desc_zero(), s2 = desc_zero();
  if (d.S) {
    s1.dense_rows = d.T; s1.groups = d.S;
    s1.A = x; s1.lda = d.D; s1.a_rows = d.T;
    s1.B0 = L.ptrs + 3 * d.E; s1.B1 = L.ptrs + 3 * d.E + d.S; s1.ldb = d.D; s1.kseg = d.D;
    s1.N = d.I_s; s1.K = d.D; s1.C = L.hs; s1.ldc = (int64_t)d.S * d.I_s; s1.c_group_col = d.I_s;
    s1.Gs = L.gs; s1.Us = L.us;
    s1.bm = gemm_tile_m(gemm_mfma_eligible(s1, d.dtype, mf));
    // shared down projection: one GEMM with K = S * I_s summing all shared experts
    s2.dense_rows = d.T; s2.groups = 1;
    s2.A = L.hs; s2.lda = (int64_t)d.S * d.I_s; s2.a_rows = d.T;
    s2.B0 = L.ptrs + 3 * d.E + 2 * d.S; s2.ldb = d.I_s; s2.kseg = d.I_s; s2.nseg = d.S;
    s2.N = d.D; s2.K = d.S * d.I_s; s2.C = L.shared_out; s2.ldc = d.D;
    s2.bm = gemm_tile_m(gemm_mfma_eligible(s2, d.dtype, mf));
  }
  if (sk) g1.Gs = g1.Us = s1.Gs = s1.Us = nullptr;  // inference: no pre-activation saves
  tm.begin(ST_GEMM1);
  rc = sk ? launch_sk_pair(g1, s1, d.S > 0, EPI_SWIGLU, d.dtype, mf, st)
          : d.S ? launch_grouped_gemm_pair(g1, s1, EPI_SWIGLU, d.dtype, nullptr, mfr, mf, st)
                : launch_grouped_gemm(g1, EPI_SWIGLU, d.dtype, nullptr, mfr, st);
  tm.end();
  if (rc) return rc;
  // down projections: routed rows written in expert-sorted order (row r of
  // o_sorted is sorted position r); the combine and the backward read slot s
  // at row slot_pos[s]
  tm.begin(ST_GEMM2);
  rc = sk ? launch_sk_pair(g2, s2, d.S > 0, EPI_STORE, d.dtype, mf, st)
          : d.S ? launch_grouped_gemm_pair(g2, s2, EPI_STORE, d.dtype, nullptr, mfr, mf, st)
                : launch_grouped_gemm(g2, EPI_STORE, d.dtype, nullptr, mfr, st);
  tm.end();
  if (rc) return rc;
  // (d) combine
  tm.begin(ST_COMBINE);
  rc = launch_combine(L.o_sorted, L.slot_pos, L.w, L.idx, L.shared_out, d, y, st);
  tm.end();
  tm.call_done(0);
  return rc;
}

// Backward workspace layout (device pointer tables, then buffers).
struct BwdLayout {
  const void** w1;
  const void** w3;
  const void** w2;
  const void** w13;   // [w1_e, w3_e] per expert: the two K segments of dx
  const void** sw1;
  const void** sw3;
  const void** sw2;
  const void** sw13;  // [sw1_0, sw3_0, sw1_1, sw3_1, ...]: one group, 2S segments, or the stack below
  void* sw13_stack;   // bf16, S > 1: the 2S blocks copied into one (2 S I_s, D) matrix (one K segment)
  void** dw1;
  void** dw3;
  void** dw2;
  void** dsw1;
  void** dsw3;
  void** dsw2;
  float* dw;          // (N) d weights, slot order
  float* dlog;        // (N) d logits of the selected experts, slot order
  MTile* sched;
  int32_t* sched_count;
  void* dgdu;         // (N, 2I)   [dg | du] in sorted order
  void* dx_slots;     // (N, D)    slot order
  void* dgdu_s;       // (T, 2 S I_s)
  void* dx_shared;    // (T, D)
  void* dy_w;         // bf16: (N, D) w * dY in sorted order (K-major operand of dW2)
  int ks13, ks2;      // split-K of the shared-expert weight gradients (bf16 MFMA path)
  float* part;        // fp32 split-K partials, max(ks13 * 2 I_s, ks2 * I_s) * S * D
  size_t total;
};

constexpr int BWD_BM = 256;  // schedule height of the backward GEMMs (MFMA tile; the SIMT tiles split it)

static BwdLayout bwd_layout(const dsmoe_dims& d, void* base) {
  Carver c(base);
  BwdLayout B;
  const int64_t N = (int64_t)d.T * d.k;
  const int es = elem_size(d.dtype);
  // pointer tables: one contiguous block, routed weights, shared weights,
  // routed gradients, shared gradients (uploaded in one call, in this order)
  const void** rt = c.take<const void*>(8 * d.E + 8 * d.S);
  B.w1 = rt;
  B.w3 = rt + d.E;
  B.w2 = rt + 2 * d.E;
  B.w13 = rt + 3 * d.E;
  const void** st = rt + 5 * d.E;
  B.sw1 = st;
  B.sw3 = st + d.S;
  B.sw2 = st + 2 * d.S;
  B.sw13 = st + 3 * d.S;
  void** ro = const_cast<void**>(st + 5 * d.S);
  B.dw1 = ro;
  B.dw3 = ro + d.E;
  B.dw2 = ro + 2 * d.E;
  void** so = ro + 3 * d.E;
  B.dsw1 = so;
  B.dsw3 = so + d.S;
  B.dsw2 = so + 2 * d.S;
  B.dw = c.take<float>(N);
  B.dlog = c.take<float>(N);
  B.sched = c.take<MTile>(sched_bound(N, d.E, BWD_BM));
  B.sched_count = c.take<int32_t>(1);
  B.dgdu = c.take<char>((size_t)N * 2 * d.I * es);
  B.dx_slots = c.take<char>((size_t)N * d.D * es);
  B.dgdu_s = d.S ? c.take<char>((size_t)d.T * 2 * d.S * d.I_s * es) : nullptr;
  B.dx_shared = d.S ? c.take<char>((size_t)d.T * d.D * es) : nullptr;
  // the shared dx GEMM sums 2S K segments; the quad-wave kernel takes two, so
  // for S > 1 the shared W1 / W3 blocks are first copied into one matrix
  B.sw13_stack = (d.S > 1 && d.dtype == DSMOE_BF16) ? c.take<char>((size_t)2 * d.S * d.I_s * d.D * es) : nullptr;
  // w * dY gathered in sorted order, for bf16 rows of whole 16-byte chunks;
  // other widths read dY through the row map with the weight as a k scale
  B.dy_w = (d.dtype == DSMOE_BF16 && d.D % 8 == 0) ? c.take<char>((size_t)N * d.D * es) : nullptr;
  B.ks13 = B.ks2 = 1;
  B.part = nullptr;
  if (d.S && d.dtype == DSMOE_BF16) {
    B.ks13 = xgemm_pick_ksplit(xgemm_tiles(2 * (int64_t)d.I_s, d.D, d.S), d.T);
    B.ks2 = xgemm_pick_ksplit(xgemm_tiles(d.D, d.I_s, d.S), d.T);
    const int64_t n13 = B.ks13 > 1 ? (int64_t)B.ks13 * 2 * d.I_s : 0;
    const int64_t n2 = B.ks2 > 1 ? (int64_t)B.ks2 * d.I_s : 0;
    const int64_t nmax = std::max(n13, n2);
    if (nmax) B.part = c.take<float>(nmax * d.S * d.D);
  }
  B.total = c.used();
  return B;
}

static XGemm xdesc_zero() {
  XGemm g;
  std::memset(static_cast<void*>(&g), 0, sizeof(g));
  g.nseg = 1;
  return g;
}

size_t dsmoe_moe_bwd_workspace_size(const dsmoe_dims* dims) {
  if (validate(dims, true)) return 0;
  return bwd_layout(*dims, nullptr).total;
}

int dsmoe_moe_bwd(const void* x, const float* gate_w, const void* const* w1, const void* const* w2,
                  const void* const* w3, const void* const* sw1, const void* const* sw2, const void* const* sw3,
                  const dsmoe_dims* dims, const void* dy, const void* fwd_workspace, void* dx, float* dgate_w,
                  void* const* dw1, void* const* dw2, void* const* dw3, void* const* dsw1, void* const* dsw2,
                  void* const* dsw3, void* workspace, size_t workspace_bytes, void* stream) {
  if (!dims) return fail(DSMOE_ERR_INVALID, "dims is NULL");
  return dsmoe_moe_bwd_ex(x, gate_w, w1, w2, w3, sw1, sw2, sw3, dims, dy, fwd_workspace, dx, dgate_w, dw1, dw2, dw3,
                          dsw1, dsw2, dsw3, dims->dtype, workspace, workspace_bytes, stream);
}

int dsmoe_moe_bwd_ex(const void* x, const float* gate_w, const void* const* w1, const void* const* w2,
                     const void* const* w3, const void* const* sw1, const void* const* sw2, const void* const* sw3,
                     const dsmoe_dims* dims, const void* dy, const void* fwd_workspace, void* dx, float* dgate_w,
                     void* const* dw1, void* const* dw2, void* const* dw3, void* const* dsw1, void* const* dsw2,
                     void* const* dsw3, int dw_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = validate(dims, true);
  if (rc) return rc;
  const dsmoe_dims& d = *dims;
  DSMOE_REQUIRE(dw_dtype == d.dtype || dw_dtype == DSMOE_F32, DSMOE_ERR_UNSUPPORTED,
                "moe_bwd: expert weight gradients are written in the compute dtype or fp32");
  const int32_t dw_f32 = dw_dtype == DSMOE_F32 && d.dtype != DSMOE_F32;
  DSMOE_REQUIRE(x && gate_w && w1 && w2 && w3 && dy && fwd_workspace && dx && dgate_w && dw1 && dw2 && dw3,
                DSMOE_ERR_INVALID, "moe_bwd: NULL required pointer");
  DSMOE_REQUIRE(d.S == 0 || (sw1 && sw2 && sw3 && dsw1 && dsw2 && dsw3), DSMOE_ERR_INVALID,
                "moe_bwd: NULL shared expert pointers");
  const size_t need = dsmoe_moe_bwd_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "moe_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the forward layout of a training call (the caller passes that workspace)
  const FwdLayout F = fwd_layout(d, 1, const_cast<void*>(fwd_workspace));
  BwdLayout B = bwd_layout(d, workspace);
  const int64_t N = (int64_t)d.T * d.k;
  StageTimer tm(st);

  std::vector<const void*> w13h(2 * d.E), sw13h(2 * d.S + 1);
  for (int e = 0; e < d.E; ++e) {
    w13h[2 * e] = w1[e];
    w13h[2 * e + 1] = w3[e];
  }
  for (int s = 0; s < d.S; ++s) {
    sw13h[2 * s] = sw1[s];
    sw13h[2 * s + 1] = sw3[s];
  }
  if (B.sw13_stack) sw13h[0] = B.sw13_stack;   // one segment: the stacked copy
  // MFMA backward GEMMs need every weight and weight-gradient pointer 16-byte aligned
  const bool mf = all_aligned16(w1, d.E) && all_aligned16(w2, d.E) && all_aligned16(w3, d.E) &&
                  all_aligned16((const void* const*)dw1, d.E) && all_aligned16((const void* const*)dw2, d.E) &&
                  all_aligned16((const void* const*)dw3, d.E) &&
                  (d.S == 0 || (all_aligned16(sw1, d.S) && all_aligned16(sw2, d.S) && all_aligned16(sw3, d.S) &&
                                all_aligned16((const void* const*)dsw1, d.S) &&
                                all_aligned16((const void* const*)dsw2, d.S) &&
                                all_aligned16((const void* const*)dsw3, d.S)));
  tm.begin(ST_BWD_PREP);
  // the four table groups are one contiguous block, in this order
  rc = upload_ptr_lists({{w1, d.E}, {w3, d.E}, {w2, d.E}, {w13h.data(), 2 * d.E},
                         {sw1, d.S}, {sw3, d.S}, {sw2, d.S}, {sw13h.data(), 2 * d.S},
                         {(const void* const*)dw1, d.E}, {(const void* const*)dw3, d.E}, {(const void* const*)dw2, d.E},
                         {(const void* const*)dsw1, d.S}, {(const void* const*)dsw3, d.S},
                         {(const void* const*)dsw2, d.S}},
                        B.w1, st);
  if (rc) return rc;
  // gate gradient path: d weights -> d logits
  rc = launch_prep_tok(dy, F.o_sorted, F.slot_pos, F.w, F.slot_pos, d.T, d.k, d.D, d.dtype, B.dw, B.dy_w, st);
  if (rc == DSMOE_ERR_UNSUPPORTED) {
    rc = launch_dw_dot(dy, F.o_sorted, F.slot_pos, N, d.k, d.D, d.dtype, B.dw, st);
    if (!rc && B.dy_w) rc = launch_scale_gather_rows(dy, F.sorted_token, F.sorted_w, N, d.D, B.dy_w, st);
  }
  if (!rc) rc = launch_gate_bwd(B.dw, F.sel, d.T, d.k, d.route_scale, B.dlog, st);
  if (!rc) rc = launch_sched32(F.offsets, d.E, BWD_BM, B.sched, B.sched_count, st);
  tm.end();
  if (rc) return rc;
  const int32_t mbound = (int32_t)sched_bound(N, d.E, BWD_BM);

  // The routed dW2, the shared experts' chain and dW_gate depend only on the
  // preparation above: with stage timing off they go on a second stream while
  // the routed dh, dx and dW1|dW3 run on the caller's, so the last, partly
  // filled round of workgroups of each launch can take work from the other
  // chain.  The caller's stream waits for the second before the dx sum.
  hipStream_t ss = st;
  SideStream* side = tm.on() ? nullptr : side_stream(st);
  if (side && hipEventRecord(side->fork, st) == hipSuccess && hipStreamWaitEvent(side->s, side->fork, 0) == hipSuccess)
    ss = side->s;
  const auto join = [&](int r) {
    if (ss != st && (hipEventRecord(side->join, ss) != hipSuccess || hipStreamWaitEvent(st, side->join, 0) != hipSuccess))
      return r ? r : fail(DSMOE_ERR_HIP, "moe_bwd: cannot join the second stream");
    return r;
  };
  XGemm w2g = xdesc_zero();
  w2g.sched_mode = XS_WGRAD; w2g.groups = d.E; w2g.k_off = F.offsets; w2g.M = d.D; w2g.N = d.I; w2g.K = (int32_t)N;
  w2g.a_mode = XA_KMAJOR; w2g.lda = d.D;
  if (B.dy_w) {
    w2g.A = B.dy_w;  // w * dY already gathered and rounded once
  } else {
    w2g.A = dy; w2g.a_map = F.sorted_token; w2g.a_kscale = F.sorted_w;
  }
  w2g.b_mode = XB_ACT_KMAJOR; w2g.Bact = F.h; w2g.ldb = d.I;
  w2g.Ctab0 = B.dw2; w2g.Ctab1 = B.dw2; w2g.msplit = d.D; w2g.ldc = d.I; w2g.c_f32 = dw_f32;
  tm.begin(ST_BWD_DW2);
  rc = launch_xgemm(w2g, XE_WGRAD, d.dtype, mf, ss);
  tm.end();
  if (rc) return join(rc);

  if (d.S) {
    const int64_t SIs = (int64_t)d.S * d.I_s;
    XGemm sh = xdesc_zero();
    sh.sched_mode = XS_DENSE; sh.dense_rows = d.T; sh.groups = d.S; sh.N = d.I_s; sh.K = d.D;
    sh.a_mode = XA_ROWS; sh.A = dy; sh.lda = d.D;
    sh.b_mode = XB_W_NN; sh.Btab = B.sw2; sh.ldb = d.I_s; sh.kseg = d.D;
    sh.C = B.dgdu_s; sh.ldc = 2 * SIs; sh.c_group_col = 2 * (int64_t)d.I_s; sh.du_off = d.I_s;
    sh.Gs = F.gs; sh.Us = F.us; sh.ld_gu = SIs; sh.gu_group_col = d.I_s;
    tm.begin(ST_BWD_DH_SHARED);
    rc = launch_xgemm(sh, XE_SWIGLU_BWD, d.dtype, mf, ss);
    tm.end();
    if (rc) return join(rc);
    XGemm sx = xdesc_zero();
    sx.sched_mode = XS_DENSE; sx.dense_rows = d.T; sx.groups = 1; sx.N = d.D; sx.K = (int32_t)(2 * SIs);
    sx.a_mode = XA_ROWS; sx.A = B.dgdu_s; sx.lda = 2 * SIs;
    sx.b_mode = XB_W_NN; sx.Btab = B.sw13; sx.ldb = d.D; sx.kseg = d.I_s; sx.nseg = 2 * d.S;
    sx.C = B.dx_shared; sx.ldc = d.D;
    tm.begin(ST_BWD_DX_SHARED);
    if (B.sw13_stack) {
      const size_t blk = (size_t)d.I_s * d.D * elem_size(d.dtype);
      for (int s = 0; s < d.S && !rc; ++s)
        for (int h = 0; h < 2 && !rc; ++h)
          if (hipMemcpyAsync(static_cast<char*>(B.sw13_stack) + (2 * s + h) * blk, h ? sw3[s] : sw1[s], blk,
                             hipMemcpyDeviceToDevice, ss) != hipSuccess)
            rc = fail(DSMOE_ERR_HIP, "moe_bwd: shared weight stack copy failed");
      sx.kseg = (int32_t)(2 * SIs);
      sx.nseg = 1;
    }
    if (!rc) rc = launch_xgemm(sx, XE_STORE, d.dtype, mf, ss);
    tm.end();
    if (rc) return join(rc);
    XGemm s13 = xdesc_zero();
    s13.sched_mode = XS_WGRAD; s13.groups = d.S; s13.M = 2 * d.I_s; s13.N = d.D; s13.K = d.T;
    s13.a_mode = XA_KMAJOR; s13.A = B.dgdu_s; s13.lda = 2 * SIs; s13.a_col = 2 * (int64_t)d.I_s;
    s13.b_mode = XB_ACT_KMAJOR; s13.Bact = x; s13.ldb = d.D;
    s13.Ctab0 = B.dsw1; s13.Ctab1 = B.dsw3; s13.msplit = d.I_s; s13.ldc = d.D;
    s13.ksplit = B.ks13; s13.part = B.part; s13.c_f32 = dw_f32;
    XGemm s2 = xdesc_zero();
    s2.sched_mode = XS_WGRAD; s2.groups = d.S; s2.M = d.D; s2.N = d.I_s; s2.K = d.T;
    s2.a_mode = XA_KMAJOR; s2.A = dy; s2.lda = d.D;
    s2.b_mode = XB_ACT_KMAJOR; s2.Bact = F.hs; s2.ldb = SIs; s2.b_col = d.I_s;
    s2.Ctab0 = B.dsw2; s2.Ctab1 = B.dsw2; s2.msplit = d.D; s2.ldc = d.I_s;
    s2.ksplit = B.ks2; s2.part = B.part; s2.c_f32 = dw_f32;
    tm.begin(ST_BWD_DW_SHARED);
    rc = launch_xgemm(s13, XE_WGRAD, d.dtype, mf, ss);
    if (!rc) rc = launch_xgemm(s2, XE_WGRAD, d.dtype, mf, ss);
    tm.end();
    if (rc) return join(rc);
  }
  tm.begin(ST_BWD_GATE);
  rc = launch_dwgate(x, B.dlog, F.sorted_slot, F.sorted_token, F.offsets, d.E, d.D, d.dtype, dgate_w, ss);
  tm.end();
  if (rc) return join(rc);
  // routed dh = w * (dy W2), SwiGLU backward -> [dg | du]
  XGemm h = xdesc_zero();
  h.sched_mode = XS_ROUTED; h.sched = B.sched; h.sched_count = B.sched_count; h.m_tiles_bound = mbound;
  h.bm = BWD_BM; h.N = d.I; h.K = d.D;
  h.a_mode = XA_ROWS; h.A = dy; h.lda = d.D; h.a_map = F.sorted_token;
  h.b_mode = XB_W_NN; h.Btab = B.w2; h.ldb = d.I; h.kseg = d.D;
  h.C = B.dgdu; h.ldc = 2 * (int64_t)d.I; h.du_off = d.I;
  h.Gs = F.g; h.Us = F.u; h.ld_gu = d.I; h.row_w = F.sorted_w;
  tm.begin(ST_BWD_DH);
  rc = launch_xgemm(h, XE_SWIGLU_BWD, d.dtype, mf, st);
  tm.end();
  if (rc) return join(rc);
  // routed dx_slot = [dg | du] [W1; W3], rows back to slot order
  XGemm xg = xdesc_zero();
  xg.sched_mode = XS_ROUTED; xg.sched = B.sched; xg.sched_count = B.sched_count; xg.m_tiles_bound = mbound;
  xg.bm = BWD_BM; xg.N = d.D; xg.K = 2 * d.I;
  xg.a_mode = XA_ROWS; xg.A = B.dgdu; xg.lda = 2 * (int64_t)d.I;
  xg.b_mode = XB_W_NN; xg.Btab = B.w13; xg.ldb = d.D; xg.kseg = d.I; xg.nseg = 2;
  xg.C = B.dx_slots; xg.ldc = d.D; xg.c_map = F.sorted_slot;
  tm.begin(ST_BWD_DX);
  rc = launch_xgemm(xg, XE_STORE, d.dtype, mf, st);
  tm.end();
  if (rc) return join(rc);
  // routed dW1, dW3 = [dg | du]^T X_e ; dW2 = (w dY)^T H_e
  XGemm w13 = xdesc_zero();
  w13.sched_mode = XS_WGRAD; w13.groups = d.E; w13.k_off = F.offsets; w13.M = 2 * d.I; w13.N = d.D; w13.K = (int32_t)N;
  w13.a_mode = XA_KMAJOR; w13.A = B.dgdu; w13.lda = 2 * (int64_t)d.I;
  w13.b_mode = XB_ACT_KMAJOR; w13.Bact = F.x_sorted; w13.ldb = d.D;
  w13.Ctab0 = B.dw1; w13.Ctab1 = B.dw3; w13.msplit = d.I; w13.ldc = d.D; w13.c_f32 = dw_f32;
  tm.begin(ST_BWD_DW13);
  rc = launch_xgemm(w13, XE_WGRAD, d.dtype, mf, st);
  tm.end();
  if (rc) return join(rc);
  rc = join(rc);
  if (rc) return rc;
  tm.begin(ST_BWD_REDUCE);
  rc = launch_dx_final(B.dx_slots, B.dx_shared, B.dlog, F.idx, gate_w, d.T, d.D, d.k, d.dtype, dx, st);
  tm.end();
  tm.call_done(1);
  return rc;
}

// Backward of the operator seam (models/moe_triton.py:438-501).  The forward
// gate/up GEMM is recomputed (g, u, h), then the same grouped GEMMs as the
// layer backward run with identity row maps: dh -> [dg | du] (SwiGLU
// backward epilogue), dx = [dg | du] [W1; W3], dW1 | dW3 = [dg | du]^T X_e and
// dW2 = dY_e^T H_e per expert, fp32 accumulation in ascending row order.
struct GroupedBwdLayout {
  const void** w1;   // [w1 E][w3 E][w2 E][w13 2E]
  const void** w3;
  const void** w2;
  const void** w13;
  void** dw1;        // [dw1 E][dw3 E][dw2 E]
  void** dw3;
  void** dw2;
  int32_t* off32;
  MTile* sched_f;    // forward recompute schedule (MFMA or SIMT tile height)
  int32_t* cnt_f;
  MTile* sched_b;    // backward schedule (BWD_BM)
  int32_t* cnt_b;
  void* g;
  void* u;
  void* h;
  void* dgdu;
  size_t total;
};

// bm_f: tile height the forward schedule is sized for (the smallest one a
// launch may use, so one layout serves both kernel choices).
static GroupedBwdLayout grouped_bwd_layout(const dsmoe_dims& d, int bm_f, void* base) {
  Carver c(base);
  GroupedBwdLayout B;
  const int64_t N = d.T;
  const int es = elem_size(d.dtype);
  const void** t = c.take<const void*>(5 * d.E);
  B.w1 = t; B.w3 = t + d.E; B.w2 = t + 2 * d.E; B.w13 = t + 3 * d.E;
  void** o = c.take<void*>(3 * d.E);
  B.dw1 = o; B.dw3 = o + d.E; B.dw2 = o + 2 * d.E;
  B.off32 = c.take<int32_t>(d.E + 1);
  B.sched_f = c.take<MTile>(sched_bound(N, d.E, bm_f));
  B.cnt_f = c.take<int32_t>(1);
  B.sched_b = c.take<MTile>(sched_bound(N, d.E, BWD_BM));
  B.cnt_b = c.take<int32_t>(1);
  B.g = c.take<char>((size_t)N * d.I * es);
  B.u = c.take<char>((size_t)N * d.I * es);
  B.h = c.take<char>((size_t)N * d.I * es);
  B.dgdu = c.take<char>((size_t)N * 2 * d.I * es);
  B.total = c.used();
  return B;
}

static bool grouped_dims_ok(const dsmoe_dims* dims) {
  return dims && (dims->dtype == DSMOE_F32 || dims->dtype == DSMOE_BF16) && dims->T >= 0 && dims->E > 0 &&
         dims->D > 0 && dims->I > 0;
}

size_t dsmoe_grouped_swiglu_bwd_workspace_size(const dsmoe_dims* dims) {
  if (!grouped_dims_ok(dims)) return 0;
  return grouped_bwd_layout(*dims, TILE_M, nullptr).total;
}

int dsmoe_grouped_swiglu_bwd(const void* x_sorted, const void* const* w1, const void* const* w2, const void* const* w3,
                             const int64_t* offsets, const void* dy_sorted, const dsmoe_dims* dims, void* dx_sorted,
                             void* const* dw1, void* const* dw2, void* const* dw3, void* workspace,
                             size_t workspace_bytes, void* stream) {
  DSMOE_REQUIRE(grouped_dims_ok(dims), DSMOE_ERR_INVALID, "grouped_bwd: bad dims");
  const dsmoe_dims& d = *dims;
  DSMOE_REQUIRE(x_sorted && w1 && w2 && w3 && offsets && dy_sorted && dx_sorted && dw1 && dw2 && dw3,
                DSMOE_ERR_INVALID, "grouped_bwd: NULL pointer");
  const size_t need = dsmoe_grouped_swiglu_bwd_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "grouped_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t N = d.T;
  const bool mf = all_aligned16(w1, d.E) && all_aligned16(w2, d.E) && all_aligned16(w3, d.E) &&
                  all_aligned16((const void* const*)dw1, d.E) && all_aligned16((const void* const*)dw2, d.E) &&
                  all_aligned16((const void* const*)dw3, d.E);
  // forward recompute descriptor (its tile height decides the forward schedule)
  GemmDesc g1 = desc_zero();
  g1.A = x_sorted; g1.lda = d.D; g1.a_rows = N; g1.ldb = d.D; g1.kseg = d.D;
  g1.N = d.I; g1.K = d.D; g1.ldc = d.I;
  const bool mfr = gemm_mfma_eligible(g1, d.dtype, mf);
  const int bm_f = gemm_tile_m(mfr);
  GroupedBwdLayout B = grouped_bwd_layout(d, TILE_M, workspace);
  std::vector<const void*> w13h(2 * d.E);
  for (int e = 0; e < d.E; ++e) {
    w13h[2 * e] = w1[e];
    w13h[2 * e + 1] = w3[e];
  }
  int rc = upload_ptr_lists({{w1, d.E}, {w3, d.E}, {w2, d.E}, {w13h.data(), 2 * d.E}}, B.w1, st);
  if (!rc)
    rc = upload_ptr_lists({{(const void* const*)dw1, d.E}, {(const void* const*)dw3, d.E},
                           {(const void* const*)dw2, d.E}},
                          (const void**)B.dw1, st);
  if (!rc) rc = launch_sched_from_offsets(offsets, d.E, bm_f, N, B.off32, B.sched_f, B.cnt_f, st);
  if (!rc) rc = launch_sched32(B.off32, d.E, BWD_BM, B.sched_b, B.cnt_b, st);
  if (rc) return rc;
  // recompute g = X W1^T, u = X W3^T, h = silu(g) * u
  g1.B0 = B.w1; g1.B1 = B.w3; g1.C = B.h; g1.Gs = B.g; g1.Us = B.u;
  g1.sched = B.sched_f; g1.sched_count = B.cnt_f; g1.m_tiles_bound = (int32_t)sched_bound(N, d.E, bm_f); g1.bm = bm_f;
  rc = launch_grouped_gemm(g1, EPI_SWIGLU, d.dtype, nullptr, mfr, st);
  if (rc) return rc;
  const int32_t mbound = (int32_t)sched_bound(N, d.E, BWD_BM);
  // dh = dY W2, SwiGLU backward -> [dg | du]
  XGemm h = xdesc_zero();
  h.sched_mode = XS_ROUTED; h.sched = B.sched_b; h.sched_count = B.cnt_b; h.m_tiles_bound = mbound;
  h.bm = BWD_BM; h.N = d.I; h.K = d.D;
  h.a_mode = XA_ROWS; h.A = dy_sorted; h.lda = d.D;
  h.b_mode = XB_W_NN; h.Btab = B.w2; h.ldb = d.I; h.kseg = d.D;
  h.C = B.dgdu; h.ldc = 2 * (int64_t)d.I; h.du_off = d.I;
  h.Gs = B.g; h.Us = B.u; h.ld_gu = d.I;
  rc = launch_xgemm(h, XE_SWIGLU_BWD, d.dtype, mf, st);
  if (rc) return rc;
  // dx = [dg | du] [W1; W3]
  XGemm xg = xdesc_zero();
  xg.sched_mode = XS_ROUTED; xg.sched = B.sched_b; xg.sched_count = B.cnt_b; xg.m_tiles_bound = mbound;
  xg.bm = BWD_BM; xg.N = d.D; xg.K = 2 * d.I;
  xg.a_mode = XA_ROWS; xg.A = B.dgdu; xg.lda = 2 * (int64_t)d.I;
  xg.b_mode = XB_W_NN; xg.Btab = B.w13; xg.ldb = d.D; xg.kseg = d.I; xg.nseg = 2;
  xg.C = dx_sorted; xg.ldc = d.D;
  rc = launch_xgemm(xg, XE_STORE, d.dtype, mf, st);
  if (rc) return rc;
  // dW1 | dW3 = [dg | du]^T X_e ; dW2 = dY_e^T H_e
  XGemm w13 = xdesc_zero();
  w13.sched_mode = XS_WGRAD; w13.groups = d.E; w13.k_off = B.off32; w13.M = 2 * d.I; w13.N = d.D; w13.K = (int32_t)N;
  w13.a_mode = XA_KMAJOR; w13.A = B.dgdu; w13.lda = 2 * (int64_t)d.I;
  w13.b_mode = XB_ACT_KMAJOR; w13.Bact = x_sorted; w13.ldb = d.D;
  w13.Ctab0 = B.dw1; w13.Ctab1 = B.dw3; w13.msplit = d.I; w13.ldc = d.D;
  rc = launch_xgemm(w13, XE_WGRAD, d.dtype, mf, st);
  if (rc) return rc;
  XGemm w2g = xdesc_zero();
  w2g.sched_mode = XS_WGRAD; w2g.groups = d.E; w2g.k_off = B.off32; w2g.M = d.D; w2g.N = d.I; w2g.K = (int32_t)N;
  w2g.a_mode = XA_KMAJOR; w2g.A = dy_sorted; w2g.lda = d.D;
  w2g.b_mode = XB_ACT_KMAJOR; w2g.Bact = B.h; w2g.ldb = d.I;
  w2g.Ctab0 = B.dw2; w2g.Ctab1 = B.dw2; w2g.msplit = d.D; w2g.ldc = d.I;
  return launch_xgemm(w2g, XE_WGRAD, d.dtype, mf, st);
}

int dsmoe_update_bias(const int32_t* counts, float* gate_bias, int E, float speed, float upper, float lower,
                      void* stream) {
  DSMOE_REQUIRE(counts && gate_bias && E > 0, DSMOE_ERR_INVALID, "update_bias: bad arguments");
  return launch_update_bias(counts, gate_bias, E, speed, upper, lower, static_cast<hipStream_t>(stream));
}

int dsmoe_update_bias_f32(const float* counts, float* gate_bias, int E, float speed, float upper, float lower,
                          void* stream) {
  DSMOE_REQUIRE(counts && gate_bias && E > 0, DSMOE_ERR_INVALID, "update_bias_f32: bad arguments");
  return launch_update_bias_f32(counts, gate_bias, E, speed, upper, lower, static_cast<hipStream_t>(stream));
}

size_t dsmoe_moe_fwd_workspace_offset(const dsmoe_dims* dims, int training, int buffer) {
  if (validate(dims, true)) return (size_t)-1;
  // carve the layout at a stand-in base address; pointers minus the base are
  // the byte offsets (the layout aligns every buffer to 256 bytes)
  constexpr uintptr_t kBase = uintptr_t(1) << 20;
  const FwdLayout L = fwd_layout(*dims, training, reinterpret_cast<void*>(kBase));
  const void* p = nullptr;
  switch (buffer) {
    case DSMOE_WS_IDX: p = L.idx; break;
    case DSMOE_WS_WEIGHTS: p = L.w; break;
    case DSMOE_WS_SEL_SCORES: p = L.sel; break;
    case DSMOE_WS_OFFSETS: p = L.offsets; break;
    case DSMOE_WS_SORTED_SLOT: p = L.sorted_slot; break;
    case DSMOE_WS_SORTED_TOKEN: p = L.sorted_token; break;
    case DSMOE_WS_SLOT_POS: p = L.slot_pos; break;
    default: return (size_t)-1;
  }
  return (size_t)(reinterpret_cast<uintptr_t>(p) - kBase);
}

int dsmoe_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  for (auto& r : g_timing.recs) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  g_timing.recs.clear();
  g_timing.calls.clear();
  g_timing.on = on != 0;
  return DSMOE_OK;
}

int dsmoe_timing_read(double* stage_ms, int max_stages, int* n_calls) {
  std::lock_guard<std::mutex> lk(g_timing.mu);
  for (int i = 0; i < max_stages; ++i) stage_ms[i] = 0.0;
  for (auto& r : g_timing.recs) {
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(DSMOE_ERR_HIP, "timing: event sync failed");
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return fail(DSMOE_ERR_HIP, "timing: elapsed failed");
    if (r.stage < max_stages) stage_ms[r.stage] += ms;
  }
  if (n_calls) *n_calls = (int)g_timing.calls.size();
  return ST_COUNT;
}

const char* dsmoe_timing_stage_name(int stage) {
  return (stage >= 0 && stage < ST_COUNT) ? kStageNames[stage] : "";
}

}  // extern "C"
