/* dsmoe — MI355X (gfx950) DeepSeekMoE layer hot path behind a C ABI.
 *
 * Every function takes raw device pointers, plain sizes and a HIP stream
 * (passed as void*), returns an int status (0 = ok, negative = error, see
 * DSMOE_ERR_*) and never throws.  dsmoe_last_error() gives a thread-local
 * message for the last failing call on the calling thread.
 *
 * Ownership: the caller allocates every buffer, including the workspace whose
 * size the *_workspace_size() functions report.  The library allocates and
 * frees no device memory and keeps no pointer past a call.  All work is
 * enqueued on the given stream; no function synchronises the host.
 *
 * Layouts (row-major, as nn.Linear stores them):
 *   x, y            (T, D)      activations, dtype DSMOE_F32 or DSMOE_BF16
 *   gate_w          (E, D)      fp32          gate.weight
 *   gate_bias       (E)         fp32          gate.bias (buffer)
 *   w1[e], w3[e]    (I, D)      activation dtype   experts.{e}.w1/w3.weight
 *   w2[e]           (D, I)      activation dtype   experts.{e}.w2.weight
 *   sw1/sw3[s]      (I_s, D), sw2[s] (D, I_s)      shared_experts.{s}.*
 * Per-expert weights are passed as HOST arrays of device pointers, so the
 * module's separate per-expert tensors are used in place (no re-stacking).
 *
 * Routing conventions (identical in the CPU oracle):
 *   scores  s = sigmoid(logit), evaluated in double and rounded once to fp32;
 *   top-k   descending (s + bias); equal values ordered by lower expert id;
 *   weights s_sel / max(sum_j s_sel, 1e-10) * route_scale, sum over j in order;
 *   sorted order = stable (expert, token); slot id = t*k + j.
 */
#ifndef DSMOE_H
#define DSMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSMOE_OK 0
#define DSMOE_ERR_INVALID (-1)     /* bad argument / shape (Python: ValueError) */
#define DSMOE_ERR_UNSUPPORTED (-2) /* dtype or shape not supported (ValueError) */
#define DSMOE_ERR_WORKSPACE (-3)   /* workspace too small (ValueError)          */
#define DSMOE_ERR_HIP (-4)         /* HIP launch/runtime error (RuntimeError)   */

#define DSMOE_F32 0
#define DSMOE_BF16 1

/* Shape of one DeepSeekMoE layer call.  Mirrors the config keys read by
 * models/moe.py:11-16,56-61 (dim, n_routed_experts, n_activated_experts,
 * moe_inter_dim, n_shared_experts, route_scale) plus T = flattened tokens and
 * I_s = shared expert inter width (extension; equals I in the reference). */
typedef struct dsmoe_dims {
  int32_t T;      /* tokens (x.view(-1, D).size(0))          */
  int32_t D;      /* dim                                     */
  int32_t E;      /* n_routed_experts                        */
  int32_t k;      /* n_activated_experts                     */
  int32_t I;      /* moe_inter_dim                           */
  int32_t S;      /* n_shared_experts                        */
  int32_t I_s;    /* shared expert inter dim                 */
  int32_t dtype;  /* DSMOE_F32 | DSMOE_BF16 (x, y, experts)  */
  float route_scale;
} dsmoe_dims;

const char* dsmoe_last_error(void);
int dsmoe_version(void);

/* ---------------------------------------------------------------------------
 * (a) Gate.  Replaces AuxLossFreeGate.forward, models/moe.py:29-37, with the
 * logits computed in fp32 from x (bf16 upcast exactly) and the fp32 weight.
 *   logits      (T,E) fp32, may be NULL
 *   idx         (T,k) int32 expert ids (descending biased score)
 *   idx64       (T,k) int64 copy for _last_indices, may be NULL
 *   weights     (T,k) fp32 renormalised weights
 *   weights_x   (T,k) weights cast to x dtype (_last_weights), may be NULL
 *   sel_scores  (T,k) fp32 unbiased scores of the selected experts, may be NULL
 *   counts      (E)   int32 per-expert histogram (== bincount(idx)), may be NULL
 */
int dsmoe_gate_fwd(const void* x, const float* gate_w, const float* gate_bias, const dsmoe_dims* dims,
                   float* logits, int32_t* idx, int64_t* idx64, float* weights, void* weights_x,
                   float* sel_scores, int32_t* counts, void* stream);

/* Route from given fp32 logits (T,E): the part of models/moe.py:32-36 after
 * F.linear, plus the bincount of models/moe.py:114.  Same outputs as above. */
int dsmoe_route_from_logits(const float* logits, const float* gate_bias, const dsmoe_dims* dims, int32_t* idx,
                            int64_t* idx64, float* weights, void* weights_x, float* sel_scores, int32_t* counts,
                            void* stream);

/* ---------------------------------------------------------------------------
 * (b) Permute.  Replaces the routing prep of models/moe.py:107-117 (and the
 * row gather flat[sorted_token_ids] of :127 / :150) without a host sync.
 *   idx          (T,k) int32
 *   offsets      (E+1) int32 (the (E+1) form of models/moe_triton.py:33)
 *   sorted_slot  (N) int32   slot id t*k+j at each sorted position
 *   sorted_token (N) int32   token id at each sorted position
 *   slot_pos     (N) int32   sorted position of each slot (inverse)
 *   counts       (E) int32, may be NULL
 *   x, x_sorted  optional row gather x_sorted[p] = x[sorted_token[p]] (both NULL to skip)
 *   sorted_w     optional (N) fp32 gather of weights (T,k) (both NULL to skip)
 *   workspace    dsmoe_permute_workspace_size() bytes
 * Each token's k ids must be distinct and in [0, E), as the gate produces
 * them.  Other input is not detected here (that would need a host sync): its
 * invalid slots are left unplaced, unset sorted positions keep what the
 * buffers held and gather zero rows; no access leaves the buffers.
 */
size_t dsmoe_permute_workspace_size(const dsmoe_dims* dims);
int dsmoe_permute(const int32_t* idx, const dsmoe_dims* dims, int32_t* offsets, int32_t* sorted_slot,
                  int32_t* sorted_token, int32_t* slot_pos, int32_t* counts, const void* x, void* x_sorted,
                  const float* weights, float* sorted_w, void* workspace, size_t workspace_bytes, void* stream);

/* dsmoe_permute without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * scratch is a static device array of DSMOE_PERMUTE_NOALLOC_BYTES that the
 * library holds on each GPU it runs on until the process ends; the call makes
 * no allocation.  A call needing more scratch than that
 * (dsmoe_permute_workspace_size(dims) > DSMOE_PERMUTE_NOALLOC_BYTES; about
 * 400k slots T*k at E = 64) returns DSMOE_ERR_UNSUPPORTED without launching.
 * Every call on one GPU shares the array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller. */
#define DSMOE_PERMUTE_NOALLOC_BYTES (2u << 20)
int dsmoe_permute_noalloc(const int32_t* idx, const dsmoe_dims* dims, int32_t* offsets, int32_t* sorted_slot,
                          int32_t* sorted_token, int32_t* slot_pos, int32_t* counts, const void* x, void* x_sorted,
                          const float* weights, float* sorted_w, void* stream);

/* ---------------------------------------------------------------------------
 * (c) Grouped SwiGLU experts on expert-sorted rows.  Replaces the operator
 * seam triton_grouped_moe_dispatch / _TritonGroupedMoeFunction.forward,
 * models/moe_triton.py:390-436,504-525, with no dimension cap:
 *   y_sorted[r] = (silu(x_sorted[r] W1[e]^T) * (x_sorted[r] W3[e]^T)) W2[e]^T * sorted_w[r]
 * for offsets[e] <= r < offsets[e+1].  sorted_w may be NULL (unweighted, the
 * Function's own output).  offsets (E+1) int64 on device; rows = offsets[E].
 * dims: D, E, I and dtype are used; T is the number of sorted rows.
 */
size_t dsmoe_grouped_swiglu_workspace_size(const dsmoe_dims* dims);
int dsmoe_grouped_swiglu_fwd(const void* x_sorted, const void* const* w1, const void* const* w2,
                             const void* const* w3, const float* sorted_w, const int64_t* offsets,
                             const dsmoe_dims* dims, void* y_sorted, void* workspace, size_t workspace_bytes,
                             void* stream);

/* Backward of the seam (_TritonGroupedMoeFunction.backward,
 * models/moe_triton.py:438-501): given dy_sorted (rows, D) of the UNWEIGHTED
 * output, writes dx_sorted (rows, D) and dW1/dW2/dW3 (per-expert device
 * pointers, weight dtype; fp32 accumulation over each expert's rows in
 * ascending order, one rounding; experts without rows get zeros).  The
 * forward gate/up GEMM is recomputed.  Workspace:
 * dsmoe_grouped_swiglu_bwd_workspace_size(). */
size_t dsmoe_grouped_swiglu_bwd_workspace_size(const dsmoe_dims* dims);
int dsmoe_grouped_swiglu_bwd(const void* x_sorted, const void* const* w1, const void* const* w2,
                             const void* const* w3, const int64_t* offsets, const void* dy_sorted,
                             const dsmoe_dims* dims, void* dx_sorted, void* const* dw1, void* const* dw2,
                             void* const* dw3, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * (d) Combine.  Replaces the weighted out-of-place index_add of
 * models/moe.py:132 and the shared add of :100-102:
 *   y[t] = sum_{j in ascending expert id} weights[t,j] * o_slots[t*k+j] + shared[t]
 * accumulated in fp32, rounded once.  shared may be NULL. */
int dsmoe_combine_fwd(const void* o_slots, const float* weights, const int32_t* idx, const void* shared,
                      const dsmoe_dims* dims, void* y, void* stream);

/* ---------------------------------------------------------------------------
 * Whole layer.  Replaces DeepSeekMoE.forward (models/moe.py:74-103) and its
 * autograd backward.  The forward workspace holds everything the backward
 * needs when training != 0, so the caller keeps it alive until backward.
 *   outputs: y (T,D); idx64/weights_x/counts/logits as in dsmoe_gate_fwd.
 */
size_t dsmoe_moe_fwd_workspace_size(const dsmoe_dims* dims, int training);
int dsmoe_moe_fwd(const void* x, const float* gate_w, const float* gate_bias, const void* const* w1,
                  const void* const* w2, const void* const* w3, const void* const* sw1, const void* const* sw2,
                  const void* const* sw3, const dsmoe_dims* dims, int training, void* y, int64_t* idx64,
                  void* weights_x, int32_t* counts, float* logits, void* workspace, size_t workspace_bytes,
                  void* stream);

/* Backward of dsmoe_moe_fwd (training != 0).  dy (T,D).  Writes dx (T,D),
 * dgate_w (E,D) fp32, and per-expert weight gradients (device pointers, the
 * weight dtype): dw1[e], dw2[e], dw3[e], dsw1[s], dsw2[s], dsw3[s].  Unrouted
 * experts receive zeros.  fwd_workspace is the forward call's workspace.
 * Work ordered on `stream` as for any other call; inside, the routed dW2, the
 * shared experts' gradients and dgate_w run on a second stream of the
 * library's (one per calling thread and device, forked from and joined back
 * into `stream` with events, so graph capture sees a fork and a join), except
 * while stage timing is enabled or when `stream` belongs to a device other
 * than the current one (then everything runs on `stream`). */
size_t dsmoe_moe_bwd_workspace_size(const dsmoe_dims* dims);
int dsmoe_moe_bwd(const void* x, const float* gate_w, const void* const* w1, const void* const* w2,
                  const void* const* w3, const void* const* sw1, const void* const* sw2, const void* const* sw3,
                  const dsmoe_dims* dims, const void* dy, const void* fwd_workspace, void* dx, float* dgate_w,
                  void* const* dw1, void* const* dw2, void* const* dw3, void* const* dsw1, void* const* dsw2,
                  void* const* dsw3, void* workspace, size_t workspace_bytes, void* stream);

/* The same backward with the expert weight gradients dw1..dsw3 written in
 * dw_dtype: the compute dtype (as dsmoe_moe_bwd), or DSMOE_F32 for a bf16
 * computation over fp32 master weights, as under the reference's bf16
 * autocast (training/pretrain.py:212-213, whose fp32 parameters receive the
 * casts' gradients): the fp32 accumulators are stored unrounded, with no
 * separate cast pass. */
int dsmoe_moe_bwd_ex(const void* x, const float* gate_w, const void* const* w1, const void* const* w2,
                     const void* const* w3, const void* const* sw1, const void* const* sw2, const void* const* sw3,
                     const dsmoe_dims* dims, const void* dy, const void* fwd_workspace, void* dx, float* dgate_w,
                     void* const* dw1, void* const* dw2, void* const* dw3, void* const* dsw1, void* const* dsw2,
                     void* const* dsw3, int dw_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* f1: aux-loss-free bias update on device (models/moe.py:21-27,194-201).
 * counts (E) int32 -> bias (E) fp32 updated in place by the +/-speed band rule. */
int dsmoe_update_bias(const int32_t* counts, float* gate_bias, int E, float speed, float upper, float lower,
                      void* stream);

/* The same update from fp32 counts (E), for callers whose counts are not the
 * gate histogram (averaged or accumulated counts may be fractional); the
 * reference casts any counts with counts.float() (models/moe.py:24).  Integer
 * counts give the reference's fp32 mean exactly.  For fractional counts the
 * mean is the fp64 sum divided by E and rounded once; torch's fp32 reduction
 * may differ from it by an ulp, which matters only for a count within an ulp
 * of a band edge. */
int dsmoe_update_bias_f32(const float* counts, float* gate_bias, int E, float speed, float upper, float lower,
                          void* stream);

/* ---------------------------------------------------------------------------
 * Inspection of a forward workspace (no counterpart in the reference, whose
 * intermediates are torch tensors): byte offset inside the dsmoe_moe_fwd
 * workspace of one routing buffer, or (size_t)-1 for bad dims or an unknown
 * id.  The buffers hold, after a forward call (N = T*k):
 *   DSMOE_WS_IDX          (T,k) int32 expert ids
 *   DSMOE_WS_WEIGHTS      (T,k) fp32 renormalised weights
 *   DSMOE_WS_SEL_SCORES   (T,k) fp32 unbiased scores of the selected experts
 *   DSMOE_WS_OFFSETS      (E+1) int32 expert offsets in the sorted order
 *   DSMOE_WS_SORTED_SLOT  (N) int32, DSMOE_WS_SORTED_TOKEN (N) int32,
 *   DSMOE_WS_SLOT_POS     (N) int32 (as dsmoe_permute's outputs) */
#define DSMOE_WS_IDX 0
#define DSMOE_WS_WEIGHTS 1
#define DSMOE_WS_SEL_SCORES 2
#define DSMOE_WS_OFFSETS 3
#define DSMOE_WS_SORTED_SLOT 4
#define DSMOE_WS_SORTED_TOKEN 5
#define DSMOE_WS_SLOT_POS 6
size_t dsmoe_moe_fwd_workspace_offset(const dsmoe_dims* dims, int training, int buffer);

/* ---------------------------------------------------------------------------
 * Stage timing for measurement tools (no counterpart in the reference, which
 * has no timing hooks).  While enabled, dsmoe_moe_fwd / dsmoe_moe_bwd record
 * HIP events on their own stream at every stage boundary;
 * dsmoe_timing_read() waits for the recorded events and returns, per stage,
 * the summed milliseconds over all calls since the last enable.  Stage ids and
 * names: dsmoe_timing_stage_name(i) for i < dsmoe_timing_read's return value. */
int dsmoe_timing_enable(int on);
int dsmoe_timing_read(double* stage_ms, int max_stages, int* n_calls);
const char* dsmoe_timing_stage_name(int stage);

/* ---------------------------------------------------------------------------
 * Multi-head latent attention forward (the fused MLA attention of
 * models/mla_triton.py:73-183, entered through triton_mla_attention,
 * models/mla_triton.py:303-329; dims as its argument shapes read them, :229-234).
 * Tensors are contiguous bf16:
 *   q_nope (B, H, S_q, D_nope)   q_pe (B, H, S_q, D_rope)   RoPE already applied
 *   ctx_kv (B, S_kv, R)          ctx_pe (B, S_kv, D_rope)   latent cache
 *   wkv_b_k (H, D_nope, R)       wkv_b_v (H, D_v, R)        per-head up-projections
 *   out (B, S_q, H, D_v)
 * out = softmax(softmax_scale * [q_nope | q_pe] [ctx_kv wkv_b_k^T | ctx_pe]^T) (ctx_kv wkv_b_v^T)
 * per (batch, head), with the causal mask key <= query + q_start when
 * is_causal (models/mla_triton.py:159-161) and no mask otherwise.  R, D_nope,
 * D_rope, D_v <= 256 as the reference requires (:186-196: DSMOE_ERR_INVALID),
 * and D_nope + D_rope <= 256 (DSMOE_ERR_UNSUPPORTED).  The workspace holds the
 * materialised K and V of every (batch, head): B * H * pad64(S_kv) *
 * (DQKp + DVp) * 2 + 256 bytes, DQKp = 2 D_nope + D_rope (D_nope + D_rope when
 * that exceeds 256) and DVp = D_v, each rounded up to a multiple of 16 and 32
 * (dsmoe_mla_attn_workspace_size gives the figure; about 2.7 GB at B 1,
 * H 128, S_kv 32768, D_nope 128, D_rope 64, D_v 128).  Row indices are 32-bit:
 * a call needs B * H * pad64(S_kv) and B * H * S_q below 2^22
 * (DSMOE_ERR_UNSUPPORTED otherwise); dsmoe.mla splits larger calls by batch,
 * so one batch's H * S_kv and H * S_q must stay below 2^22. */
typedef struct dsmoe_mla_dims {
  int32_t B, H, S_q, S_kv;
  int32_t R;          /* kv_lora_rank        */
  int32_t D_nope;     /* qk_nope_head_dim    */
  int32_t D_rope;     /* qk_rope_head_dim    */
  int32_t D_v;        /* v_head_dim          */
  int32_t dtype;      /* DSMOE_BF16          */
  int32_t is_causal;
  int32_t q_start;
  float softmax_scale;
} dsmoe_mla_dims;
size_t dsmoe_mla_attn_workspace_size(const dsmoe_mla_dims* dims);
int dsmoe_mla_attn_fwd(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                       const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out,
                       void* workspace, size_t workspace_bytes, void* stream);
/* dsmoe_mla_attn_fwd that also writes lse (B, H, S_q) fp32, each query's
 * base-2 log-sum-exp of its scaled scores: log2(sum over visible keys of
 * exp(softmax_scale q.k)), +inf for a query without a visible key.  The
 * training forward of models/mla_triton.py:200-267 (_TritonMlaAttentionFunction.forward),
 * whose backward needs the probabilities again. */
int dsmoe_mla_attn_fwd_lse(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                           const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out,
                           float* lse, void* workspace, size_t workspace_bytes, void* stream);
/* K and V of every (batch, head) into kv_ws (dsmoe_mla_attn_workspace_size
 * bytes), the first launch of dsmoe_mla_attn_fwd on its own: for a backward
 * whose caller did not keep the forward's workspace.  No counterpart in the
 * reference (its backward recomputes everything, models/mla_triton.py:269-296). */
int dsmoe_mla_attn_kv(const void* ctx_kv, const void* ctx_pe, const void* wkv_b_k, const void* wkv_b_v,
                      const dsmoe_mla_dims* dims, void* kv_ws, size_t kv_bytes, void* stream);
/* Backward of the attention (models/mla_triton.py:269-296,
 * _TritonMlaAttentionFunction.backward, which differentiates a torch recompute of
 * the same function), for the per-head operands.  Given the forward's queries,
 * kv_ws as dsmoe_mla_attn_fwd(_lse) left it for the same inputs and dims
 * (or as dsmoe_mla_attn_kv fills it), the forward's out and lse, and dout
 * (B, S_q, H, D_v) bf16, writes
 *   dq_nope (B, H, S_q, D_nope) fp32   dq_pe (B, H, S_q, D_rope) fp32
 *   dkv (B, S_kv, H, D_nope + D_v) bf16: rows [dk_nope | dv]
 *   dk_pe (B, S_kv, H, D_rope) fp32
 * the gradients of q, of k_nope = ctx_kv wkv_b_k^T, v = ctx_kv wkv_b_v^T and
 * k_pe = ctx_pe (per head).  A (B S_kv, H (D_nope + D_v)) view of dkv pairs
 * with the weight in the wkv_b layout (per head the D_nope k rows, then the
 * D_v v rows: an (H (D_nope + D_v), R) matrix W), so the caller finishes with
 * two GEMMs: d ctx_kv = dkv W and [dW_k | dW_v] = dkv^T ctx_kv; ctx_pe's
 * gradient is dk_pe summed over heads.  The gradient is that of the function
 * the forward computes (for is_causal = 0 no mask, square or not).  Every
 * element of the four outputs is written (zeros where no probability reaches
 * it).  The probabilities and dZ enter their MFMAs in bf16 with fp32
 * accumulation; dkv is rounded to bf16 once (the operand of those GEMMs).
 * Workspace: dsmoe_mla_attn_bwd_workspace_size bytes (packed query and dO
 * rows, lse and rowsum(dout * out) for S_q rounded up to 64 rows); dims and
 * limits as dsmoe_mla_attn_fwd. */
size_t dsmoe_mla_attn_bwd_workspace_size(const dsmoe_mla_dims* dims);
int dsmoe_mla_attn_bwd(const void* q_nope, const void* q_pe, const dsmoe_mla_dims* dims, const void* kv_ws,
                       size_t kv_bytes, const void* out, const void* dout, const float* lse, float* dq_nope,
                       float* dq_pe, void* dkv, float* dk_pe, void* workspace, size_t workspace_bytes,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSMOE_H */
