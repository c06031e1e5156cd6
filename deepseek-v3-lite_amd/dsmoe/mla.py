"""Fused MLA attention over the dsmoe C ABI (device tensors only).

``mla_attention`` mirrors ``triton_mla_attention`` of models/mla_triton.py:303-329
(same arguments, output (B, S_q, H, D_v), the same ValueError for a dimension
above 256, models/mla_triton.py:186-196); ``triton_mla_attention`` is the same
function under the reference's name, so a caller can swap the import.  Both
directions run the HIP kernels of csrc/mla.hip (bf16 operands, fp32
accumulation).  The reference's backward (models/mla_triton.py:269-296)
differentiates a torch recompute of the attention; here the training forward
also keeps each query's log-sum-exp, and the backward rebuilds the
probabilities from it in two flash-attention kernels (dsmoe_mla_attn_bwd:
dq per query block, dk and dv per key block) and maps the per-head key
gradients onto ctx_kv, wkv_b_k and wkv_b_v with two GEMMs (bf16 operands,
fp32 accumulation and results, as autocast computes weight gradients).  The gradient is
that of the function the forward computes: its masking (causal only when
``is_causal``; the reference's recompute, mla_attention_reference, also masks
a square non-causal call, models/mla_triton.py:52-57, which its forward
kernel does not).

Dtypes: the kernels compute in bf16.  Under bf16 autocast the reference's
layer hands the operator a mix (models/mla.py:127-129,209-220 with
training/pretrain.py:154,212-213): bf16 queries, fp32 views of the fp32
``wkv_b.weight``, and fp32 or bf16 latent rows depending on the KV cache's
dtype.  Each tensor is rounded to bf16 once per call (the weight views are
H (D_nope + D_v) R elements, a few MB) and the output takes ``q_nope``'s dtype,
as the reference's ``out`` does (models/mla_triton.py:218).  The backward
returns each input's gradient in that input's dtype.  fp32 queries outside a
bf16 autocast region raise ``ValueError`` (the reference layer then uses its
SDPA path), since rounding them to bf16 would be a precision loss the caller
did not ask for.
"""
from __future__ import annotations

import torch

from . import _lib as L


def _check_mla_dim_limits(R: int, D_nope: int, D_rope: int, D_v: int) -> None:
    for name, val in (("R", R), ("D_nope", D_nope), ("D_rope", D_rope), ("D_v", D_v)):
        if val > 256:
            raise ValueError(f"mla_attention: {name}={val} exceeds the 256 cap. "
                             "Reduce or tile manually before launching the kernel.")


def _dims(q_nope, q_pe, ctx_kv, wkv_b_v, softmax_scale, is_causal, q_start) -> "L.MlaDims":
    B, H, S_q, D_nope = q_nope.shape
    d = L.MlaDims()
    d.B, d.H, d.S_q, d.S_kv = B, H, S_q, ctx_kv.size(1)
    d.R, d.D_nope, d.D_rope, d.D_v = ctx_kv.size(-1), D_nope, q_pe.shape[-1], wkv_b_v.size(1)
    d.dtype = 1
    d.is_causal = 1 if is_causal else 0
    d.q_start = int(q_start)
    d.softmax_scale = float(softmax_scale)
    return d


_ROWS_PER_CALL = 1 << 22

# Successful launches of the HIP kernels (a caller can check that the fused
# path ran rather than a fallback of its own).
hip_calls = 0


def _bf16_inputs(ts):
    """The six inputs in bf16 for the kernels, or ValueError when the call is
    not a bf16 one: q_nope in bf16, or a bf16 autocast region on its device."""
    q = ts[0]
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("mla_attention: tensors must be on a ROCm GPU (no CPU implementation)")
        if t.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"mla_attention: bf16 or fp32 tensors only (got {t.dtype})")
    dt = q.device.type
    bf16_call = q.dtype == torch.bfloat16 or (torch.is_autocast_enabled(dt)
                                               and torch.get_autocast_dtype(dt) == torch.bfloat16)
    if not bf16_call:
        raise ValueError("mla_attention: the kernels compute in bf16; fp32 queries need a bf16 autocast region")
    return tuple(t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16) for t in ts)


def _prepare(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v):
    """The six inputs as contiguous bf16 tensors (shapes checked) and the
    batch chunk of one launch."""
    ts = _bf16_inputs((q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
    q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v = ts
    B, H, S_q, D_nope = q_nope.shape
    R, D_rope, D_v = ctx_kv.size(-1), q_pe.shape[-1], wkv_b_v.size(1)
    _check_mla_dim_limits(R, D_nope, D_rope, D_v)
    if (q_pe.shape[:3] != (B, H, S_q) or ctx_kv.dim() != 3 or ctx_kv.size(0) != B
            or tuple(ctx_pe.shape) != (B, ctx_kv.size(1), D_rope) or tuple(wkv_b_k.shape) != (H, D_nope, R)
            or wkv_b_v.dim() != 3 or wkv_b_v.size(0) != H or wkv_b_v.size(2) != R):
        raise ValueError("mla_attention: inconsistent shapes")
    # the kernels index rows with 32-bit offsets: B H pad64(S_kv) and B H S_q
    # below 2^22 per call, so larger calls run in batch chunks
    S_kv = ctx_kv.size(1)
    per_batch = H * max(-(-S_kv // 64) * 64, S_q)
    if per_batch >= _ROWS_PER_CALL:
        raise ValueError(f"mla_attention: H * S_kv = {H * S_kv} (H * S_q = {H * S_q}) reaches 2^22, the limit of "
                         "one batch row of the kernels' 32-bit row offsets")
    bc = min(B, (_ROWS_PER_CALL - 1) // per_batch)
    return tuple(t.contiguous() for t in ts), bc


def _forward(ts, bc: int, softmax_scale: float, is_causal: bool, q_start: int, want_lse: bool):
    """dsmoe_mla_attn_fwd (or _fwd_lse) over the batch chunks: bf16 out, the
    fp32 lse (None unless asked for) and the workspace, which holds the last
    chunk's K and V."""
    q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v = ts
    B, H, S_q, _ = q_nope.shape
    D_v = wkv_b_v.size(1)
    dev = q_nope.device
    lib = L.load()
    d = _dims(q_nope[:bc], q_pe[:bc], ctx_kv[:bc], wkv_b_v, softmax_scale, is_causal, q_start)
    nbytes = int(lib.dsmoe_mla_attn_workspace_size(d))
    if nbytes == 0:
        L.check(lib.dsmoe_mla_attn_fwd(None, None, None, None, None, None, d, None, None, 0, None),
                "dsmoe_mla_attn_fwd")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(B, S_q, H, D_v, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, S_q, dtype=torch.float32, device=dev) if want_lse else None
    for b0 in range(0, B, bc):
        b1 = min(B, b0 + bc)
        d = _dims(q_nope[b0:b1], q_pe[b0:b1], ctx_kv[b0:b1], wkv_b_v, softmax_scale, is_causal, q_start)
        ins = (L.ptr(q_nope[b0:b1]), L.ptr(q_pe[b0:b1]), L.ptr(ctx_kv[b0:b1]), L.ptr(ctx_pe[b0:b1]),
               L.ptr(wkv_b_k), L.ptr(wkv_b_v), d, L.ptr(out[b0:b1]))
        if want_lse:
            L.check(lib.dsmoe_mla_attn_fwd_lse(*ins, L.ptr(lse[b0:b1]), L.ptr(ws), nbytes, L.stream_ptr(dev)),
                    "dsmoe_mla_attn_fwd_lse")
        else:
            L.check(lib.dsmoe_mla_attn_fwd(*ins, L.ptr(ws), nbytes, L.stream_ptr(dev)), "dsmoe_mla_attn_fwd")
    return out, lse, ws


def mla_attention_fwd(q_nope: torch.Tensor, q_pe: torch.Tensor, ctx_kv: torch.Tensor, ctx_pe: torch.Tensor,
                      wkv_b_k: torch.Tensor, wkv_b_v: torch.Tensor, softmax_scale: float, is_causal: bool = False,
                      q_start: int = 0) -> torch.Tensor:
    """dsmoe_mla_attn_fwd: (B, S_q, H, D_v) in q_nope's dtype, no autograd."""
    global hip_calls
    out_dtype = q_nope.dtype
    ts, bc = _prepare(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v)
    out, _, _ = _forward(ts, bc, softmax_scale, is_causal, q_start, want_lse=False)
    hip_calls += 1
    return out if out_dtype == torch.bfloat16 else out.to(out_dtype)


def mla_attention_bwd_heads(ts, bc: int, out: torch.Tensor, lse: torch.Tensor, dout: torch.Tensor,
                            softmax_scale: float, is_causal: bool, q_start: int, kv_ws=None):
    """dsmoe_mla_attn_bwd over the batch chunks: fp32 dq_nope (B, H, S_q, Dn)
    and dq_pe (B, H, S_q, Dr), the bf16 key-side rows dkv (B, S_kv, H, Dn + Dv)
    = [dk_nope | dv] and fp32 dk_pe (B, S_kv, H, Dr).  ``ts`` and ``bc`` as
    ``_prepare`` returns them; out, lse from the training forward; kv_ws the
    forward's workspace when it ran in one chunk (its K and V are reused),
    else None (K and V are rebuilt per chunk by dsmoe_mla_attn_kv)."""
    q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v = ts
    B, H, S_q, Dn = q_nope.shape
    S_kv, Dr, Dv = ctx_kv.size(1), q_pe.size(-1), wkv_b_v.size(1)
    dev = q_nope.device
    dout = dout.to(torch.bfloat16).contiguous()
    lib = L.load()
    d = _dims(q_nope[:bc], q_pe[:bc], ctx_kv[:bc], wkv_b_v, softmax_scale, is_causal, q_start)
    nbytes = int(lib.dsmoe_mla_attn_bwd_workspace_size(d))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if kv_ws is not None and bc < B:
        raise ValueError("mla_attention_bwd_heads: a forward workspace holds one chunk's K and V")
    if kv_ws is None:
        kv_ws = torch.empty(int(lib.dsmoe_mla_attn_workspace_size(d)), dtype=torch.uint8, device=dev)
        rebuild = True
    else:
        rebuild = False
    f32 = dict(dtype=torch.float32, device=dev)
    dq_nope, dq_pe = torch.empty(B, H, S_q, Dn, **f32), torch.empty(B, H, S_q, Dr, **f32)
    dkv = torch.empty(B, S_kv, H, Dn + Dv, dtype=torch.bfloat16, device=dev)
    dk_pe = torch.empty(B, S_kv, H, Dr, **f32)
    st = L.stream_ptr(dev)
    for b0 in range(0, B, bc):
        b1 = min(B, b0 + bc)
        d = _dims(q_nope[b0:b1], q_pe[b0:b1], ctx_kv[b0:b1], wkv_b_v, softmax_scale, is_causal, q_start)
        if rebuild:
            L.check(lib.dsmoe_mla_attn_kv(L.ptr(ctx_kv[b0:b1]), L.ptr(ctx_pe[b0:b1]), L.ptr(wkv_b_k), L.ptr(wkv_b_v),
                                          d, L.ptr(kv_ws), kv_ws.numel(), st), "dsmoe_mla_attn_kv")
        rc = lib.dsmoe_mla_attn_bwd(
            L.ptr(q_nope[b0:b1]), L.ptr(q_pe[b0:b1]), d, L.ptr(kv_ws), kv_ws.numel(), L.ptr(out[b0:b1]),
            L.ptr(dout[b0:b1]), L.ptr(lse[b0:b1]), L.ptr(dq_nope[b0:b1]), L.ptr(dq_pe[b0:b1]), L.ptr(dkv[b0:b1]),
            L.ptr(dk_pe[b0:b1]), L.ptr(ws), nbytes, st)
        L.check(rc, "dsmoe_mla_attn_bwd")
    return dq_nope, dq_pe, dkv, dk_pe


def _project_kv_grads(ctx_kv, wkv_b_k, wkv_b_v, dkv, dk_pe):
    """Key-side gradients onto the latent rows and the up-projections: with
    W = [W_k; W_v] per head (wkv_b's layout, (H (Dn + Dv), R)), k_nope and v
    are ctx_kv W^T split per head, so d ctx_kv = dkv W and [dW_k | dW_v] =
    dkv^T ctx_kv (bf16 operands, fp32 accumulation and results; the second
    product split over row slices whose fp32 partials are summed), and
    d ctx_pe = dk_pe summed over heads."""
    B, S_kv, H, Dkv = dkv.shape
    Dn, R = wkv_b_k.size(1), ctx_kv.size(-1)
    rows = B * S_kv
    d2 = dkv.view(rows, H * Dkv)
    w = torch.cat([wkv_b_k, wkv_b_v], dim=1).reshape(H * Dkv, R)
    dctx_kv = torch.mm(d2, w, out_dtype=torch.float32)
    n = next(k for k in (8, 4, 2, 1) if rows % k == 0 and rows // k >= 256 or k == 1)
    dw = torch.bmm(d2.view(n, rows // n, H * Dkv).transpose(1, 2), ctx_kv.reshape(n, rows // n, R),
                   out_dtype=torch.float32).sum(0).view(H, Dkv, R)
    return dctx_kv.view(B, S_kv, R), dk_pe.sum(2), dw[:, :Dn], dw[:, Dn:]


class _MlaAttentionFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal, q_start):
        global hip_calls
        out_dtype = q_nope.dtype
        ctx.dtypes = tuple(t.dtype for t in (q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
        ts, bc = _prepare(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v)
        out, lse, kv_ws = _forward(ts, bc, softmax_scale, is_causal, q_start, want_lse=True)
        hip_calls += 1
        # the backward runs on the bf16 operands the kernels saw, and on the
        # forward's K and V when one launch covered the batch (B H pad64(S_kv)
        # (DQKp + DVp) bf16, held until the backward); otherwise it rebuilds them
        ctx.save_for_backward(*ts, out, lse)
        ctx.kv_ws = kv_ws if bc >= ts[0].size(0) else None
        ctx.args = (bc, softmax_scale, is_causal, q_start)
        return out if out_dtype == torch.bfloat16 else out.to(out_dtype)

    @staticmethod
    def backward(ctx, dout):
        *ts, out, lse = ctx.saved_tensors
        bc, softmax_scale, is_causal, q_start = ctx.args
        with torch.autocast(dout.device.type, enabled=False):
            dq_nope, dq_pe, dkv, dk_pe = mla_attention_bwd_heads(ts, bc, out, lse, dout, softmax_scale, is_causal,
                                                                 q_start, ctx.kv_ws)
            ctx.kv_ws = None
            dctx_kv, dctx_pe, dwk, dwv = _project_kv_grads(ts[2], ts[4], ts[5], dkv, dk_pe)
        grads = (dq_nope, dq_pe, dctx_kv, dctx_pe, dwk, dwv)
        return tuple(g.to(dt) for g, dt in zip(grads, ctx.dtypes)) + (None, None, None)


def mla_attention(q_nope: torch.Tensor, q_pe: torch.Tensor, ctx_kv: torch.Tensor, ctx_pe: torch.Tensor,
                  wkv_b_k: torch.Tensor, wkv_b_v: torch.Tensor, softmax_scale: float, is_causal: bool = False,
                  q_start: int = 0) -> torch.Tensor:
    """Fused MLA attention (models/mla_triton.py:303-329).  Returns (B, S_q, H, D_v).

    ``q_start`` offsets the query positions in the KV context so a cached
    mid-sequence prefill stays causal."""
    return _MlaAttentionFunction.apply(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal,
                                       q_start)


triton_mla_attention = mla_attention
