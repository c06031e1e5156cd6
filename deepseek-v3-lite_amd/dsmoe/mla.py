"""Fused MLA attention over the dsmoe C ABI (device tensors only).

``mla_attention`` mirrors ``triton_mla_attention`` of models/mla_triton.py:303-329
(same arguments, output (B, S_q, H, D_v), the same ValueError for a dimension
above 256, models/mla_triton.py:186-196); ``triton_mla_attention`` is the same
function under the reference's name, so a caller can swap the import.  The
forward runs the HIP kernels of csrc/mla.hip (bf16).  The backward, as in the
reference (models/mla_triton.py:257-296), recomputes the attention with torch
ops and differentiates that; it follows the forward's masking (causal only when
``is_causal``).

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


def mla_attention_fwd(q_nope: torch.Tensor, q_pe: torch.Tensor, ctx_kv: torch.Tensor, ctx_pe: torch.Tensor,
                      wkv_b_k: torch.Tensor, wkv_b_v: torch.Tensor, softmax_scale: float, is_causal: bool = False,
                      q_start: int = 0) -> torch.Tensor:
    """dsmoe_mla_attn_fwd: (B, S_q, H, D_v) in q_nope's dtype, no autograd."""
    global hip_calls
    out_dtype = q_nope.dtype
    ts = _bf16_inputs((q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
    q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v = ts
    B, H, S_q, D_nope = q_nope.shape
    R, D_rope, D_v = ctx_kv.size(-1), q_pe.shape[-1], wkv_b_v.size(1)
    _check_mla_dim_limits(R, D_nope, D_rope, D_v)
    if (q_pe.shape[:3] != (B, H, S_q) or ctx_kv.dim() != 3 or ctx_kv.size(0) != B
            or tuple(ctx_pe.shape) != (B, ctx_kv.size(1), D_rope) or tuple(wkv_b_k.shape) != (H, D_nope, R)
            or wkv_b_v.dim() != 3 or wkv_b_v.size(0) != H or wkv_b_v.size(2) != R):
        raise ValueError("mla_attention: inconsistent shapes")
    dev = q_nope.device
    q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v = (t.contiguous() for t in ts)
    # the kernels index rows with 32-bit offsets: B H pad64(S_kv) and B H S_q
    # below 2^22 per call, so larger calls run in batch chunks
    S_kv = ctx_kv.size(1)
    per_batch = H * max(-(-S_kv // 64) * 64, S_q)
    if per_batch >= _ROWS_PER_CALL:
        raise ValueError(f"mla_attention: H * S_kv = {H * S_kv} (H * S_q = {H * S_q}) reaches 2^22, the limit of "
                         "one batch row of the kernels' 32-bit row offsets")
    bc = min(B, (_ROWS_PER_CALL - 1) // per_batch)
    lib = L.load()
    d = _dims(q_nope[:bc], q_pe[:bc], ctx_kv[:bc], wkv_b_v, softmax_scale, is_causal, q_start)
    nbytes = int(lib.dsmoe_mla_attn_workspace_size(d))
    if nbytes == 0:
        L.check(lib.dsmoe_mla_attn_fwd(None, None, None, None, None, None, d, None, None, 0, None),
                "dsmoe_mla_attn_fwd")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(B, S_q, H, D_v, dtype=torch.bfloat16, device=dev)
    for b0 in range(0, B, bc):
        b1 = min(B, b0 + bc)
        d = _dims(q_nope[b0:b1], q_pe[b0:b1], ctx_kv[b0:b1], wkv_b_v, softmax_scale, is_causal, q_start)
        rc = lib.dsmoe_mla_attn_fwd(L.ptr(q_nope[b0:b1]), L.ptr(q_pe[b0:b1]), L.ptr(ctx_kv[b0:b1]),
                                    L.ptr(ctx_pe[b0:b1]), L.ptr(wkv_b_k), L.ptr(wkv_b_v), d, L.ptr(out[b0:b1]),
                                    L.ptr(ws), nbytes, L.stream_ptr(dev))
        L.check(rc, "dsmoe_mla_attn_fwd")
    hip_calls += 1
    return out if out_dtype == torch.bfloat16 else out.to(out_dtype)


def _attention_torch(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal, q_start):
    """The forward's math in float32 torch ops, for the recompute backward."""
    k_nope = torch.einsum("bsr,hdr->bhsd", ctx_kv, wkv_b_k)
    v = torch.einsum("bsr,hdr->bhsd", ctx_kv, wkv_b_v)
    B, H, S_kv, _ = k_nope.shape
    k = torch.cat([k_nope, ctx_pe.unsqueeze(1).expand(B, H, S_kv, ctx_pe.size(-1))], dim=-1)
    q = torch.cat([q_nope, q_pe], dim=-1)
    s = torch.einsum("bhqd,bhkd->bhqk", q, k) * softmax_scale
    if is_causal:
        qi = torch.arange(q.size(2), device=s.device)[:, None] + q_start
        ki = torch.arange(S_kv, device=s.device)[None, :]
        s = s.masked_fill(qi < ki, float("-inf"))
    o = torch.einsum("bhqk,bhkd->bhqd", s.softmax(dim=-1), v)
    return o.permute(0, 2, 1, 3).contiguous()


class _MlaAttentionFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal, q_start):
        out = mla_attention_fwd(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal, q_start)
        ctx.save_for_backward(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v)
        ctx.args = (softmax_scale, is_causal, q_start)
        return out

    @staticmethod
    def backward(ctx, dout):
        saved = ctx.saved_tensors
        # fp32 recompute whatever autocast state the backward runs under
        with torch.enable_grad(), torch.autocast(saved[0].device.type, enabled=False):
            ins = [t.detach().float().requires_grad_() for t in saved]
            ref = _attention_torch(*ins, *ctx.args)
            grads = torch.autograd.grad(ref, ins, grad_outputs=dout.float(), allow_unused=True)
        return tuple(g.to(t.dtype) if g is not None else torch.zeros_like(t) for g, t in zip(grads, saved)) + (
            None, None, None)


def mla_attention(q_nope: torch.Tensor, q_pe: torch.Tensor, ctx_kv: torch.Tensor, ctx_pe: torch.Tensor,
                  wkv_b_k: torch.Tensor, wkv_b_v: torch.Tensor, softmax_scale: float, is_causal: bool = False,
                  q_start: int = 0) -> torch.Tensor:
    """Fused MLA attention (models/mla_triton.py:303-329).  Returns (B, S_q, H, D_v).

    ``q_start`` offsets the query positions in the KV context so a cached
    mid-sequence prefill stays causal."""
    return _MlaAttentionFunction.apply(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale, is_causal,
                                       q_start)


triton_mla_attention = mla_attention
