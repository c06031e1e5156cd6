"""CPU restatement of the reference MLA attention — TEST INFRASTRUCTURE ONLY.

Parity oracle for ``dsmoe.mla`` (the HIP kernels in ``csrc/mla.hip``).  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it, and only as the checker / the timed CPU baseline.

* ``mla_attention_oracle`` <- ``models/mla_triton.py:73-183`` (the fused
  kernel ``_mla_flash_fwd_kernel`` as launched by ``triton_mla_attention``,
  ``:303-329``): per (batch, head) K_nope = ctx_kv W_k^T, V = ctx_kv W_v^T
  (``:146-147``), scores = scale ([q_nope | q_pe] . [K_nope | ctx_pe])
  (``:154-155``), causal mask key <= query + q_start only when ``is_causal``
  (``:157-160``), softmax over keys, output (B, S_q, H, D_v) (``:178-183``).
  Evaluated in float64 from the given (bf16-representable) inputs.
* ``mla_attention_bwd_oracle`` <- ``models/mla_triton.py:269-296`` (the
  backward: autograd of a recompute of the same function): the gradients of
  ``mla_attention_oracle`` in closed form, float64.
* ``mla_attention_sdpa_torch`` restates the reference layer's default SDPA
  path (``models/mla.py:155-172``) with torch ops: the attention's CPU
  baseline in bench.py (pinned against ``mla_attention_oracle``).
* ``square_mask=True`` adds what ``mla_attention_reference``
  (``models/mla_triton.py:28-68``) also does: for ``is_causal=False`` with
  ``S_q == S_kv`` it applies a triu(-inf) mask anyway (``:52-57``), which the
  fused kernel it documents does not.  The HIP path follows the kernel; the
  flag exists so the tests can state the difference.

Pinned by (``tests/test_mla_oracle.py``): torch's
``scaled_dot_product_attention`` in float64 on separately materialised K and
V; the absorbed formulation (scores through q_nope W_k and the latent cache,
output through the latent then W_v^T), which associates every product
differently; closed forms (one key gives its V row, equal scores give the mean
of the visible V rows); and the reference's own CPU test cases
(``tests/test_mla_triton.py:68-110``: a last-position query attends every key,
q_start offsets block future keys).  The backward is pinned against torch
float64 autograd of scaled_dot_product_attention on the materialised K and V
(a different evaluation of the chain rule), against central finite
differences of ``mla_attention_oracle``, and by the invariants that the
probabilities' gradient rows sum to zero (so the logits' gradient does too)
and that dV sums, over keys, to dO summed over queries.
"""
from __future__ import annotations

import numpy as np


def _f64(t) -> np.ndarray:
    if hasattr(t, "detach"):
        import torch
        t = t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64)


def mla_kv_oracle(ctx_kv, ctx_pe, wkv_b_k, wkv_b_v):
    """Materialised K = [ctx_kv W_k^T | ctx_pe] (B, H, S_kv, Dn + Dr) and
    V = ctx_kv W_v^T (B, H, S_kv, Dv) (models/mla_triton.py:146-152)."""
    kv, pe, wk, wv = map(_f64, (ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
    k_nope = np.einsum("bsr,hdr->bhsd", kv, wk)
    v = np.einsum("bsr,hdr->bhsd", kv, wv)
    B, H, S, _ = k_nope.shape
    k = np.concatenate([k_nope, np.broadcast_to(pe[:, None], (B, H, S, pe.shape[-1]))], axis=-1)
    return k, v


def mla_mask_oracle(S_q: int, S_kv: int, is_causal: bool, q_start: int, square_mask: bool = False) -> np.ndarray:
    """Boolean (S_q, S_kv): True where query i may attend key j."""
    allow = np.ones((S_q, S_kv), dtype=bool)
    if is_causal:
        allow = (np.arange(S_q)[:, None] + q_start) >= np.arange(S_kv)[None, :]
    elif square_mask and S_q == S_kv:
        allow = np.arange(S_q)[:, None] >= np.arange(S_kv)[None, :]
    return allow


def mla_attention_oracle(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale: float,
                         is_causal: bool = False, q_start: int = 0, square_mask: bool = False) -> np.ndarray:
    """(B, S_q, H, D_v) float64 attention output (models/mla_triton.py:73-183)."""
    qn, qp = _f64(q_nope), _f64(q_pe)
    k, v = mla_kv_oracle(ctx_kv, ctx_pe, wkv_b_k, wkv_b_v)
    q = np.concatenate([qn, qp], axis=-1)                      # (B, H, S_q, Dn + Dr)
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * float(softmax_scale)
    allow = mla_mask_oracle(q.shape[2], k.shape[2], is_causal, q_start, square_mask)
    s = np.where(allow[None, None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqk,bhkd->bhqd", p, v)
    return np.ascontiguousarray(o.transpose(0, 2, 1, 3))


def mla_attention_bwd_oracle(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, dout, softmax_scale: float,
                             is_causal: bool = False, q_start: int = 0) -> dict:
    """float64 gradients of ``mla_attention_oracle`` for dout (B, S_q, H, D_v).

    The reference's backward (models/mla_triton.py:269-296) is torch autograd
    of a recompute of the same function; this states the chain rule in
    closed form: with P the probabilities, z = scale q.k the logits and
    O = P V, per (batch, head)
      dV = P^T dO,  dP = dO V^T,  dz = P (dP - rowsum(dO O)),
      dq = scale dz K,  dK = scale dz^T q,
    then through K_nope = ctx_kv W_k^T, V = ctx_kv W_v^T, K_pe = ctx_pe:
      d ctx_kv = sum_h (dK_nope W_k + dV W_v),  dW_k = sum_{b,s} dK_nope^T ctx_kv,
      dW_v likewise,  d ctx_pe = sum_h dK_pe.
    Returns the six input gradients (keys q_nope .. wkv_b_v) and the per-head
    ones (dk_nope, dk_pe, dv in (B, H, S_kv, D) order)."""
    qn, qp = _f64(q_nope), _f64(q_pe)
    kv, pe, wk, wv = map(_f64, (ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
    do = _f64(dout).transpose(0, 2, 1, 3)                     # (B, H, S_q, Dv)
    Dn = qn.shape[-1]
    k, v = mla_kv_oracle(kv, pe, wk, wv)
    q = np.concatenate([qn, qp], axis=-1)
    sc = float(softmax_scale)
    z = np.einsum("bhqd,bhkd->bhqk", q, k) * sc
    allow = mla_mask_oracle(q.shape[2], k.shape[2], is_causal, q_start)
    z = np.where(allow[None, None], z, -np.inf)
    zmax = z.max(axis=-1, keepdims=True)
    p = np.exp(z - np.where(np.isfinite(zmax), zmax, 0.0))
    tot = p.sum(axis=-1, keepdims=True)
    p = np.divide(p, tot, out=np.zeros_like(p), where=tot > 0)
    o = np.einsum("bhqk,bhkd->bhqd", p, v)
    dv = np.einsum("bhqk,bhqd->bhkd", p, do)
    dp = np.einsum("bhqd,bhkd->bhqk", do, v)
    dz = p * (dp - (do * o).sum(axis=-1, keepdims=True))
    dq = np.einsum("bhqk,bhkd->bhqd", dz, k) * sc
    dk = np.einsum("bhqk,bhqd->bhkd", dz, q) * sc
    dk_nope, dk_pe = dk[..., :Dn], dk[..., Dn:]
    return {
        "q_nope": dq[..., :Dn], "q_pe": dq[..., Dn:],
        "ctx_kv": np.einsum("bhsd,hdr->bsr", dk_nope, wk) + np.einsum("bhsd,hdr->bsr", dv, wv),
        "ctx_pe": dk_pe.sum(axis=1),
        "wkv_b_k": np.einsum("bhsd,bsr->hdr", dk_nope, kv), "wkv_b_v": np.einsum("bhsd,bsr->hdr", dv, kv),
        "dk_nope": dk_nope, "dk_pe": dk_pe, "dv": dv,
    }


def mla_attention_absorbed(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale: float,
                           is_causal: bool = False, q_start: int = 0) -> np.ndarray:
    """The same attention through the latent space (models/mla.py:149-152,
    192-202 associate it this way): scores = (q_nope W_k) ctx_kv^T +
    q_pe ctx_pe^T, output = (P ctx_kv) W_v^T.  A check of the oracle, not a
    second oracle."""
    qn, qp, kv, pe, wk, wv = map(_f64, (q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v))
    q_abs = np.einsum("bhqd,hdr->bhqr", qn, wk)
    s = (np.einsum("bhqr,bkr->bhqk", q_abs, kv) + np.einsum("bhqd,bkd->bhqk", qp, pe)) * float(softmax_scale)
    allow = mla_mask_oracle(qn.shape[2], kv.shape[1], is_causal, q_start)
    s = np.where(allow[None, None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    lat = np.einsum("bhqk,bkr->bhqr", p, kv)
    o = np.einsum("bhqr,hdr->bhqd", lat, wv)
    return np.ascontiguousarray(o.transpose(0, 2, 1, 3))


def mla_attention_sdpa_torch(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, softmax_scale: float,
                             is_causal: bool = False):
    """The reference layer's default attention path, restated with the same
    torch ops (models/mla.py:155-172): K_nope and V of every head in one bmm
    of the latent rows with [W_k; W_v], then scaled_dot_product_attention over
    [q_nope | q_pe] and [K_nope | ctx_pe] (the layer's causal mask as
    ``is_causal``).  Runs on the tensors' device in their dtype; bench.py times
    it on the host cores as the attention's CPU baseline.  Returns
    (B, S_q, H, D_v)."""
    import torch
    B, H, S_q, Dn = q_nope.shape
    S_kv, R = ctx_kv.shape[1], ctx_kv.shape[2]
    Dv = wkv_b_v.shape[1]
    kv_rows = ctx_kv.reshape(B * S_kv, R).unsqueeze(0).expand(H, -1, -1)
    w_kv = torch.cat([wkv_b_k, wkv_b_v], dim=1)
    kv = torch.bmm(kv_rows, w_kv.transpose(-1, -2))
    k_nope, v = kv.split([Dn, Dv], dim=-1)
    k_nope = k_nope.reshape(H, B, S_kv, Dn).permute(1, 0, 2, 3)
    v = v.reshape(H, B, S_kv, Dv).permute(1, 0, 2, 3).contiguous()
    k = torch.cat([k_nope, ctx_pe.unsqueeze(1).expand(-1, H, -1, -1)], dim=-1)
    q = torch.cat([q_nope, q_pe], dim=-1)
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=is_causal, scale=softmax_scale)
    return o.transpose(1, 2)


def mla_flops(B: int, H: int, S_q: int, S_kv: int, R: int, Dn: int, Dr: int, Dv: int, is_causal: bool,
              q_start: int = 0) -> dict:
    """Algorithmic flops: attention over the visible (query, key) pairs
    (2 (Dn + Dr) + 2 Dv per pair) and the one-pass K, V materialisation
    (2 R (Dn + Dv) per (batch, head, key))."""
    if is_causal:
        vis = int(np.clip(np.arange(S_q) + q_start + 1, 0, S_kv).sum())
    else:
        vis = S_q * S_kv
    attn = 2.0 * B * H * vis * (Dn + Dr + Dv)
    kv = 2.0 * B * H * S_kv * R * (Dn + Dv)
    return {"attention": attn, "kv": kv, "total": attn + kv, "pairs": B * H * vis}
