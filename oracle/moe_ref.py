"""CPU restatement of the reference DeepSeekMoE layer — TEST INFRASTRUCTURE ONLY.

This module is the parity oracle for the HIP implementation in
``deepseek-v3-lite_amd/dsmoe``.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as the
checker / the timed CPU baseline.  The product path never calls it.

It restates, with torch CPU ops, the reference's default ("stacked") forward:

* ``gate_ref``            <- ``models/moe.py:29-37``  (AuxLossFreeGate.forward)
* ``routed_stacked_ref``  <- ``models/moe.py:105-133`` (_routed_forward_stacked)
* ``shared_ref``          <- ``models/moe.py:166-179`` (_shared_forward)
* ``moe_forward_ref``     <- ``models/moe.py:74-103``  (DeepSeekMoE.forward)
* ``grouped_moe_ref``     <- ``models/moe_triton.py:28-51`` (grouped_moe_pytorch)
* ``balance_loss_ref``    <- ``models/moe.py:181-192``
* ``update_bias_ref``     <- ``models/moe.py:21-27``
* ``expert_grad_slice_ref`` <- autograd of ``models/moe.py:128-132`` for one expert,
  restricted to a slice of its inter columns

Deliberate, documented deviation: the gate is evaluated on ``x.float()`` with
an fp32 gate weight (the reference runs ``F.linear`` in ``x.dtype``, i.e. bf16
under bf16, ``models/moe.py:32``).  For fp32 inputs the two are identical.

Extension: ``shared_inter_dim`` (default ``moe_inter_dim``) lets a shared expert
have a different inter width than routed experts.  One SwiGLU of inter ``2m``
equals the sum of two SwiGLUs of inter ``m`` holding the row halves of W1/W3 and
the column halves of W2; ``tests/test_oracle.py`` checks that identity.

Gradients of the oracle are ``torch.autograd`` through these functions.
Pinned by: golden vectors written by the real reference
(``tests/golden/*.npz``), the reference's own known-answer tests, closed forms
and brute-force loops (see ``tests/test_oracle.py``).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------------------
# Parameters of one layer, in the reference's per-expert layout.
# ----------------------------------------------------------------------------
@dataclass
class MoEParams:
    """Weights of one DeepSeekMoE layer, per-expert as in the reference
    ``state_dict`` (``models/moe.py:17-19,44-46,63-64``):
    gate_w (E, D) fp32, gate_bias (E,) fp32, w1/w3 (I, D), w2 (D, I)."""
    gate_w: torch.Tensor
    gate_bias: torch.Tensor
    w1: List[torch.Tensor]
    w2: List[torch.Tensor]
    w3: List[torch.Tensor]
    sw1: List[torch.Tensor] = field(default_factory=list)
    sw2: List[torch.Tensor] = field(default_factory=list)
    sw3: List[torch.Tensor] = field(default_factory=list)

    def tensors(self) -> List[torch.Tensor]:
        return [self.gate_w, *self.w1, *self.w2, *self.w3, *self.sw1, *self.sw2, *self.sw3]

    def to(self, dtype: torch.dtype) -> "MoEParams":
        """Cast expert weights to ``dtype``; the gate stays fp32."""
        c = lambda ts: [t.to(dtype) for t in ts]
        return MoEParams(self.gate_w.float(), self.gate_bias.float(), c(self.w1), c(self.w2), c(self.w3),
                         c(self.sw1), c(self.sw2), c(self.sw3))


def make_params(D: int, E: int, I: int, S: int, I_s: Optional[int] = None, *, seed: int = 0,
                std: float = 0.02, bias: Optional[torch.Tensor] = None) -> MoEParams:
    """Seeded synthetic weights in a fixed generation order (fp32, CPU):
    gate W, then per routed expert w1, w3, w2, then per shared expert w1, w3, w2.
    All ~N(0, std).  ``bias`` defaults to zeros."""
    I_s = I if I_s is None else I_s
    g = torch.Generator().manual_seed(seed)
    rn = lambda *shape: torch.randn(*shape, generator=g, dtype=torch.float32) * std
    gate_w = rn(E, D)
    w1, w2, w3 = [], [], []
    for _ in range(E):
        w1.append(rn(I, D)); w3.append(rn(I, D)); w2.append(rn(D, I))
    sw1, sw2, sw3 = [], [], []
    for _ in range(S):
        sw1.append(rn(I_s, D)); sw3.append(rn(I_s, D)); sw2.append(rn(D, I_s))
    b = torch.zeros(E, dtype=torch.float32) if bias is None else bias.float().clone()
    return MoEParams(gate_w, b, w1, w2, w3, sw1, sw2, sw3)


# ----------------------------------------------------------------------------
# Gate (models/moe.py:29-37)
# ----------------------------------------------------------------------------
def gate_logits_ref(x: torch.Tensor, gate_w: torch.Tensor) -> torch.Tensor:
    """fp32 logits ``x.float() @ W_gate.T`` (models/moe.py:32, fp32 variant)."""
    return F.linear(x.float(), gate_w.float())


def route_from_logits_ref(logits: torch.Tensor, bias: torch.Tensor, k: int, route_scale: float = 1.0,
                          indices: Optional[torch.Tensor] = None):
    """models/moe.py:32-36 from given fp32 logits, with torch's own sigmoid/topk.
    ``indices`` (T,k), when given, replaces the top-k selection (a routing
    fixed elsewhere, e.g. the layer's own at a near-tie); the weights are still
    gathered from these scores and renormalised.

    Returns (weights fp32 (T,k), indices int64 (T,k), scores fp32 (T,E))."""
    scores = logits.sigmoid()
    biased = scores + bias.to(scores.dtype)
    if indices is None:
        indices = biased.topk(k, dim=-1)[1]
    else:
        indices = indices.to(torch.int64)
    weights = scores.gather(1, indices)
    weights = weights / weights.sum(dim=-1, keepdim=True).clamp(min=1e-10) * route_scale
    return weights, indices, scores


def gate_ref(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor, k: int, route_scale: float = 1.0,
             indices: Optional[torch.Tensor] = None):
    """AuxLossFreeGate.forward (models/moe.py:29-37) on x.float() with an fp32
    gate weight; weights are cast to ``x.dtype`` as in models/moe.py:36."""
    w, idx, _ = route_from_logits_ref(gate_logits_ref(x, gate_w), bias, k, route_scale, indices)
    return w.to(x.dtype), idx


# ----------------------------------------------------------------------------
# Routed experts, stacked path (models/moe.py:105-133)
# ----------------------------------------------------------------------------
def routing_prep_ref(indices: torch.Tensor, E: int):
    """models/moe.py:107-117 with the canonical stable order.

    Returns (order, sorted_token_ids, counts (E,), offsets (E+1,)) as int64."""
    T, k = indices.shape
    flat_idx = indices.reshape(-1)
    token_id = torch.arange(T).repeat_interleave(k)
    order = torch.argsort(flat_idx, stable=True)
    counts = torch.bincount(flat_idx, minlength=E)
    offsets = torch.cat([torch.zeros(1, dtype=counts.dtype), counts.cumsum(0)])
    return order, token_id[order], counts, offsets


def routed_stacked_ref(flat: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor,
                       w1: List[torch.Tensor], w2: List[torch.Tensor], w3: List[torch.Tensor]) -> torch.Tensor:
    """Per-expert loop in ascending expert id; out-of-place index_add in
    ``flat.dtype`` exactly as models/moe.py:118-133."""
    E = len(w1)
    sw1 = torch.stack(list(w1), 0).to(flat.dtype)
    sw2 = torch.stack(list(w2), 0).to(flat.dtype)
    sw3 = torch.stack(list(w3), 0).to(flat.dtype)
    order, sorted_token_ids, counts, offsets = routing_prep_ref(indices, E)
    sorted_weights = weights.reshape(-1)[order]
    counts_l, offs_l = counts.tolist(), offsets.tolist()
    y = torch.zeros_like(flat)
    for e in range(E):
        cnt = counts_l[e]
        if cnt == 0:
            continue
        s = offs_l[e]
        tok = sorted_token_ids[s:s + cnt]
        cw = sorted_weights[s:s + cnt]
        xin = flat[tok]
        g = xin @ sw1[e].t()
        u = xin @ sw3[e].t()
        h = F.silu(g) * u
        out = h @ sw2[e].t()
        y = y.index_add(0, tok, out * cw.unsqueeze(-1))
    return y


def shared_ref(flat: torch.Tensor, sw1: List[torch.Tensor], sw2: List[torch.Tensor], sw3: List[torch.Tensor]) -> torch.Tensor:
    """models/moe.py:166-179: one bmm per projection over the S shared experts, then sum(0)."""
    S = len(sw1)
    if S == 0:
        return torch.zeros_like(flat)
    a = torch.stack(list(sw1), 0).to(flat.dtype)
    b = torch.stack(list(sw2), 0).to(flat.dtype)
    c = torch.stack(list(sw3), 0).to(flat.dtype)
    xs = flat.unsqueeze(0).expand(S, -1, -1)
    # Transposed operands are made contiguous before bmm (bf16 bmm with a
    # transposed right operand is avoided on purpose).
    g = torch.bmm(xs, a.transpose(-1, -2).contiguous())
    u = torch.bmm(xs, c.transpose(-1, -2).contiguous())
    h = F.silu(g) * u
    out = torch.bmm(h, b.transpose(-1, -2).contiguous())
    return out.sum(dim=0)


def moe_forward_ref(x: torch.Tensor, p: MoEParams, k: int, route_scale: float = 1.0, return_routing: bool = False,
                    indices: Optional[torch.Tensor] = None):
    """DeepSeekMoE.forward (models/moe.py:74-103): gate -> stacked routed -> + shared.
    ``indices``: see route_from_logits_ref."""
    D = p.gate_w.shape[1]
    shape = x.shape
    flat = x.reshape(-1, D)
    weights, indices = gate_ref(flat, p.gate_w, p.gate_bias, k, route_scale, indices)
    y = routed_stacked_ref(flat, indices, weights, p.w1, p.w2, p.w3)
    if p.sw1:
        y = y + shared_ref(flat, p.sw1, p.sw2, p.sw3)
    y = y.view(shape)
    if return_routing:
        return y, weights, indices
    return y


# ----------------------------------------------------------------------------
# Operator seam (models/moe_triton.py:28-51)
# ----------------------------------------------------------------------------
def grouped_moe_ref(x_sorted, w1, w2, w3, expert_offsets, sorted_weights):
    """grouped_moe_pytorch: per-expert SwiGLU over (E+1,) offsets, weighted rows."""
    E = w1.shape[0]
    y = torch.zeros(x_sorted.shape, dtype=x_sorted.dtype)
    offs = expert_offsets.tolist()
    for e in range(E):
        s, t = offs[e], offs[e + 1]
        if s == t:
            continue
        ch = x_sorted[s:t]
        h = F.silu(ch @ w1[e].t()) * (ch @ w3[e].t())
        y[s:t] = (h @ w2[e].t()) * sorted_weights[s:t].unsqueeze(-1)
    return y


# ----------------------------------------------------------------------------
# Balance metric and bias update (models/moe.py:21-27, 181-201)
# ----------------------------------------------------------------------------
def balance_loss_ref(weights: torch.Tensor, indices: torch.Tensor, E: int) -> torch.Tensor:
    T = weights.size(0)
    counts = torch.bincount(indices.flatten(), minlength=E).float()
    f = counts / counts.sum().clamp(min=1e-10)
    one_hot = F.one_hot(indices.flatten(), num_classes=E).float()
    P = (one_hot * weights.flatten().float().unsqueeze(-1)).view(T, -1, E).sum(dim=1).mean(dim=0)
    return (f * P).sum() * E


def update_bias_ref(bias: torch.Tensor, counts: torch.Tensor, speed: float, upper: float = 0.10,
                    lower: float = 0.10) -> torch.Tensor:
    b = bias.clone()
    c = counts.float()
    avg = c.mean()
    b[c > avg * (1.0 + upper)] -= speed
    b[c < avg * (1.0 - lower)] += speed
    return b


# ----------------------------------------------------------------------------
# Weight gradients of one expert, restricted to a slice of its inter columns.
# ----------------------------------------------------------------------------
def expert_grad_slice_ref(x_rows: torch.Tensor, dy_rows: torch.Tensor, w_rows: torch.Tensor, w1: torch.Tensor,
                          w2: torch.Tensor, w3: torch.Tensor, i0: int, i1: int):
    """fp32 weight gradients of one SwiGLU expert for inter columns [i0, i1).

    The expert sees rows ``x_rows`` (n, D) with routing weights ``w_rows``
    (n,) and the upstream gradient ``dy_rows`` (n, D) of the layer output,
    which holds ``w * W2 (silu(W1 x) * W3 x)`` for these rows
    (models/moe.py:128-132; shared experts: w = 1, models/moe.py:175-179).
    Column i of h depends only on row i of W1 and W3, and only column i of W2
    reads it, so the output splits into a sum over inter slices and the slice
    [i0, i1) of every weight gradient is the gradient of that slice's term:
    autograd of ``(w * silu(x W1s^T) * (x W3s^T)) W2s^T`` with W1s = W1[i0:i1],
    W3s = W3[i0:i1], W2s = W2[:, i0:i1], all in fp32.
    Returns (dW1[i0:i1] (m, D), dW2[:, i0:i1] (D, m), dW3[i0:i1] (m, D))."""
    x = x_rows.float()
    a = w1[i0:i1].detach().float().clone().requires_grad_(True)
    b = w2[:, i0:i1].detach().float().clone().requires_grad_(True)
    c = w3[i0:i1].detach().float().clone().requires_grad_(True)
    h = F.silu(x @ a.t()) * (x @ c.t())
    out = (h @ b.t()) * w_rows.float().unsqueeze(-1)
    out.backward(dy_rows.float())
    return a.grad, b.grad, c.grad


# ----------------------------------------------------------------------------
# Autograd convenience: forward + backward of the restatement.
# ----------------------------------------------------------------------------
def moe_forward_backward_ref(x: torch.Tensor, p: MoEParams, k: int, dy: torch.Tensor,
                             route_scale: float = 1.0, indices: Optional[torch.Tensor] = None) -> Dict[str, object]:
    """Runs moe_forward_ref under autograd and returns y and all gradients.

    Leaves: x, gate_w and every expert weight.  ``dy`` has x's shape.
    ``indices``: see route_from_logits_ref."""
    xl = x.detach().clone().requires_grad_(True)
    leaves = [t.detach().clone().requires_grad_(True) for t in p.tensors()]
    E, S = len(p.w1), len(p.sw1)
    it = iter(leaves)
    gw = next(it)
    w1 = [next(it) for _ in range(E)]
    w2 = [next(it) for _ in range(E)]
    w3 = [next(it) for _ in range(E)]
    sw1 = [next(it) for _ in range(S)]
    sw2 = [next(it) for _ in range(S)]
    sw3 = [next(it) for _ in range(S)]
    q = MoEParams(gw, p.gate_bias, w1, w2, w3, sw1, sw2, sw3)
    y, weights, indices = moe_forward_ref(xl, q, k, route_scale, return_routing=True, indices=indices)
    y.backward(dy)
    z = lambda t: t.grad if t.grad is not None else torch.zeros_like(t)
    return {
        "y": y.detach(), "weights": weights.detach(), "indices": indices.detach(),
        "dx": z(xl), "dgate_w": z(gw),
        "dw1": [z(t) for t in w1], "dw2": [z(t) for t in w2], "dw3": [z(t) for t in w3],
        "dsw1": [z(t) for t in sw1], "dsw2": [z(t) for t in sw2], "dsw3": [z(t) for t in sw3],
    }
