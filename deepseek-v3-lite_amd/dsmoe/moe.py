"""Drop-in DeepSeekMoE layer on the dsmoe HIP kernels.

Same constructor config keys, submodule names, ``state_dict`` keys, forward
signature and side state as the reference (models/moe.py:7-201):

* ``AuxLossFreeGate``  weight (E, dim) Parameter, fp32 ``bias`` buffer,
  ``update_bias(counts, speed)``, ``forward(x) -> (weights, indices)``.
* ``Expert``           w1/w3 (inter, dim), w2 (dim, inter) bias-free Linears.
* ``DeepSeekMoE``      gate, experts, shared_experts, ``forward(x)``,
  ``_last_weights``/``_last_indices``, ``get_load_balance_loss()``,
  ``update_gate_bias(speed)``, and ``_stacked_w*``/``_shared_w*`` (stacked on
  access only; the forward reads the per-expert tensors in place).

Compute runs only through libdsmoe.so on a ROCm device; a forward on CPU
tensors raises.  The gate computes fp32 logits from x (bf16 is upcast
exactly) and the fp32 gate weight.  ``moe_dispatch`` is accepted for config
compatibility and does not select a backend.  ``shared_inter_dim`` (extension,
default ``moe_inter_dim``) sets the shared experts' inter width.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.optim.optimizer import register_optimizer_step_post_hook

from . import ops


def _flt(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 else t.float()


# Parameter generation for the cast copies of fp32 expert weights.  A fused
# optimizer step (torch.optim.AdamW(fused=True), the reference trainer's choice
# on GPU, training/pretrain.py:197) rewrites the parameters in place without
# moving their version counters, so a copy keyed on (_version, data_ptr) alone
# would go stale.  Every torch.optim optimizer runs the global step post-hooks,
# whichever implementation (fused, foreach, for-loop) it takes, so the
# generation moves on every optimizer step of any optimizer.  Writes through
# ``p.data`` outside an optimizer move neither counter: callers that do that
# call ``invalidate_weight_casts()``.
_weight_generation = [0]


def invalidate_weight_casts() -> None:
    """Marks every cached cast copy of an expert weight as stale (each is made
    again on its next use).  Optimizer steps and in-place updates through the
    parameter itself do this on their own; writes through ``param.data`` do not."""
    _weight_generation[0] += 1


def _after_optimizer_step(_optimizer, _args, _kwargs) -> None:
    _weight_generation[0] += 1


_optimizer_hook = register_optimizer_step_post_hook(_after_optimizer_step)


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    """Arithmetic dtype of the expert GEMMs.  Under a bf16 autocast region
    (the reference's training step, training/pretrain.py:212-213) fp32
    activations and weights are cast to bf16, as autocast does for the
    reference's matmul/bmm calls (models/moe.py:128-131,175-178); the output
    and ``_last_weights`` keep x's dtype.  Other autocast dtypes leave fp32."""
    dt = x.device.type
    if (x.dtype == torch.float32 and torch.is_autocast_enabled(dt)
            and torch.get_autocast_dtype(dt) == torch.bfloat16):
        return torch.bfloat16
    return x.dtype


class _CachedCast(torch.autograd.Function):
    """Returns the cached cast copy ``wc`` of parameter ``w`` as an
    autograd-visible tensor; the backward hands the gradient to ``w`` in its
    dtype (the backward of autocast's weight cast)."""

    @staticmethod
    def forward(ctx, w, wc):
        ctx.dtype = w.dtype
        return wc.view_as(wc)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dtype), None


class AuxLossFreeGate(nn.Module):
    """Sigmoid top-k router with a non-trainable fp32 bias (models/moe.py:7-37)."""

    def __init__(self, config: dict):
        super().__init__()
        self.dim = config["dim"]
        self.topk = config["n_activated_experts"]
        self.n_routed_experts = config["n_routed_experts"]
        self.route_scale = config.get("route_scale", 1.0)
        self.bias_upper = config.get("bias_upper_threshold", 0.10)
        self.bias_lower = config.get("bias_lower_threshold", 0.10)
        self.weight = nn.Parameter(torch.empty(self.n_routed_experts, self.dim))
        nn.init.normal_(self.weight, std=0.006)
        self.register_buffer("bias", torch.zeros(self.n_routed_experts, dtype=torch.float32))

    @torch.no_grad()
    def update_bias(self, counts: torch.Tensor, speed: float = 0.001) -> None:
        """models/moe.py:21-27.  On a ROCm device this is one kernel and no host
        sync; on CPU the same band rule runs as buffer arithmetic."""
        if self.bias.is_cuda and self.bias.dtype == torch.float32 and self.bias.is_contiguous():
            ops.update_bias_(counts.to(self.bias.device), self.bias, speed, self.bias_upper, self.bias_lower)
            return
        counts = counts.float()
        avg = counts.mean()
        self.bias[counts > avg * (1.0 + self.bias_upper)] -= speed
        self.bias[counts < avg * (1.0 - self.bias_lower)] += speed

    def forward(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Normalised top-k weights (x dtype) and int64 expert indices."""
        out = ops.gate_forward(x, _flt(self.weight), _flt(self.bias), self.topk, self.route_scale)
        return out["weights_x"], out["idx64"]


class Expert(nn.Module):
    """Single SwiGLU expert ``W2(silu(W1 x) * W3 x)`` (models/moe.py:40-49)."""

    def __init__(self, dim: int, inter_dim: int):
        super().__init__()
        self.w1 = nn.Linear(dim, inter_dim, bias=False)
        self.w2 = nn.Linear(inter_dim, dim, bias=False)
        self.w3 = nn.Linear(dim, inter_dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Runs as a one-group call of the grouped HIP operator."""
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        off = torch.tensor([0, flat.shape[0]], dtype=torch.int64, device=flat.device)
        ones = torch.ones(flat.shape[0], dtype=flat.dtype, device=flat.device)
        y = ops.grouped_moe_dispatch(flat, self.w1.weight.unsqueeze(0), self.w2.weight.unsqueeze(0),
                                     self.w3.weight.unsqueeze(0), ones, off)
        return y.view(shape)


class DeepSeekMoE(nn.Module):
    """DeepSeekMoE with routed experts, shared experts and bias balancing (models/moe.py:52-201)."""

    def __init__(self, config: dict):
        super().__init__()
        self.dim = config["dim"]
        self.n_routed_experts = config["n_routed_experts"]
        self.n_shared_experts = config["n_shared_experts"]
        self.moe_inter_dim = config["moe_inter_dim"]
        self.shared_inter_dim = config.get("shared_inter_dim", self.moe_inter_dim)
        self.moe_dispatch = config.get("moe_dispatch", "stacked")
        self.gate = AuxLossFreeGate(config)
        self.experts = nn.ModuleList([Expert(self.dim, self.moe_inter_dim) for _ in range(self.n_routed_experts)])
        self.shared_experts = nn.ModuleList([Expert(self.dim, self.shared_inter_dim)
                                             for _ in range(self.n_shared_experts)])
        self._last_weights: Optional[torch.Tensor] = None
        self._last_indices: Optional[torch.Tensor] = None
        self._last_counts: Optional[torch.Tensor] = None
        self._counts_of: Optional[torch.Tensor] = None  # the _last_indices _last_counts was computed from
        self._stack_dtype: Optional[torch.dtype] = None
        # id(parameter) -> ((generation, version, data_ptr, dtype), cast copy); see _cast
        self._cast_cache: dict = {}

    # -------------------------------------------------------------- forward
    def _cast(self, w: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """w in ``dtype`` for the expert GEMMs.  Under autocast the weights
        are fp32 parameters and the GEMMs read bf16: the cast copy is cached
        and made again only when the parameter may have changed (an optimizer
        step of any torch.optim optimizer, an in-place update that moves its
        version counter, new storage), so a forward does not re-cast all
        expert weights.  The gradient flows back to the parameter in its own
        dtype, as through autocast's cast."""
        if w.dtype == dtype:
            return w
        if torch.compiler.is_compiling():
            return w.to(dtype)
        copy = self._cached_copy(w, dtype)
        if not (torch.is_grad_enabled() and w.requires_grad):
            return copy
        return _CachedCast.apply(w, copy)

    def _cached_copy(self, w: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """The detached cast copy of w, made again when w may have changed: the
        optimizer-step generation, w's version counter or its storage moved.
        Between a forward and its checkpoint recompute none of them moves, so
        the recompute reads the same copy."""
        key = (_weight_generation[0], w._version, w.data_ptr(), dtype)
        ent = self._cast_cache.get(id(w))
        if ent is None or ent[0] != key:
            with torch.no_grad():
                ent = (key, w.detach().to(dtype))
            self._cast_cache[id(w)] = ent
        return ent[1]

    def _expert_params(self):
        """Expert weight parameters in the layer operator's order."""
        return ([e.w1.weight for e in self.experts] + [e.w2.weight for e in self.experts] +
                [e.w3.weight for e in self.experts] + [e.w1.weight for e in self.shared_experts] +
                [e.w2.weight for e in self.shared_experts] + [e.w3.weight for e in self.shared_experts])

    def _apply(self, fn, *args, **kwargs):
        # .to() / .cuda() / .half() replace parameter data: drop the cast copies
        self._cast_cache.clear()
        return super()._apply(fn, *args, **kwargs)

    def _expert_weights(self, dtype: torch.dtype):
        def cast(w):
            return self._cast(w, dtype)
        w1 = [cast(e.w1.weight) for e in self.experts]
        w2 = [cast(e.w2.weight) for e in self.experts]
        w3 = [cast(e.w3.weight) for e in self.experts]
        s1 = [cast(e.w1.weight) for e in self.shared_experts]
        s2 = [cast(e.w2.weight) for e in self.shared_experts]
        s3 = [cast(e.w3.weight) for e in self.shared_experts]
        return w1, w2, w3, s1, s2, s3

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Flatten -> fused gate -> permute -> grouped SwiGLU -> combine + shared."""
        if not x.is_cuda:
            raise RuntimeError("dsmoe.DeepSeekMoE.forward needs a ROCm GPU tensor; there is no CPU implementation")
        shape = x.shape
        flat = x.reshape(-1, self.dim)
        cdt = _compute_dtype(flat)
        params = self._expert_params()
        masters = None
        if (cdt == torch.bfloat16 and torch.is_grad_enabled() and not torch.compiler.is_compiling() and
                all(p.dtype == torch.float32 and p.requires_grad for p in params)):
            # fp32 parameters under bf16 autocast: the GEMMs read the cached
            # bf16 copies and the backward writes fp32 gradients for the
            # parameters themselves (no per-parameter cast nodes)
            masters = params
            copies = [self._cached_copy(p, cdt) for p in params]
            E, S = self.n_routed_experts, self.n_shared_experts
            w1, w2, w3 = copies[:E], copies[E:2 * E], copies[2 * E:3 * E]
            s1, s2, s3 = copies[3 * E:3 * E + S], copies[3 * E + S:3 * E + 2 * S], copies[3 * E + 2 * S:]
        else:
            w1, w2, w3, s1, s2, s3 = self._expert_weights(cdt)
        y, idx64, wx, counts = ops.moe_layer(flat.to(cdt), _flt(self.gate.weight), _flt(self.gate.bias), w1, w2, w3,
                                             s1, s2, s3, k=self.gate.topk, route_scale=self.gate.route_scale,
                                             master_weights=masters)
        self._last_weights = wx.detach().to(flat.dtype)
        self._last_indices = idx64.detach()
        self._last_counts = counts.detach()
        self._counts_of = self._last_indices
        self._stack_dtype = cdt
        return y.to(flat.dtype).view(shape)

    # -------------------------------------------------------------- stacked views (read on access)
    def _stack(self, mods, name):
        if self._stack_dtype is None:
            return None
        ws = [getattr(m, name).weight for m in mods]
        return torch.stack(ws, 0).to(self._stack_dtype) if ws else None

    @property
    def _stacked_w1(self):
        return self._stack(self.experts, "w1")

    @property
    def _stacked_w2(self):
        return self._stack(self.experts, "w2")

    @property
    def _stacked_w3(self):
        return self._stack(self.experts, "w3")

    @property
    def _shared_w1(self):
        return self._stack(self.shared_experts, "w1")

    @property
    def _shared_w2(self):
        return self._stack(self.shared_experts, "w2")

    @property
    def _shared_w3(self):
        return self._stack(self.shared_experts, "w3")

    # -------------------------------------------------------------- balance metric / bias update
    def _counts(self) -> torch.Tensor:
        """Per-expert counts of the latest routing: the kernel histogram when the
        latest forward produced one, else bincount of _last_indices."""
        # The reference assigns _last_indices directly (e.g. to plant a
        # routing in tests); the kernel histogram only describes the indices
        # of the forward that produced it.
        if self._last_counts is not None and self._counts_of is self._last_indices:
            return self._last_counts
        return torch.bincount(self._last_indices.flatten(), minlength=self.n_routed_experts)

    def get_load_balance_loss(self) -> torch.Tensor:
        """models/moe.py:181-192: E * sum_i f_i P_i from the latest forward."""
        if self._last_weights is None or self._last_indices is None:
            return torch.tensor(0.0, device=self.gate.weight.device)
        weights = self._last_weights
        indices = self._last_indices
        T = weights.size(0)
        E = self.n_routed_experts
        counts = self._counts().float()
        f = counts / counts.sum().clamp(min=1e-10)
        one_hot = F.one_hot(indices.flatten(), num_classes=E).float()
        P = (one_hot * weights.flatten().float().unsqueeze(-1)).view(T, -1, E).sum(dim=1).mean(dim=0)
        return (f * P).sum() * E

    def update_gate_bias(self, speed: float = 0.001) -> None:
        """models/moe.py:194-201, fed by the device histogram (no host sync)."""
        if self._last_indices is None:
            return
        self.gate.update_bias(self._counts(), speed=speed)

