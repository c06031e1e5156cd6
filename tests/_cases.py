"""Config shapes and seeded synthetic inputs shared by tests, smoke() and bench.py.

Generation order (CPU, fp32, then cast): x, then the layer weights as in
``oracle.moe_ref.make_params`` (gate W, per routed expert w1, w3, w2, per
shared expert w1, w3, w2), then the upstream gradient (seed + 1).
"""
from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Optional

import torch

from oracle import moe_ref as R


@dataclass(frozen=True)
class Case:
    name: str
    T: int
    D: int
    E: int
    I: int
    k: int
    S: int
    I_s: int
    dtype: torch.dtype
    bias: str = "zeros"       # zeros | normal | skew
    route_scale: float = 1.0

    @property
    def N(self) -> int:
        return self.T * self.k

    def config(self) -> dict:
        return {"dim": self.D, "n_routed_experts": self.E, "n_shared_experts": self.S, "moe_inter_dim": self.I,
                "n_activated_experts": self.k, "shared_inter_dim": self.I_s, "route_scale": self.route_scale}

    def with_tokens(self, T: int) -> "Case":
        return Case(self.name + f"_T{T}", T, self.D, self.E, self.I, self.k, self.S, self.I_s, self.dtype, self.bias,
                    self.route_scale)


# The five BASELINE configs (0-indexed, as in BASELINE.json "configs").
C0 = Case("c0", 1024, 64, 4, 128, 2, 1, 128, torch.float32)
C1 = Case("c1", 8192, 1024, 16, 512, 4, 1, 1024, torch.bfloat16, bias="normal")
C2 = Case("c2", 8192, 1024, 16, 512, 4, 1, 1024, torch.bfloat16, bias="skew")
C3 = Case("c3", 8192, 2048, 64, 1408, 6, 2, 1408, torch.bfloat16)
C3_DECODE = Case("c3_decode", 64, 2048, 64, 1408, 6, 2, 1408, torch.bfloat16)
C4 = Case("c4", 16384, 2048, 64, 1408, 6, 2, 1408, torch.bfloat16)


def make_bias(case: Case, seed: int = 0) -> torch.Tensor:
    if case.bias == "zeros":
        return torch.zeros(case.E)
    if case.bias == "normal":
        return torch.randn(case.E, generator=torch.Generator().manual_seed(seed + 7)) * 0.01
    if case.bias == "skew":
        b = torch.zeros(case.E)
        b[:2] = 3.0
        return b
    raise ValueError(case.bias)


@functools.lru_cache(maxsize=2)
def _params(D, E, I, S, I_s, seed, bias_kind, dtype):
    c = Case("_", 1, D, E, I, 1, S, I_s, dtype, bias_kind)
    return R.make_params(D, E, I, S, I_s, seed=seed + 1, bias=make_bias(c, seed)).to(dtype)


def make_inputs(case: Case, seed: int = 0, with_dy: bool = False):
    """-> (x (T,D) in case.dtype, params (fp32 gate, experts in case.dtype), dy or None), all on CPU.
    The weights do not depend on T, so one generation serves every token count."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(case.T, case.D, generator=g)
    p = _params(case.D, case.E, case.I, case.S, case.I_s, seed, case.bias, case.dtype)
    dy = torch.randn(case.T, case.D, generator=torch.Generator().manual_seed(seed + 2)) if with_dy else None
    x = x.to(case.dtype)
    if dy is not None:
        dy = dy.to(case.dtype)
    return x, p, dy


def params_to(p: R.MoEParams, device) -> R.MoEParams:
    mv = lambda ts: [t.to(device) for t in ts]
    return R.MoEParams(p.gate_w.to(device), p.gate_bias.to(device), mv(p.w1), mv(p.w2), mv(p.w3), mv(p.sw1),
                       mv(p.sw2), mv(p.sw3))


def load_module(case: Case, p: R.MoEParams, device, module_cls):
    """Build ``module_cls(case.config())`` holding the weights of ``p``."""
    m = module_cls(case.config())
    sd = {"gate.weight": p.gate_w, "gate.bias": p.gate_bias}
    for e in range(case.E):
        sd[f"experts.{e}.w1.weight"] = p.w1[e]
        sd[f"experts.{e}.w2.weight"] = p.w2[e]
        sd[f"experts.{e}.w3.weight"] = p.w3[e]
    for s in range(case.S):
        sd[f"shared_experts.{s}.w1.weight"] = p.sw1[s]
        sd[f"shared_experts.{s}.w2.weight"] = p.sw2[s]
        sd[f"shared_experts.{s}.w3.weight"] = p.sw3[s]
    m = m.to(device=device, dtype=case.dtype)
    m.gate.float()
    m.load_state_dict(sd)
    return m


def grouped_case(T, D, E, I, counts, dtype, seed, scale=0.1):
    """Inputs of the grouped operator seam (models/moe_triton.py:504-525):
    x_sorted (T,D), w1/w3 (E,I,D), w2 (E,D,I), (E+1,) int64 offsets from
    per-expert row counts, sorted gate weights (T,)."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, D, generator=g) * scale).to(dtype)
    w1 = (torch.randn(E, I, D, generator=g) * scale).to(dtype)
    w2 = (torch.randn(E, D, I, generator=g) * scale).to(dtype)
    w3 = (torch.randn(E, I, D, generator=g) * scale).to(dtype)
    off = torch.cat([torch.zeros(1, dtype=torch.int64), torch.tensor(counts).cumsum(0)])
    gw = (torch.rand(T, generator=g) * 0.1).to(dtype)
    return x, w1, w2, w3, off, gw
