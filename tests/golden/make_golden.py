"""Write golden input/output vectors from the reference DeepSeekMoE layer.

Run once, in the build container, where the reference checkout is mounted:

    python tests/golden/make_golden.py /root/reference [fixture names...]

It imports ``models/moe.py`` and ``models/moe_triton.py`` from that checkout
(both import only torch), runs them on CPU in fp32, and stores inputs,
outputs and gradients as ``.npz`` fixtures next to this script.  The
fixtures are data only; nothing under ``tests/`` imports the reference.

What the fixtures pin that closed forms cannot: the exact op order and dtype
casts of ``DeepSeekMoE.forward`` (models/moe.py:74-103), the out-of-place
``index_add`` accumulation (:132), the batched shared path (:166-179), the
balance metric (:181-192) and autograd gradients through all of it.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _stack(mods, name):
    return torch.stack([getattr(m, name).weight.detach() for m in mods], 0)


def _set_weights(moe, g, std=0.02, bias=None):
    with torch.no_grad():
        for p in moe.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * std)
        if bias is not None:
            moe.gate.bias.copy_(bias)


def _collect(moe, x, y, dy=None):
    out = {
        "x": x.detach().numpy(),
        "gate_w": moe.gate.weight.detach().numpy(),
        "gate_bias": moe.gate.bias.detach().numpy(),
        "w1": _stack(moe.experts, "w1").numpy(), "w2": _stack(moe.experts, "w2").numpy(),
        "w3": _stack(moe.experts, "w3").numpy(),
        "y": y.detach().numpy(),
        "last_indices": moe._last_indices.numpy().astype(np.int64),
        "last_weights": moe._last_weights.float().numpy(),
        "counts": torch.bincount(moe._last_indices.flatten(), minlength=moe.n_routed_experts).numpy(),
        "balance_loss": np.float32(moe.get_load_balance_loss().item()),
    }
    if len(moe.shared_experts):
        out.update(sw1=_stack(moe.shared_experts, "w1").numpy(), sw2=_stack(moe.shared_experts, "w2").numpy(),
                   sw3=_stack(moe.shared_experts, "w3").numpy())
    if dy is not None:
        out["dy"] = dy.numpy()
        out["dx"] = x.grad.numpy()
        out["dgate_w"] = moe.gate.weight.grad.numpy()
        for nm in ("w1", "w2", "w3"):
            out["d" + nm] = torch.stack([getattr(m, nm).weight.grad for m in moe.experts], 0).numpy()
            if len(moe.shared_experts):
                out["ds" + nm] = torch.stack([getattr(m, nm).weight.grad for m in moe.shared_experts], 0).numpy()
    return out


def main(ref_root: str, only=()) -> None:
    """Writes every fixture, or only those named in ``only`` (file stems)."""
    sys.path.insert(0, ref_root)
    from models.moe import DeepSeekMoE  # noqa: E402  (reference, read-only checkout)
    from models.moe_triton import grouped_moe_pytorch  # noqa: E402

    torch.set_num_threads(1)

    def save(name: str, **arrays) -> None:
        if not only or name in only:
            np.savez_compressed(HERE / f"{name}.npz", **arrays)

    # 1) C0 shape (dim 64, 4 routed inter 128, 1 shared, top-2), fp32, fwd + bwd.
    cfg = {"dim": 64, "n_routed_experts": 4, "n_shared_experts": 1, "moe_inter_dim": 128,
           "n_activated_experts": 2}
    g = torch.Generator().manual_seed(0)
    moe = DeepSeekMoE(cfg)
    _set_weights(moe, g)
    x = torch.randn(2, 128, 64, generator=g).requires_grad_(True)
    y = moe(x)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(1))
    y.backward(dy)
    save("c0_fp32", **_collect(moe, x, y, dy))

    # 2) No shared experts, route_scale != 1, non-zero bias, custom thresholds.
    cfg2 = {"dim": 16, "n_routed_experts": 6, "n_shared_experts": 0, "moe_inter_dim": 8,
            "n_activated_experts": 3, "route_scale": 2.5}
    g = torch.Generator().manual_seed(2)
    moe2 = DeepSeekMoE(cfg2)
    _set_weights(moe2, g, std=0.2, bias=torch.tensor([0.02, -0.01, 0.0, 0.05, -0.03, 0.01]))
    x2 = torch.randn(40, 16, generator=g).requires_grad_(True)
    y2 = moe2(x2)
    dy2 = torch.randn(y2.shape, generator=torch.Generator().manual_seed(3))
    y2.backward(dy2)
    d2 = _collect(moe2, x2, y2, dy2)
    d2["route_scale"] = np.float32(2.5)
    save("noshared_scale", **d2)

    # 3) bf16 experts with the gate evaluated in fp32: the reference gate module
    #    is run on x.float() with an fp32 weight and its weights cast to bf16,
    #    the rest of the reference layer runs in bf16 unchanged.
    g = torch.Generator().manual_seed(4)
    moe3 = DeepSeekMoE(cfg)
    _set_weights(moe3, g)
    x3 = (torch.randn(256, 64, generator=g)).to(torch.bfloat16)
    gate32 = moe3.gate
    moe3 = moe3.to(torch.bfloat16)
    gate32 = gate32.float()

    class _Fp32Gate(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, flat):
            w, idx = self.inner(flat.float())
            return w.to(flat.dtype), idx

    gate_w32 = gate32.weight.detach().clone()
    moe3.gate = _Fp32Gate(gate32)
    with torch.no_grad():
        y3 = moe3(x3)
    save(
        "c0_bf16_fp32gate",
        x_bits=_bf16_bits(x3), gate_w=gate_w32.numpy(), gate_bias=gate32.bias.numpy(),
        w1_bits=_bf16_bits(_stack(moe3.experts, "w1")), w2_bits=_bf16_bits(_stack(moe3.experts, "w2")),
        w3_bits=_bf16_bits(_stack(moe3.experts, "w3")),
        sw1_bits=_bf16_bits(_stack(moe3.shared_experts, "w1")),
        sw2_bits=_bf16_bits(_stack(moe3.shared_experts, "w2")),
        sw3_bits=_bf16_bits(_stack(moe3.shared_experts, "w3")),
        y_bits=_bf16_bits(y3), last_indices=moe3._last_indices.numpy().astype(np.int64),
        last_weights_bits=_bf16_bits(moe3._last_weights))

    # 4) The grouped operator's CPU reference at the shape of the reference's own test.
    torch.manual_seed(0)
    T, D, E, I = 24, 16, 5, 12
    xs = torch.randn(T, D)
    w1 = torch.randn(E, I, D) * 0.1
    w2 = torch.randn(E, D, I) * 0.1
    w3 = torch.randn(E, I, D) * 0.1
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64), torch.tensor([6, 4, 5, 3, 6]).cumsum(0)])
    gw = torch.rand(T) * 0.2
    ys = grouped_moe_pytorch(xs, w1, w2, w3, offsets, gw)
    save("grouped_op", x_sorted=xs.numpy(), w1=w1.numpy(), w2=w2.numpy(),
                        w3=w3.numpy(), offsets=offsets.numpy(), sorted_weights=gw.numpy(), y_sorted=ys.numpy())
    # 5) bf16 forward and backward through the fp32-gate wrapper of (3): the
    #    reference layer's bf16 autograd (its rounding points in the routed
    #    loop, index_add and shared bmm), at the C0 shape with a normal bias.
    g = torch.Generator().manual_seed(6)
    moe5 = DeepSeekMoE(cfg)
    _set_weights(moe5, g, bias=torch.randn(4, generator=g) * 0.01)
    x5 = torch.randn(256, 64, generator=g).to(torch.bfloat16).requires_grad_(True)
    dy5 = torch.randn(256, 64, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    gate5 = moe5.gate
    moe5 = moe5.to(torch.bfloat16)
    gate5 = gate5.float()
    moe5.gate = _Fp32Gate(gate5)
    y5 = moe5(x5)
    y5.backward(dy5)
    d5 = {"x_bits": _bf16_bits(x5.detach()), "gate_w": gate5.weight.detach().numpy(),
          "gate_bias": gate5.bias.numpy(), "dy_bits": _bf16_bits(dy5), "y_bits": _bf16_bits(y5.detach()),
          "last_indices": moe5._last_indices.numpy().astype(np.int64),
          "dx_bits": _bf16_bits(x5.grad), "dgate_w": gate5.weight.grad.numpy()}
    for nm in ("w1", "w2", "w3"):
        d5[nm + "_bits"] = _bf16_bits(_stack(moe5.experts, nm))
        d5["s" + nm + "_bits"] = _bf16_bits(_stack(moe5.shared_experts, nm))
        d5["d" + nm + "_bits"] = _bf16_bits(torch.stack([getattr(m, nm).weight.grad for m in moe5.experts], 0))
        d5["ds" + nm + "_bits"] = _bf16_bits(torch.stack([getattr(m, nm).weight.grad for m in moe5.shared_experts], 0))
    save("c0_bf16_fwd_bwd", **d5)

    # 6) Wide routing: 16 routed experts, top-4 (the C1 routing width), two
    #    shared experts, a normal bias, route_scale 1.5, fp32 forward and backward.
    cfg6 = {"dim": 32, "n_routed_experts": 16, "n_shared_experts": 2, "moe_inter_dim": 24,
            "n_activated_experts": 4, "route_scale": 1.5}
    g = torch.Generator().manual_seed(8)
    moe6 = DeepSeekMoE(cfg6)
    _set_weights(moe6, g, std=0.1, bias=torch.randn(16, generator=g) * 0.01)
    x6 = torch.randn(200, 32, generator=g).requires_grad_(True)
    y6 = moe6(x6)
    dy6 = torch.randn(y6.shape, generator=torch.Generator().manual_seed(9))
    y6.backward(dy6)
    d6 = _collect(moe6, x6, y6, dy6)
    d6["route_scale"] = np.float32(1.5)
    save("e16_k4_fp32", **d6)
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", tuple(sys.argv[2:]))
