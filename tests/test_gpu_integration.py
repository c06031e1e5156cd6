"""The drop-in layer inside the reference's training step
(training/pretrain.py:172-175,212-213; models/transformer.py:80-85):

* bf16 autocast over fp32 parameters gives exactly the explicit bf16 layer
  (bf16-rounded weights and activations) with the output, ``_last_weights``
  and every gradient back in fp32; the expert weight gradients are the same
  fp32 accumulators unrounded (rounded to bf16 they are the bf16 layer's);
* activation checkpointing (``use_reentrant=False``) recomputes the forward
  with identical routing, so outputs and gradients are bit-identical to the
  plain run;
* ``torch.compile(fullgraph=True)`` traces the layer as one operator (no
  graph break) and gives the eager results bit for bit.
"""
import pytest
import torch

from tests import _cases as CS

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CASE32 = CS.Case("integ_fp32", 384, 256, 8, 128, 2, 1, 128, torch.float32, "normal")
CASE16 = CS.Case("integ_bf16", 384, 256, 8, 128, 2, 1, 128, torch.bfloat16, "normal")


def _grads(m):
    return {n: p.grad.detach().clone() for n, p in m.named_parameters()}


def _step(m, x, dy, fn=None):
    xin = x.detach().clone().to(DEV).requires_grad_(True)
    y = (m if fn is None else fn)(xin)
    (y.float() * dy.to(DEV).float()).sum().backward()
    torch.cuda.synchronize()
    return y.detach(), xin.grad.detach(), _grads(m)


def test_bf16_autocast_over_fp32_parameters():
    from dsmoe import DeepSeekMoE
    x, p, dy = CS.make_inputs(CASE32, with_dy=True)
    m32 = CS.load_module(CASE32, p, DEV, DeepSeekMoE)
    xin = x.clone().to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = m32(xin)
    assert y.dtype == torch.float32 and m32._last_weights.dtype == torch.float32
    (y * dy.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    # the explicit bf16 layer on the same (bf16-rounded) values
    m16 = CS.load_module(CASE16, p, DEV, DeepSeekMoE)
    y16, dx16, g16 = _step(m16, x.to(torch.bfloat16), dy)
    assert torch.equal(y, y16.float())
    assert torch.equal(m32._last_indices, m16._last_indices)
    assert torch.equal(m32._last_weights, m16._last_weights.float())
    assert xin.grad.dtype == torch.float32 and torch.equal(xin.grad, dx16.float())
    for n, prm in m32.named_parameters():
        assert prm.grad.dtype == torch.float32, n
        _same_gradient(n, prm.grad, g16[n])


def _same_gradient(name, g32, g16):
    """The gate gradient is fp32 in both layers (equal); an expert weight's
    fp32 gradient is the bf16 layer's accumulator before its rounding."""
    if name.startswith("gate."):
        assert torch.equal(g32, g16.float()), name
        return
    assert torch.equal(g32.to(torch.bfloat16), g16), name
    assert not torch.equal(g32, g16.float()), name   # unrounded (a bf16 cast pass would make them equal)


def test_activation_checkpoint_recompute_is_identical():
    from torch.utils.checkpoint import checkpoint
    from dsmoe import DeepSeekMoE
    x, p, dy = CS.make_inputs(CASE16, with_dy=True)
    m = CS.load_module(CASE16, p, DEV, DeepSeekMoE)
    y0, dx0, g0 = _step(m, x, dy)
    idx0 = m._last_indices.clone()
    m.zero_grad(set_to_none=True)
    y1, dx1, g1 = _step(m, x, dy, fn=lambda t: checkpoint(m, t, use_reentrant=False))
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1)
    assert torch.equal(idx0, m._last_indices)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


def test_torch_compile_traces_the_layer_as_one_op():
    import torch._dynamo
    from dsmoe import DeepSeekMoE
    x, p, dy = CS.make_inputs(CASE16, with_dy=True)
    m = CS.load_module(CASE16, p, DEV, DeepSeekMoE)
    y0, dx0, g0 = _step(m, x, dy)
    m.zero_grad(set_to_none=True)
    torch._dynamo.reset()
    cm = torch.compile(m, backend="aot_eager", fullgraph=True)
    y1, dx1, g1 = _step(m, x, dy, fn=cm)
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
    # the side state is set by the compiled forward too
    assert m._last_indices.shape == (CASE16.T, CASE16.k) and m._last_weights.dtype == torch.bfloat16


def test_torch_compile_inductor_backend():
    """The trainer's default compile backend (inductor) around the layer: one
    custom operator, results bit-identical to eager."""
    import torch._dynamo
    from dsmoe import DeepSeekMoE
    x, p, dy = CS.make_inputs(CASE16, with_dy=True)
    m = CS.load_module(CASE16, p, DEV, DeepSeekMoE)
    y0, dx0, g0 = _step(m, x, dy)
    m.zero_grad(set_to_none=True)
    torch._dynamo.reset()
    cm = torch.compile(m, backend="inductor", fullgraph=True)
    y1, dx1, g1 = _step(m, x, dy, fn=cm)
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n


@pytest.mark.parametrize("optimizer", ["sgd", "adamw_fused", "adamw_foreach"])
def test_autocast_weight_copies_follow_optimizer_steps(optimizer):
    """Under bf16 autocast the fp32 expert weights are cast once per
    parameter change: two training steps with an optimizer update between
    them give the explicit bf16 layer's results on the updated (bf16-rounded)
    weights.  The fused AdamW of the reference trainer (training/pretrain.py:197)
    rewrites the parameters without moving their version counters; the cast
    copies follow it through the optimizer step hook."""
    from dsmoe import DeepSeekMoE
    x, p, dy = CS.make_inputs(CASE32, with_dy=True)
    m32 = CS.load_module(CASE32, p, DEV, DeepSeekMoE)
    if optimizer == "sgd":
        opt = torch.optim.SGD(m32.parameters(), lr=0.5)
    else:
        # a large rate so every weight moves by more than a bf16 ulp
        opt = torch.optim.AdamW(m32.parameters(), lr=1e-2, weight_decay=0.1,
                                fused=optimizer == "adamw_fused", foreach=optimizer == "adamw_foreach")
    for step in range(2):
        opt.zero_grad(set_to_none=True)
        xin = x.clone().to(DEV).requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = m32(xin)
        (y * dy.to(DEV)).sum().backward()
        torch.cuda.synchronize()
        # the same parameters, experts rounded to bf16, the gate kept fp32
        m16 = DeepSeekMoE(CASE16.config()).to(DEV, torch.bfloat16)
        m16.gate.float()
        m16.load_state_dict({k: v.detach().clone() for k, v in m32.state_dict().items()})
        y16, dx16, g16 = _step(m16, x.to(torch.bfloat16), dy)
        assert torch.equal(y, y16.float()), step
        assert torch.equal(xin.grad, dx16.float()), step
        for n, prm in m32.named_parameters():
            _same_gradient(f"{n} (step {step})" if not n.startswith("gate.") else n, prm.grad, g16[n])
        before = m32.experts[0].w1.weight.detach().to(torch.bfloat16)
        opt.step()
        # the update is visible at bf16 precision, so a stale copy would fail above
        assert not torch.equal(before, m32.experts[0].w1.weight.detach().to(torch.bfloat16)), step
