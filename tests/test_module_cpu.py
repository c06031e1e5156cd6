"""Host-side behaviour of the drop-in module (CPU only, no kernel launches):
constructor contract, state_dict keys, buffers, error on CPU forward, balance
metric and bias update from planted routings, config-compat helper.  Mirrors
the reference's tests/test_models.py:287-389,757-800 and tests/test_force_back.py."""
import pytest
import torch

from dsmoe import AuxLossFreeGate, DeepSeekMoE, Expert, enforce_triton_env_var, next_pow2
from oracle import moe_ref as R


def test_construction_and_state_dict_keys(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    assert len(moe.experts) == 4 and len(moe.shared_experts) == 1
    assert isinstance(moe.gate, AuxLossFreeGate)
    keys = set(moe.state_dict())
    expect = {"gate.weight", "gate.bias"}
    for e in range(4):
        expect |= {f"experts.{e}.w1.weight", f"experts.{e}.w2.weight", f"experts.{e}.w3.weight"}
    expect |= {"shared_experts.0.w1.weight", "shared_experts.0.w2.weight", "shared_experts.0.w3.weight"}
    assert keys == expect
    assert moe.experts[0].w1.weight.shape == (64, 64) and moe.experts[0].w2.weight.shape == (64, 64)
    assert moe.moe_dispatch == "stacked"
    assert DeepSeekMoE(dict(small_cfg, moe_dispatch="triton_grouped")).moe_dispatch == "triton_grouped"


def test_shared_inter_dim_extension(small_cfg):
    moe = DeepSeekMoE(dict(small_cfg, shared_inter_dim=128))
    assert moe.shared_experts[0].w1.weight.shape == (128, 64)
    assert moe.experts[0].w1.weight.shape == (64, 64)


def test_gate_contract(small_cfg):
    gate = AuxLossFreeGate(small_cfg)
    assert gate.weight.shape == (4, 64) and gate.bias.shape == (4,) and gate.bias.dtype == torch.float32
    assert id(gate.bias) not in {id(p) for p in gate.parameters()}
    assert "bias" in gate.state_dict()
    assert gate.route_scale == 1.0 and gate.bias_upper == 0.10 and gate.bias_lower == 0.10


def test_forward_on_cpu_raises(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    with pytest.raises(RuntimeError, match="ROCm"):
        moe(torch.randn(2, 8, 64))
    with pytest.raises(RuntimeError, match="ROCm"):
        moe.gate(torch.randn(8, 64))
    with pytest.raises(RuntimeError, match="ROCm"):
        Expert(64, 32)(torch.randn(3, 64))


def test_balance_loss_zero_before_forward(small_cfg):
    assert DeepSeekMoE(small_cfg).get_load_balance_loss().item() == 0.0


def test_balance_loss_from_planted_routing_matches_oracle(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    g = torch.Generator().manual_seed(0)
    idx = torch.stack([torch.randperm(4, generator=g)[:2] for _ in range(128)])
    w = torch.rand(128, 2, generator=g)
    w = w / w.sum(1, keepdim=True)
    moe._last_indices, moe._last_weights = idx, w
    assert abs(moe.get_load_balance_loss().item() - R.balance_loss_ref(w, idx, 4).item()) < 1e-6


def test_update_gate_bias_kat_all_to_expert0(small_cfg):
    """tests/test_models.py:325-345."""
    moe = DeepSeekMoE(small_cfg)
    moe._last_indices = torch.zeros(128, 2, dtype=torch.long)
    moe._last_weights = torch.ones(128, 2) / 2
    moe.update_gate_bias(speed=0.1)
    assert torch.equal(moe.gate.bias, torch.tensor([-0.1, 0.1, 0.1, 0.1]))


def test_update_bias_sign_rule_kat():
    """tests/test_models.py:760-777."""
    gate = AuxLossFreeGate({"dim": 8, "n_activated_experts": 2, "n_routed_experts": 4,
                            "bias_upper_threshold": 0.10, "bias_lower_threshold": 0.10})
    gate.update_bias(torch.tensor([10, 5, 5, 0], dtype=torch.float32), speed=0.01)
    assert torch.equal(gate.bias, torch.tensor([-0.01, 0.0, 0.0, 0.01]))


def test_update_gate_bias_noop_without_routing(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    moe.update_gate_bias(0.5)
    assert torch.equal(moe.gate.bias, torch.zeros(4))


def test_stacked_views_absent_before_forward(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    assert moe._stacked_w1 is None and moe._shared_w1 is None


@pytest.mark.parametrize("env,cfg,expect,warned", [
    (None, {"moe_dispatch": "triton_grouped"}, "stacked", True),
    ("1", {"moe_dispatch": "triton_grouped"}, "triton_grouped", False),
    (None, {"moe_dispatch": "stacked"}, "stacked", False),
])
def test_enforce_triton_env_var_compat(monkeypatch, env, cfg, expect, warned):
    """tests/test_force_back.py:29-72 behaviour of models/_triton_dispatch.py."""
    if env is None:
        monkeypatch.delenv("ENABLE_TRITON_KERNELS", raising=False)
    else:
        monkeypatch.setenv("ENABLE_TRITON_KERNELS", env)
    log = []
    enforce_triton_env_var(cfg, log.append)
    assert cfg["moe_dispatch"] == expect
    assert bool(log) == warned


def test_next_pow2():
    assert [next_pow2(n) for n in (0, 1, 2, 3, 64, 65, 384)] == [1, 1, 2, 4, 64, 128, 512]
