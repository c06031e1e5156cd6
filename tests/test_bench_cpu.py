"""bench.py's contract, on the CPU (no device work): a request for more than
one GPU is refused before anything touches a device; the metric is the one
BASELINE.json names and the headline config is its 8192-token, 64-expert
top-6 layer; the FLOP and byte counts behind the reported rooflines are
pinned by counting the work element by element on small shapes (so a dropped
term, a missing gate/up factor or a wrong element size fails), and at C3 they
are the figures the committed profile summaries quote."""
import itertools
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n)], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that did not happen


def test_metric_and_headline_config_follow_baseline():
    base = json.loads((ROOT / "BASELINE.json").read_text())
    assert bench.METRIC == base["metric"]
    T, D, E, I, k, S, I_s, dt, _ = bench.CONFIGS["c3"]
    # north_star: the 8192-token, 64-expert top-6 bf16 layer
    assert (T, E, k, dt) == (8192, 64, 6, "bfloat16")
    assert bench.PEAK_BF16_TFLOPS == 2500.0 and bench.PEAK_HBM_GBS == 8000.0


def _count(cfg):
    """Multiply-adds and bytes of one forward, counted element by element."""
    T, D, E, I, k, S, I_s, dt, _ = cfg
    es = 2 if dt == "bfloat16" else 4
    N = T * k
    # gate/up: every routed slot's row times the W1 and the W3 rows of its
    # expert; every token's row times each shared expert's W1 and W3 rows
    g1 = sum(1 for _slot, _w, _n, _d in itertools.product(range(N), ("w1", "w3"), range(I), range(D)))
    g1 += sum(1 for _t, _s, _w, _n, _d in itertools.product(range(T), range(S), ("w1", "w3"), range(I_s), range(D)))
    # down projection: every slot's h row times W2; every token's shared h
    g2 = sum(1 for _slot, _o, _i in itertools.product(range(N), range(D), range(I)))
    g2 += sum(1 for _t, _s, _o, _i in itertools.product(range(T), range(S), range(D), range(I_s)))
    gate = T * D * es + E * D * 4 + N * 4 + N * 4 + E * 4   # x, fp32 W_gate, weights, indices, counts
    permute = N * 4 + 3 * N * 4 + E * 4 + E * 4  # indices in; sorted slot, token, position out; counts, offsets
    combine = N * D * es + T * D * es + N * 4 + N * 4 + T * D * es  # slot rows, shared rows, weights, indices, y
    return 2 * g1, 2 * g2, gate, permute, combine


@pytest.mark.parametrize("cfg", [(3, 4, 2, 5, 2, 1, 3, "bfloat16", "zeros"),
                                 (5, 8, 3, 2, 1, 2, 4, "bfloat16", "zeros"),
                                 (4, 4, 4, 3, 3, 0, 0, "float32", "zeros")])
def test_roofline_counts_by_enumeration(cfg):
    f1, f2, gate, permute, combine = _count(cfg)
    ms = {"gate": 1.0, "permute": 1.0, "gemm1": 1.0, "gemm2": 1.0, "combine": 1.0}
    r = bench.stage_rooflines(cfg, ms)
    assert r["gemm1"]["flop"] == f1
    assert r["gemm2"]["flop"] == f2
    assert r["gate"]["bytes"] == gate
    assert r["permute"]["bytes"] == permute
    assert r["combine"]["bytes"] == combine
    # 1 ms per stage: the rates are the counts per millisecond
    assert r["gemm1"]["TFLOP/s"] == pytest.approx(f1 / 1e-3 / 1e12)
    assert r["combine"]["frac_hbm"] == pytest.approx(combine / 1e-3 / 1e9 / 8000.0)


def test_c3_counts_are_the_profiles_figures():
    r = bench.stage_rooflines(bench.CONFIGS["c3"], {s: 1.0 for s in ("gate", "permute", "gemm1", "gemm2", "combine")})
    trace = (ROOT / "profiles" / "moe_fwd_c3_kernel_trace.md").read_text()
    assert "755.9 GFLOP" in trace and "378.0 GFLOP" in trace
    assert round(r["gemm1"]["flop"] / 1e9, 1) == 755.9
    assert round(r["gemm2"]["flop"] / 1e9, 1) == 378.0
    assert round(r["combine"]["bytes"] / 1e6, 1) == 268.8
    assert round(r["gate"]["bytes"] / 1e6, 1) == 34.5


def test_committed_traffic_is_the_gemm1_launch():
    t = json.loads((ROOT / "profiles" / "traffic_c3.json").read_text())
    assert t["gemm1_bytes"] == t["bytes_per_launch"]["c3 gemm1 (routed + shared gate/up, SwiGLU)"]
    # more than the launch's algorithmic bytes (operands once, h out), less than re-reading every operand
    T, D, E, I, k, S, I_s, _, _ = bench.CONFIGS["c3"]
    once = 2 * (T * D + E * 2 * I * D + S * 2 * I_s * D + T * k * I + T * S * I_s)
    assert once < t["gemm1_bytes"] < 3 * once
