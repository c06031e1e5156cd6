#!/usr/bin/env python3
"""Benchmark of the dsmoe DeepSeekMoE layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

A step is one forward pass of the whole MoE layer (fused gate, permute,
grouped SwiGLU GEMMs for routed and shared experts, combine) over one batch
of synthetic tokens already resident in HBM.  The default workload is
BASELINE config 3 (prefill): T=8192 tokens, dim 2048, 64 routed experts
(inter 1408) top-6, 2 shared experts (inter 1408), bf16 activations and
experts, fp32 gate.  ``value`` is routed tokens/s = T / step time.

Printed as one JSON line, with
* ``roofline`` for the dominant kernel, the gate/up SwiGLU grouped GEMM (one
  launch covering the routed experts and the shared experts): algorithmic
  FLOPs per launch (4*N*D*I + 4*T*D*S*I_s, N = T*k slots) over its mean
  launch time measured with HIP events recorded by the library on the launch
  stream;
* ``cpu_baseline``: the CPU restatement of the reference stacked path
  (oracle/moe_ref.py) timed on this host on a bounded token sample;
* ``fwd_bwd``: the training step of BASELINE config 4 (the config-3 layer at
  T=16384: forward, then backward to dx, dW_gate and every expert's dW),
  timed over K / 2 steps after W warm-up steps, with its own per-stage
  times and CPU baseline (the oracle under autograd).

Order: the headline workload's W + K steps first, in a process that has not
used the GPU yet (``cold_start``: the clock is still ramping into its loaded
state for the first ~30 steps), then the other workloads (decode, C1, C2, MLA
attention, the vendor library's dense GEMMs, the training step), then the
headline's W + K steps again on the loaded GPU (``value``, ``ms_per_step``,
the stage times and the roofline), then the autocast figures, and the
host-side CPU baselines last.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import Optional

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "deepseek-v3-lite_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE-layer routed tokens/sec (fwd, fwd+bwd) at 1 GPU; % bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0

# name: (T, D, E, I, k, S, I_s, dtype, bias)
CONFIGS = {
    "c0": (1024, 64, 4, 128, 2, 1, 128, "float32", "zeros"),
    "c1": (8192, 1024, 16, 512, 4, 1, 1024, "bfloat16", "normal"),
    "c2": (8192, 1024, 16, 512, 4, 1, 1024, "bfloat16", "skew"),
    "c3": (8192, 2048, 64, 1408, 6, 2, 1408, "bfloat16", "zeros"),
    "c3_decode": (64, 2048, 64, 1408, 6, 2, 1408, "bfloat16", "zeros"),
    "c4": (16384, 2048, 64, 1408, 6, 2, 1408, "bfloat16", "zeros"),
}
FWD_ONLY = ("c0", "c1", "c2", "c3", "c3_decode")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_layer(cfg, device, seed: int = 0):
    """Seeded synthetic inputs generated on the GPU: x ~ N(0,1), weights ~ N(0, 0.02)."""
    import torch
    T, D, E, I, k, S, I_s, dt, bias_kind = cfg
    dtype = getattr(torch, dt)
    g = torch.Generator(device=device).manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, device=device, dtype=torch.float32)
    x = rn(T, D).to(dtype)
    gate_w = rn(E, D) * 0.02
    w1, w2, w3 = [], [], []
    for _ in range(E):
        w1.append((rn(I, D) * 0.02).to(dtype)); w3.append((rn(I, D) * 0.02).to(dtype))
        w2.append((rn(D, I) * 0.02).to(dtype))
    s1, s2, s3 = [], [], []
    for _ in range(S):
        s1.append((rn(I_s, D) * 0.02).to(dtype)); s3.append((rn(I_s, D) * 0.02).to(dtype))
        s2.append((rn(D, I_s) * 0.02).to(dtype))
    bias = torch.zeros(E, device=device)
    if bias_kind == "normal":
        bias = rn(E) * 0.01
    elif bias_kind == "skew":
        bias[:2] = 3.0
    return x, gate_w, bias, (w1, w2, w3, s1, s2, s3)


def cpu_baseline(cfg, x, gate_w, bias, weights, budget_s: float = 16.0, backward: bool = False,
                 min_tokens: int = 0):
    """Times oracle/moe_ref.py's restatement of the reference stacked forward
    (models/moe.py:74-179) on this host on a token sample sized to the budget
    (at least ``min_tokens``); with ``backward`` the autograd forward+backward
    of the same path.  A first pass over min(T, 256) tokens is the warm-up and,
    with the timed sample, gives a fit of the CPU time as fixed + per-token
    cost (the fixed part is the per-call weight work, which does not shrink
    with the sample)."""
    import torch
    from oracle import moe_ref as R
    T, D, E, I, k, S, I_s, dt, _ = cfg
    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024")))
    torch.set_num_threads(cores)
    w1, w2, w3, s1, s2, s3 = weights
    cpu = lambda ts: [t.detach().cpu() for t in ts]
    p = R.MoEParams(gate_w.detach().cpu(), bias.cpu(), cpu(w1), cpu(w2), cpu(w3), cpu(s1), cpu(s2), cpu(s3))
    xs = x.detach().cpu()
    dys = torch.randn(xs.shape, generator=torch.Generator().manual_seed(2)).to(xs.dtype) if backward else None

    def run(n):
        if backward:
            R.moe_forward_backward_ref(xs[:n], p, k, dys[:n])
        else:
            with torch.no_grad():
                R.moe_forward_ref(xs[:n], p, k)

    n1 = min(T, 256)
    t0 = time.perf_counter()
    run(n1)
    dt1 = time.perf_counter() - t0
    n = int(min(T, max(n1, min_tokens, n1 * (budget_s / 4.0) / max(dt1, 1e-6))))
    reps = 3 if not backward else 2
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run(n)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    what = "forward+backward (autograd) passes" if backward else "forward passes"
    out = {"value": n / med, "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"first {n} of {T} tokens, same weights; median of {reps} {what} "
                     f"({med * 1e3:.1f} ms each) after a {n1}-token warm-up pass; torch {torch.__version__} "
                     f"{torch.backends.cpu.get_cpu_capability()}"}
    if n > n1:
        per_tok = (med - dt1) / (n - n1)
        fixed = dt1 - per_tok * n1
        out["fit"] = {"fixed_s": fixed, "per_token_s": per_tok, "from": f"{n1} and {n} tokens",
                      "full_T_tokens_per_s": T / (fixed + per_tok * T) if fixed + per_tok * T > 0 else None}
    return out


def time_steps(step, steps: int, warmup: int):
    """-> (ms per step from events on the current stream, host wall ms per step)."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps, (time.perf_counter() - t0) * 1e3 / steps


def stage_times(step, steps: int):
    """Per-stage ms per step from the HIP events the library records on its
    launch stream (a training step makes two library calls, forward and
    backward, so totals are divided by steps, not by calls)."""
    import dsmoe._lib as L
    L.timing_enable(True)
    try:
        for _ in range(steps):
            step()
        torch_sync()
        stages, _ncalls = L.timing_read()
    finally:
        L.timing_enable(False)
    return {kname: v / steps for kname, v in stages.items()}


def stage_times_flushed(step, steps: int, dev):
    """stage_times with the caches flushed before every call: a 512 MiB write
    (twice the 256 MB MALL) between calls, outside the library's events, so
    the HBM-bound stages read their inputs from HBM."""
    import torch
    import dsmoe._lib as L
    scratch = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    L.timing_enable(True)
    try:
        for i in range(steps):
            scratch.fill_(i & 0xFF)
            step()
        torch_sync()
        stages, _ncalls = L.timing_read()
    finally:
        L.timing_enable(False)
    del scratch
    return {kname: v / steps for kname, v in stages.items()}


def stage_rooflines(cfg, stage_ms):
    """Per-stage rates against the stage's roof.  Algorithmic bytes / flops
    per forward (bf16 activations and expert weights, fp32 gate):
      gate     2TD (x) + 4ED (W_gate) + 8N (weights, indices) + 4E (counts)
      permute  4N (indices read) + 12N (sorted_slot, sorted_token, slot_pos) + 8E
      combine  2ND (slot rows) + 2TD (shared) + 4N (weights) + 4N (indices) + 2TD (y)
      GEMMs    gemm1 (routed + shared gate/up) 4 N D I + 4 T D S I_s, gemm2
               (down projections) 2 N D I + 2 T D S I_s flops (bf16 MFMA)"""
    T, D, E, I, k, S, I_s, dt, _ = cfg
    es = 2 if dt == "bfloat16" else 4
    N = T * k
    out = {}
    hbm = {"gate": es * T * D + 4 * E * D + 8 * N + 4 * E,
           "permute": 16 * N + 8 * E,
           "combine": es * N * D + 2 * es * T * D + 8 * N}
    for name, nbytes in hbm.items():
        ms = stage_ms.get(name)
        if ms:
            gbs = nbytes / (ms * 1e-3) / 1e9
            out[name] = {"ms": ms, "bytes": nbytes, "GB/s": gbs, "frac_hbm": gbs / PEAK_HBM_GBS}
    flops = {"gemm1": 4.0 * N * D * I + 4.0 * T * D * S * I_s, "gemm2": 2.0 * N * D * I + 2.0 * T * D * S * I_s}
    for name, f in flops.items():
        ms = stage_ms.get(name)
        if ms:
            tf = f / (ms * 1e-3) / 1e12
            out[name] = {"ms": ms, "flop": f, "TFLOP/s": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS}
    return out


def decode_bench(dev, steps: int, warmup: int):
    """Config 3 decode (T=64): the forward streams the weights of every expert
    that receives a token; reported as HBM GB/s of those weights against
    8 TB/s.  Weight bytes = sum over routed experts with rows of 3 D I (bf16)
    + the shared experts + the fp32 gate weight."""
    import torch
    from dsmoe import moe_layer
    cfg = CONFIGS["c3_decode"]
    T, D, E, I, k, S, I_s, dt, _ = cfg
    log(f"[bench] decode config c3_decode: T={T}")
    x, gate_w, bias, (w1, w2, w3, s1, s2, s3) = make_layer(cfg, dev)

    def step():
        return moe_layer(x, gate_w, bias, w1, w2, w3, s1, s2, s3, k=k, training=False)

    with torch.no_grad():
        counts = step()[3]
        ms, wall = time_steps(step, steps, warmup)
        stage_ms = stage_times(step, steps)
    touched = int((counts > 0).sum().item())
    nbytes = touched * 3 * D * I * 2 + S * 3 * D * I_s * 2 + E * D * 4
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] decode: {ms:.4f} ms/step, {touched} experts touched, {gbs:.0f} GB/s")
    return {"workload": f"c3_decode: T={T} tokens, dim={D}, {E} routed (inter {I}) top-{k}, {S} shared, bf16",
            "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3), "experts_touched": touched,
            "weight_bytes": nbytes, "GB/s": gbs, "frac_hbm": gbs / PEAK_HBM_GBS, "stage_ms": stage_ms}


# MLA attention shape: configs/pretrain_a100_422m.yaml:20-45 (micro batch 8, full 2048 sequence, causal)
MLA_SHAPE = {"B": 8, "H": 12, "S": 2048, "R": 192, "Dn": 48, "Dr": 24, "Dv": 64}


def mla_inputs(dev):
    """Seeded bf16 inputs of the MLA bench shape (q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v) and the scale."""
    import torch
    sh = MLA_SHAPE
    B, H, S, R, Dn, Dr, Dv = (sh[k] for k in ("B", "H", "S", "R", "Dn", "Dr", "Dv"))
    g = torch.Generator(device=dev).manual_seed(0)
    rn = lambda *s_: torch.randn(*s_, generator=g, device=dev, dtype=torch.float32)
    ts = [t.to(torch.bfloat16) for t in (rn(B, H, S, Dn), rn(B, H, S, Dr), rn(B, S, R), rn(B, S, Dr),
                                         rn(H, Dn, R) * 0.1, rn(H, Dv, R) * 0.1)]
    return ts, (Dn + Dr) ** -0.5


def mla_cpu_baseline(dev, gpu_ms: float):
    """The reference layer's default attention path (models/mla.py:155-172:
    K, V by bmm, then scaled_dot_product_attention) restated with torch ops
    (oracle/mla_ref.py) and timed on the host cores on the whole bench call."""
    import torch
    from oracle.mla_ref import mla_attention_sdpa_torch
    sh = MLA_SHAPE
    B, H, S = sh["B"], sh["H"], sh["S"]
    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024")))
    torch.set_num_threads(cores)
    ts, scale = mla_inputs(dev)
    cpu = [t.cpu() for t in ts]
    with torch.no_grad():
        mla_attention_sdpa_torch(*cpu, scale, is_causal=True)          # warm-up
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            mla_attention_sdpa_torch(*cpu, scale, is_causal=True)
            times.append(time.perf_counter() - t0)
    dt = statistics.median(times)
    return {"value": B * S / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"the whole call (B={B}, H={H}, S={S}, causal, bf16): the reference layer's SDPA path "
                      f"(models/mla.py:155-172) restated with torch ops (oracle/mla_ref.py "
                      f"mla_attention_sdpa_torch), median of 3 ({dt * 1e3:.1f} ms each) after a warm-up call; "
                      f"torch {torch.__version__} {torch.backends.cpu.get_cpu_capability()}"}, dt / (gpu_ms * 1e-3)


def mla_bench(dev, steps: int, warmup: int):
    """Fused MLA attention forward (models/mla_triton.py:303-329) at the 422m
    config's shape, causal: the two kernels of csrc/mla.hip (K, V
    materialisation + flash attention) per call; then the operator's
    training step (forward and backward to every input) as "fwd_bwd".  Algorithmic flops: 2 (Dn +
    Dr + Dv) per visible (query, key) pair plus 2 R (Dn + Dv) per (batch,
    head, key) for K and V.  Beside it, the reference's default SDPA path
    (models/mla.py:155-172: K, V materialised with bmm, then
    scaled_dot_product_attention) run by torch on the same GPU, when a fused
    SDPA backend takes the shape."""
    import torch
    from dsmoe.mla import mla_attention_fwd
    sh = MLA_SHAPE
    B, H, S, R, Dn, Dr, Dv = (sh[k] for k in ("B", "H", "S", "R", "Dn", "Dr", "Dv"))
    ts, scale = mla_inputs(dev)
    log(f"[bench] mla: B={B} H={H} S={S} R={R} Dn={Dn} Dr={Dr} Dv={Dv} causal")

    def step():
        return mla_attention_fwd(*ts, scale, True, 0)

    with torch.no_grad():
        ms, _ = time_steps(step, steps, warmup)
    vis = S * (S + 1) // 2
    flop_attn = 2.0 * B * H * vis * (Dn + Dr + Dv)
    flop_kv = 2.0 * B * H * S * R * (Dn + Dv)
    tf = (flop_attn + flop_kv) / (ms * 1e-3) / 1e12
    out = {"workload": f"MLA attention forward, B={B} H={H} S_q=S_kv={S} R={R} D_nope={Dn} D_rope={Dr} "
                       f"D_v={Dv}, causal, bf16 (configs/pretrain_a100_422m.yaml shape)",
           "ms_per_call": ms, "tokens_per_s": B * S / (ms * 1e-3), "flop": flop_attn + flop_kv,
           "TFLOP/s": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS,
           # the reference kernel rebuilds K, V of every visible 64-key block
           # for each 64-query block (models/mla_triton.py:135-147)
           "reference_kernel_flop": 2.0 * B * H * vis * (Dn + Dr + Dv)
           + 2.0 * B * H * sum(min(i + 1, (S + 63) // 64) for i in range((S + 63) // 64)) * 64 * R * (Dn + Dv)}
    # the reference's SDPA path on this GPU (fused backends only: the math
    # path's bf16 batched products are avoided on this pool)
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        qn, qp, kv, pe, wk, wv = ts
        wkv = torch.cat([wk, wv], dim=1).transpose(-1, -2).contiguous()          # (H, R, Dn + Dv)

        def ref_step():
            kvb = kv.reshape(B * S, R).unsqueeze(0).expand(H, -1, -1).contiguous()
            kvh = torch.bmm(kvb, wkv)
            k_n, v_h = kvh.split([Dn, Dv], dim=-1)
            k_n = k_n.reshape(H, B, S, Dn).permute(1, 0, 2, 3)
            v_h = v_h.reshape(H, B, S, Dv).permute(1, 0, 2, 3)
            # V padded to the q/k head width (the fused SDPA backends take one width)
            v_h = torch.nn.functional.pad(v_h, (0, Dn + Dr - Dv)).contiguous()
            k = torch.cat([k_n, pe.unsqueeze(1).expand(-1, H, -1, -1)], dim=-1).contiguous()
            q = torch.cat([qn, qp], dim=-1).contiguous()
            return torch.nn.functional.scaled_dot_product_attention(q, k, v_h, is_causal=True, scale=scale)[..., :Dv]

        with torch.no_grad(), sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            ref_ms, _ = time_steps(ref_step, max(3, steps // 2), max(2, warmup // 2))
        out["reference_sdpa_ms"] = ref_ms
        out["speedup_vs_reference_sdpa"] = ref_ms / ms
    except Exception as e:  # no fused SDPA backend for this shape
        out["reference_sdpa_ms"] = None
        out["reference_sdpa_note"] = f"{type(e).__name__}: {str(e)[:160]}"
    # training step of the operator: forward (with the log-sum-exp) and the
    # backward to all six inputs (csrc/mla.hip backward kernels + the two
    # projection GEMMs); algorithmic flops: the forward's, then per visible
    # pair dV, dP, dQ, dK (2 (2 (Dn + Dr) + 2 Dv)) and the projections
    # d ctx_kv, dW (2 x 2 B S H (Dn + Dv) R); the backward's recompute of K, V
    # and of the scores is not counted
    from dsmoe.mla import mla_attention
    ins = [t.clone().requires_grad_(True) for t in ts]
    g = torch.Generator(device=dev).manual_seed(1)
    dout = torch.randn(B, S, H, Dv, generator=g, device=dev).to(torch.bfloat16)

    def train_step():
        o = mla_attention(*ins, scale, True, 0)
        return torch.autograd.grad(o, ins, dout)

    ms_fb, _ = time_steps(train_step, max(3, steps // 2), max(2, warmup))
    flop_fb = flop_attn + flop_kv + 2.0 * B * H * vis * (2 * (Dn + Dr) + 2 * Dv) + 4.0 * B * S * H * (Dn + Dv) * R
    out["fwd_bwd"] = {"ms_per_step": ms_fb, "flop": flop_fb, "TFLOP/s": flop_fb / (ms_fb * 1e-3) / 1e12,
                      "tokens_per_s": B * S / (ms_fb * 1e-3)}
    log(f"[bench] mla: {ms:.4f} ms/call, {tf:.0f} TFLOP/s ({tf / PEAK_BF16_TFLOPS:.1%}), "
        f"reference SDPA {out.get('reference_sdpa_ms')}; forward + backward {ms_fb:.4f} ms "
        f"({out['fwd_bwd']['TFLOP/s']:.0f} TFLOP/s)")
    return out


def fwd_bench(name: str, dev, steps: int, warmup: int):
    """Forward of another BASELINE config (C1, C2 with its skewed bias): step
    time, routed tokens/s, the grouped GEMMs' rate, per-stage times and the
    largest expert's share of the slots."""
    import torch
    from dsmoe import moe_layer
    cfg = CONFIGS[name]
    T, D, E, I, k, S, I_s, dt, bias_kind = cfg
    log(f"[bench] forward config {name}: T={T} D={D} E={E} I={I} k={k} S={S}x{I_s} {dt} bias={bias_kind}")
    x, gate_w, bias, (w1, w2, w3, s1, s2, s3) = make_layer(cfg, dev)

    def step():
        return moe_layer(x, gate_w, bias, w1, w2, w3, s1, s2, s3, k=k, training=False)

    with torch.no_grad():
        counts = step()[3]
        ms, wall = time_steps(step, steps, warmup)
        stage_ms = stage_times(step, steps)
    N = T * k
    gemm_flops = 6.0 * N * D * I + 6.0 * T * D * S * I_s
    gemm_ms = sum(stage_ms.get(s, 0.0) for s in ("gemm1", "gemm2"))
    tf = gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None
    log(f"[bench] {name}: {ms:.4f} ms/step, grouped GEMMs {tf:.0f} TFLOP/s")
    return {"workload": f"{name}: DeepSeekMoE layer forward, T={T}, dim={D}, {E} routed (inter {I}) top-{k}, "
                        f"{S} shared (inter {I_s}), {dt}, fp32 gate, gate bias {bias_kind}",
            "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3), "grouped_gemm_tflops": tf,
            "grouped_gemm_frac": tf / PEAK_BF16_TFLOPS if tf else None, "stage_ms": stage_ms,
            "max_expert_share": float(counts.max().item()) / N}


def autocast_bench(dev, steps: int, warmup: int, ref_fwd_ms: float, ref_fwd_bwd_ms: Optional[float]):
    """The drop-in module (fp32 parameters) under bf16 autocast, the way the
    reference trains (training/pretrain.py:212-213): C3 forward and, when the
    bf16-weights training step was timed, the C4 forward+backward to every
    parameter.  Reported beside the bf16-weights layer times; the module casts
    its fp32 expert weights once per parameter change, not per call."""
    import torch
    from dsmoe import DeepSeekMoE
    out = {}
    for name, ref_ms, train in (("c3", ref_fwd_ms, False), ("c4", ref_fwd_bwd_ms, True)):
        if ref_ms is None:
            continue
        T, D, E, I, k, S, I_s, dt, _ = CONFIGS[name]
        torch.manual_seed(0)
        mod = DeepSeekMoE({"dim": D, "n_routed_experts": E, "n_shared_experts": S, "n_activated_experts": k,
                           "moe_inter_dim": I, "shared_inter_dim": I_s}).to(dev)
        x = torch.randn(T, D, device=dev, dtype=torch.bfloat16)
        if train:
            x.requires_grad_(True)
            dy = torch.randn(T, D, device=dev, dtype=torch.bfloat16)
            leaves = [x] + [p for p in mod.parameters() if p.requires_grad]

            def step():
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    y = mod(x)
                return torch.autograd.grad(y, leaves, dy)
            ms, _ = time_steps(step, max(3, steps // 4), max(2, warmup // 4))
        else:
            def step():
                with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                    return mod(x)
            ms, _ = time_steps(step, steps, warmup)
        key = "fwd_bwd_c4" if train else "fwd_c3"
        out[key] = {"ms_per_step": ms, "bf16_weights_ms_per_step": ref_ms, "ratio": ms / ref_ms}
        log(f"[bench] autocast {key}: {ms:.4f} ms/step vs {ref_ms:.4f} with bf16 weights ({ms / ref_ms:.3f}x)")
        del mod, x
        torch.cuda.empty_cache()
    return out


def blas_dense_reference(dev, cfg, steps: int = 30, warmup: int = 10):
    """The vendor library on the dense problems of the config's grouped GEMMs:
    torch.matmul (hipBLASLt) of bf16 NT products with all T*k routed rows as one
    matrix, gate/up (N = 2 I, K = D) and down (N = D, K = I).  Not the MoE
    layer: a reference point for the grouped GEMMs' fraction of peak at these
    shapes (no gather, no ragged tiles, no epilogue)."""
    import torch
    T, D, E, I, k, S, I_s, dt, _ = cfg
    N = T * k
    out = {}
    for name, (m, n, kk) in (("gate_up", (N, 2 * I, D)), ("down", (N, D, I))):
        a = torch.randn(m, kk, device=dev, dtype=torch.bfloat16)
        b = torch.randn(n, kk, device=dev, dtype=torch.bfloat16)
        for _ in range(warmup):
            c = a @ b.t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            c = a @ b.t()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        tf = 2.0 * m * n * kk / (ms * 1e-3) / 1e12
        out[name] = {"M": m, "N": n, "K": kk, "ms": ms, "TFLOP/s": tf, "frac_mfma": tf / PEAK_BF16_TFLOPS}
        del a, b, c
    log("[bench] hipBLASLt dense reference: " + ", ".join(f"{k_} {v['TFLOP/s']:.0f} TFLOP/s" for k_, v in out.items()))
    return out


def torch_sync():
    import torch
    torch.cuda.synchronize()


def fwd_bwd_bench(name: str, dev, steps: int, warmup: int):
    """Training step of the layer (config 4): forward, then backward to dx,
    dW_gate and every expert dW (torch.autograd.grad, no accumulation)."""
    import torch
    from dsmoe import moe_layer
    cfg = CONFIGS[name]
    T, D, E, I, k, S, I_s, dt, _ = cfg
    log(f"[bench] fwd+bwd config {name}: T={T} D={D} E={E} I={I} k={k} S={S}x{I_s} {dt}")
    x, gate_w, bias, weights = make_layer(cfg, dev)
    w1, w2, w3, s1, s2, s3 = [[t.requires_grad_(True) for t in ws] for ws in weights]
    x.requires_grad_(True)
    gate_w.requires_grad_(True)
    dy = torch.randn(x.shape, generator=torch.Generator(device=dev).manual_seed(2), device=dev).to(x.dtype)
    leaves = [x, gate_w, *w1, *w2, *w3, *s1, *s2, *s3]

    def step():
        y = moe_layer(x, gate_w, bias, w1, w2, w3, s1, s2, s3, k=k, training=True)[0]
        return torch.autograd.grad(y, leaves, dy)

    ms, wall = time_steps(step, steps, warmup)
    log(f"[bench] fwd+bwd timed {steps} steps: {ms:.3f} ms/step (host wall {wall:.3f} ms/step)")
    stage_ms = stage_times(step, steps)
    log(f"[bench] fwd+bwd stages (ms/call): " + ", ".join(f"{a}={b:.4f}" for a, b in stage_ms.items()))
    N = T * k
    flops = 3.0 * (6.0 * N * D * I + 6.0 * T * D * S * I_s)
    gemm_ms = sum(v for s, v in stage_ms.items() if s.startswith(("gemm", "bwd_d")) and s != "bwd_dw_dot")
    out = {"workload": f"{name}: DeepSeekMoE layer forward+backward (dx, dW_gate, every expert dW), T={T}, dim={D}, "
                       f"{E} routed (inter {I}) top-{k}, {S} shared (inter {I_s}), {dt}, fp32 gate",
           "value": T / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms, "steps": steps, "warmup": warmup,
           "gemm_tflops": flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None,
           "gemm_frac": flops / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS if gemm_ms > 0 else None,
           "stage_ms": stage_ms}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5, help="untimed steps before the timed ones")
    ap.add_argument("--config", default="c3", choices=FWD_ONLY)
    ap.add_argument("--fwd-bwd-config", default="c4", choices=sorted(CONFIGS),
                    help="training-step workload reported under fwd_bwd")
    ap.add_argument("--no-fwd-bwd", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-3 decode (T=64) measurement")
    ap.add_argument("--no-extra-configs", action="store_true", help="skip the C1 / C2 forward figures")
    ap.add_argument("--no-autocast", action="store_true", help="skip the module-under-autocast figures")
    ap.add_argument("--no-mla", action="store_true", help="skip the MLA attention figures")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="instead of the layer, run --steps device copies of this many MiB (counter calibration)")
    ap.add_argument("--dma-mb", type=int, default=0,
                    help="instead of the layer, run --steps direct global->LDS reads of this many MiB "
                         "(counter calibration for the GEMMs' load path)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the multi-GPU (expert-parallel) path is not built", file=sys.stderr)
        return 2

    import torch
    from dsmoe import moe_layer

    dev = torch.device("cuda:0")
    if args.copy_mb:
        n = args.copy_mb * (1 << 20)
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": args.steps}), flush=True)
        return 0
    if args.dma_mb:
        # the measurement-only probe library (include/dsmoe_probe.h), not the layer's
        import ctypes
        import dsmoe._lib as L
        probe = ctypes.CDLL(str(L.LIB_PATH.with_name("libdsmoe_probe.so")))
        probe.dsmoe_probe_dma_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        probe.dsmoe_probe_dma_read.restype = ctypes.c_int
        n = args.dma_mb * (1 << 20)
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        sink = torch.empty(args.dma_mb, dtype=torch.int32, device=dev)
        for _ in range(args.steps):
            rc = probe.dsmoe_probe_dma_read(L.ptr(src), n, L.ptr(sink), L.stream_ptr(dev))
            if rc != 0:
                raise RuntimeError(f"dsmoe_probe_dma_read failed with status {rc}")
        torch.cuda.synchronize()
        print(json.dumps({"dma_read_bytes_per_launch": n, "launches": args.steps}), flush=True)
        return 0
    cfg = CONFIGS[args.config]
    T, D, E, I, k, S, I_s, dt, bias_kind = cfg
    log(f"[bench] config {args.config}: T={T} D={D} E={E} I={I} k={k} S={S}x{I_s} {dt}")
    x, gate_w, bias, weights = make_layer(cfg, dev)
    w1, w2, w3, s1, s2, s3 = weights

    def step():
        return moe_layer(x, gate_w, bias, w1, w2, w3, s1, s2, s3, k=k, training=False)

    extra = {}
    with torch.no_grad():
        # the same W + K protocol on a GPU that has run nothing yet.  After an
        # idle gap (100 ms is enough) the GPU's clock ramps back up over about
        # 30 ms of load: measured on MI355X, the first 10 C3 steps average
        # 1.29-1.37 ms and steps 30 onwards 1.09 ms, and after 0.5 s of matmul
        # load the first 10 average 1.094 ms.  So this is reported beside the
        # headline, which is timed on the loaded GPU
        cold_ms, _ = time_steps(step, args.steps, args.warmup)
        log(f"[bench] cold start ({args.warmup} warm-up steps in a fresh process): {cold_ms:.3f} ms/step")
    # the other workloads, then the headline on the loaded GPU: the MFMA-heavy
    # ones (the vendor library's dense GEMMs, the training step) run last
    # before it, since lighter work (attention, decode) leaves the clock below
    # its loaded state
    if not args.no_decode and args.config == "c3":
        extra["decode"] = decode_bench(dev, max(10, args.steps), max(3, args.warmup))
    if not args.no_extra_configs and args.config == "c3":
        extra["configs_fwd"] = {c: fwd_bench(c, dev, args.steps, args.warmup) for c in ("c1", "c2")}
    if not args.no_mla and args.config == "c3":
        extra["mla"] = mla_bench(dev, args.steps, args.warmup)
    if not args.no_extra_configs and args.config == "c3":
        extra["blas_dense_reference"] = blas_dense_reference(dev, cfg)
    if not args.no_fwd_bwd:
        extra["fwd_bwd"] = fwd_bwd_bench(args.fwd_bwd_config, dev, max(3, args.steps // 2), max(1, args.warmup))
    with torch.no_grad():
        ms, wall = time_steps(step, args.steps, args.warmup)
        log(f"[bench] timed {args.steps} steps: {ms:.3f} ms/step (host wall {wall:.3f} ms/step)")
        stage_ms = stage_times(step, args.steps)
        flushed_ms = stage_times_flushed(step, args.steps, dev)
    log(f"[bench] stages (ms/call): " + ", ".join(f"{a}={b:.4f}" for a, b in stage_ms.items()))
    log(f"[bench] stages, caches flushed before each call (ms/call): " +
        ", ".join(f"{a}={b:.4f}" for a, b in flushed_ms.items()))

    N = T * k
    stages = stage_rooflines(cfg, stage_ms)
    g1_flops = 4.0 * N * D * I + 4.0 * T * D * S * I_s
    g1_ms = stage_ms.get("gemm1", float("nan"))
    achieved = g1_flops / (g1_ms * 1e-3) / 1e12
    gemm_flops = 6.0 * N * D * I + 6.0 * T * D * S * I_s
    gemm_ms = sum(stage_ms.get(s, 0.0) for s in ("gemm1", "gemm2"))
    traffic = None
    prof = ROOT / "profiles" / f"traffic_{args.config}.json"
    if prof.exists():
        traffic = json.loads(prof.read_text()).get("gemm1_bytes")

    result = {
        "metric": METRIC,
        "value": T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dt == "bfloat16" else "f32",
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) weights, generated on device)",
        "config": {"workload": f"{args.config}: DeepSeekMoE layer forward, T={T} tokens, dim={D}, "
                               f"{E} routed experts (inter {I}) top-{k}, {S} shared (inter {I_s}), {dt}, fp32 gate",
                   "T": T, "D": D, "E": E, "I": I, "k": k, "S": S, "I_s": I_s},
        "roofline": {"bound": "mfma", "kernel": "gemm1 (gate/up SwiGLU grouped GEMM, routed + shared experts)",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic},
        "slots_per_s": N / (ms * 1e-3),
        "grouped_gemm_tflops": gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None,
        "grouped_gemm_frac": (gemm_flops / (gemm_ms * 1e-3) / 1e12) / PEAK_BF16_TFLOPS if gemm_ms > 0 else None,
        "stage_ms": stage_ms,
        "stages": stages,
        # the same stages with L2 and MALL flushed before each call (HBM-bound
        # stages then read their inputs from HBM)
        "stages_flushed": {kname: v for kname, v in stage_rooflines(cfg, flushed_ms).items()
                           if kname in ("gate", "permute", "combine")},
    }
    result["cold_start"] = {
        "ms_per_step": cold_ms, "tokens_per_s": T / (cold_ms * 1e-3),
        "note": f"the same {args.warmup} warm-up + {args.steps} timed steps as the first GPU work of the process; "
                "the headline is timed after the other workloads, on the loaded GPU"}
    result.update(extra)
    if not args.no_autocast and args.config == "c3":
        fb = result.get("fwd_bwd")
        result["autocast"] = autocast_bench(dev, args.steps, args.warmup, ms,
                                            fb["ms_per_step"] if fb and args.fwd_bwd_config == "c4" else None)
    # the host-side baselines last: a GPU left idle for a second runs its next
    # few tens of steps at a lower clock, so no GPU figure is taken after them
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU restatement of the reference path ...")
        result["cpu_baseline"] = cpu_baseline(cfg, x, gate_w, bias, weights)
        result["speedup_vs_cpu"] = result["value"] / result["cpu_baseline"]["value"]
        if "mla" in result:
            result["mla"]["cpu_baseline"], result["mla"]["speedup_vs_cpu"] = mla_cpu_baseline(
                dev, result["mla"]["ms_per_call"])
        if "fwd_bwd" in result:
            del x, weights, w1, w2, w3, s1, s2, s3
            fcfg = CONFIGS[args.fwd_bwd_config]
            log("[bench] timing the CPU restatement of the reference path (fwd+bwd) ...")
            fx, fgw, fb_, fws = make_layer(fcfg, dev)
            fb = result["fwd_bwd"]
            fb["cpu_baseline"] = cpu_baseline(fcfg, fx, fgw, fb_, fws, budget_s=12.0, backward=True,
                                              min_tokens=fcfg[0])
            fb["speedup_vs_cpu"] = fb["value"] / fb["cpu_baseline"]["value"]
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
