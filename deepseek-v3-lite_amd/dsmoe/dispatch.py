"""Config compatibility for the reference's backend-selection keys.

The reference rewrites ``moe_dispatch='triton_grouped'`` to ``'stacked'``
unless ``ENABLE_TRITON_KERNELS=1`` (models/_triton_dispatch.py:13-35).  Here
there is one backend: ``DeepSeekMoE`` accepts any ``moe_dispatch`` value and
always runs the HIP kernels, so this helper keeps the reference's config
rewriting (callers that construct a model through it see the same config) but
selects nothing.
"""
from __future__ import annotations

import os
from typing import Callable

_DISPATCH = {
    ("attn_impl", "triton"): "sdpa",
    ("moe_dispatch", "triton_grouped"): "stacked",
}


def enforce_triton_env_var(model_cfg: dict, log: Callable[[str], None]) -> None:
    """Same config rewrite and single warning as models/_triton_dispatch.py:19-35."""
    if os.environ.get("ENABLE_TRITON_KERNELS", "0") == "1":
        return
    forced = []
    for (key, triton_val), default in _DISPATCH.items():
        if model_cfg.get(key) == triton_val:
            model_cfg[key] = default
            forced.append(f"{key}='{triton_val}' -> '{default}'")
    if forced:
        log("[warn] Triton dispatch keys set without ENABLE_TRITON_KERNELS=1; "
            f"forcing {', '.join(forced)}. Set ENABLE_TRITON_KERNELS=1 to enable the fused Triton paths.")


def next_pow2(n: int) -> int:
    """Smallest power of two >= n (models/_triton_dispatch.py:38-42)."""
    return 1 if n <= 1 else 1 << (n - 1).bit_length()
