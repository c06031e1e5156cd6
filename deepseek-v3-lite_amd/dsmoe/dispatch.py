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

# The MoE layer's key only; the attention key the reference rewrites too
# belongs to MLA attention, which this package does not provide.
_REWRITES = {("moe_dispatch", "triton_grouped"): "stacked"}


def enforce_triton_env_var(model_cfg: dict, log: Callable[[str], None]) -> None:
    """Config rewrite of models/_triton_dispatch.py:19-35 for the MoE key:
    without ENABLE_TRITON_KERNELS=1 a 'triton_grouped' dispatch becomes
    'stacked', announced by one log call per rewritten config."""
    if os.environ.get("ENABLE_TRITON_KERNELS", "0") == "1":
        return
    changed = []
    for (key, value), replacement in _REWRITES.items():
        if model_cfg.get(key) == value:
            model_cfg[key] = replacement
            changed.append(f"{key}: {value!r} becomes {replacement!r}")
    if changed:
        log("[warn] ENABLE_TRITON_KERNELS is not 1, so the config's Triton selections are reset ("
            + "; ".join(changed) + "). The dsmoe layer runs its HIP kernels under either value.")


def next_pow2(n: int) -> int:
    """Smallest power of two >= n (models/_triton_dispatch.py:38-42)."""
    return 1 if n <= 1 else 1 << (n - 1).bit_length()
