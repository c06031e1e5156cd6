"""Config compatibility for the reference's backend-selection keys.

The reference rewrites ``moe_dispatch='triton_grouped'`` to ``'stacked'`` and
``attn_impl='triton'`` to ``'sdpa'`` unless ``ENABLE_TRITON_KERNELS=1``
(models/_triton_dispatch.py:13-35), at ``Transformer`` construction
(models/transformer.py:48).  Here the MoE layer has one backend:
``DeepSeekMoE`` accepts any ``moe_dispatch`` value and always runs the HIP
kernels.  The attention key still selects in the reference's layer
(models/mla.py:136-172): only ``attn_impl='triton'`` calls the fused operator,
which ``dsmoe.mla.triton_mla_attention`` replaces, so a model that should run
the HIP attention kernels is built with ``ENABLE_TRITON_KERNELS=1``.  This
helper keeps the reference's rewriting so callers see the same config.
"""
from __future__ import annotations

import os
from typing import Callable

# Each Triton selection and the portable default it is reset to.
_REWRITES = {("attn_impl", "triton"): "sdpa", ("moe_dispatch", "triton_grouped"): "stacked"}


def enforce_triton_env_var(model_cfg: dict, log: Callable[[str], None]) -> None:
    """Config rewrite of models/_triton_dispatch.py:19-35: without
    ENABLE_TRITON_KERNELS=1 a 'triton_grouped' MoE dispatch becomes 'stacked'
    and a 'triton' attention becomes 'sdpa', announced by one log call per
    rewritten config."""
    if os.environ.get("ENABLE_TRITON_KERNELS", "0") == "1":
        return
    changed = []
    for (key, value), replacement in _REWRITES.items():
        if model_cfg.get(key) == value:
            model_cfg[key] = replacement
            changed.append(f"{key}: {value!r} becomes {replacement!r}")
    if changed:
        log("[warn] ENABLE_TRITON_KERNELS is not 1, so the config's Triton selections are reset ("
            + "; ".join(changed) + "). The dsmoe MoE layer runs its HIP kernels under either value; the "
            "attention reaches the fused operator only with ENABLE_TRITON_KERNELS=1.")


def next_pow2(n: int) -> int:
    """Smallest power of two >= n (models/_triton_dispatch.py:38-42)."""
    return 1 if n <= 1 else 1 << (n - 1).bit_length()
