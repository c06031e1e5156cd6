"""dsmoe — MI355X-native DeepSeekMoE layer hot path.

Drop-in for models/moe.py of atandra2000/DeepSeek-v3-Lite: ``DeepSeekMoE``,
``AuxLossFreeGate``, ``Expert`` and the grouped operator seam
``grouped_moe_dispatch`` (models/moe_triton.py:504-525), computed by the HIP
kernels of libdsmoe.so (csrc/).
"""
from .moe import AuxLossFreeGate, DeepSeekMoE, Expert, invalidate_weight_casts
from .ops import grouped_moe_dispatch, moe_layer
from .dispatch import enforce_triton_env_var, next_pow2

__all__ = ["AuxLossFreeGate", "DeepSeekMoE", "Expert", "grouped_moe_dispatch", "moe_layer",
           "enforce_triton_env_var", "next_pow2", "invalidate_weight_casts"]
