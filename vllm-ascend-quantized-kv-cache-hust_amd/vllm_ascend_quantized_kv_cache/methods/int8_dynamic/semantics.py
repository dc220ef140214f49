# SPDX-License-Identifier: Apache-2.0
"""Dynamic per-channel INT8 scheme: scales from the first K/V, symmetric codes.

Same contract as ``pkg/methods/int8_dynamic/semantics.py:22-95``:
``inv = 127 / amax(|x|)`` over tokens per (head, dim) with a 1e-12 floor,
offset 0, ``code = clamp(round(x*inv), -128, 127)``, ``x = code * (1/inv)``,
all in the activation dtype.  The arithmetic runs in the HIP kernels
(``ops.int8_ops``); this object takes GPU tensors.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch


@dataclass
class Int8DynamicScales:
    """Per-layer scales: ``*_inv_scale``/``*_offset`` are ``[1, H, D]``,
    the ``*_aq_*`` antiquant views ``[1, H, 1, D]``."""

    k_inv_scale: Any
    k_offset: Any
    v_inv_scale: Any
    v_offset: Any
    k_aq_scale: Any
    k_aq_offset: Any
    v_aq_scale: Any
    v_aq_offset: Any


class Int8DynamicSemantics:
    def __init__(self, config: Any) -> None:
        self.config = config

    def calc_scales(self, key: Any, value: Any) -> Int8DynamicScales:
        from ...ops.int8_ops import int8_calc_scales

        k_inv, v_inv, k_aq, v_aq = int8_calc_scales(key, value)
        return Int8DynamicScales(
            k_inv_scale=k_inv,
            k_offset=torch.zeros_like(k_inv),
            v_inv_scale=v_inv,
            v_offset=torch.zeros_like(v_inv),
            k_aq_scale=k_aq,
            k_aq_offset=torch.zeros_like(k_aq),
            v_aq_scale=v_aq,
            v_aq_offset=torch.zeros_like(v_aq),
        )

    @staticmethod
    def quantize(x: Any, inv_scale: Any, offset: Any = None) -> Any:
        """``[T, H, D]`` (or ``[T, H*D]``) activations -> int8 codes (offset is 0)."""
        from ...ops.int8_ops import int8_quantize

        return int8_quantize(x, inv_scale)

    @staticmethod
    def dequantize(x: Any, inv_scale: Any, offset: Any, target_dtype: Any) -> Any:
        from ...ops.int8_ops import int8_dequantize

        return int8_dequantize(x, inv_scale, target_dtype)

    def describe(self) -> dict[str, Any]:
        return {
            "scheme": "int8_dynamic_per_channel",
            "scale_shape": [1, self.config.num_kv_heads, self.config.head_size],
            "scale_axis": "token-amax (dim=0), computed on first prefill",
            "symmetric": True,
            "kernels": "HIP gfx950",
        }


__all__ = ["Int8DynamicScales", "Int8DynamicSemantics"]
