# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head scheme: E4M3 codes with a dynamic fp32 scale per (token, head).

Same contract as ``pkg/methods/fp8_per_token_head/semantics.py:36-82``::

    scale = max(amax(|x|) / 448, 1e-6)          # 448: largest e4m3fn normal
    q     = e4m3fn(clamp(x / scale, -448, 448))  # round to nearest even
    x_hat = float(q) * scale

The arithmetic runs in the HIP kernels (``ops.fp8_ops``); this object takes
GPU tensors.  ``quantize`` writes the codes through the paged store kernel into
a one-page layout (slot t = token t) and ``dequantize`` reads them back
through the gather kernel, so these calls and the paged cache share one code
path.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

E4M3_MAX = 448.0
#: the fp32 rounding of 1e-6, the scale floor of the host kernel
SCALE_FLOOR = 1e-6


class Fp8PerTokenHeadSemantics:
    e4m3_max = E4M3_MAX

    def __init__(self, config: Any) -> None:
        head_size = getattr(config, "head_size", None)
        if not isinstance(head_size, int) or head_size <= 0 or head_size % 4:
            raise ValueError(
                "fp8_per_token_head requires head_size positive and divisible "
                f"by 4 (fp32 scale alignment), got {head_size!r}"
            )
        self.head_size = head_size

    def compute_scale(self, values: torch.Tensor) -> torch.Tensor:
        """``[T, KVH, D] -> [T, KVH, 1]`` fp32 scales."""
        return self.quantize(values)[1]

    def quantize(self, values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """``[T, KVH, D]`` -> (``float8_e4m3fn [T, KVH, D]``, fp32 ``[T, KVH, 1]``)."""
        from ...ops.fp8_ops import fp8_per_token_head_store

        t, kvh, d = values.shape
        dev = values.device
        data = torch.empty((2, 1, max(t, 1), kvh, d), dtype=torch.uint8, device=dev)
        scale = torch.empty((2, 1, max(t, 1), kvh, 1), dtype=torch.float32, device=dev)
        if t:
            slots = torch.arange(t, dtype=torch.int64, device=dev)
            x = values.contiguous()
            fp8_per_token_head_store(x, x, slots, data[0], scale[0], data[1], scale[1])
        return data[0, 0, :t].view(torch.float8_e4m3fn), scale[0, 0, :t]

    def dequantize(self, packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """(E4M3 codes, scales) -> dense fp32 ``[T, KVH, D]``."""
        from ...ops.fp8_ops import fp8_per_token_head_dequant_gather

        t, kvh, d = packed.shape
        if t == 0:
            return torch.empty((0, kvh, d), dtype=torch.float32, device=packed.device)
        data = packed.contiguous().view(torch.uint8).view(1, t, kvh, d)
        sc = scale.to(torch.float32).contiguous().view(1, t, kvh, 1)
        table = torch.zeros((1, 1), dtype=torch.int32, device=packed.device)
        out, _ = fp8_per_token_head_dequant_gather(
            data, sc, data, sc, table, [t], torch.float32,
            block_table_host=np.zeros((1, 1), dtype=np.int64),
        )
        return out

    def fake_quant(self, values: torch.Tensor) -> torch.Tensor:
        """Write-then-read round trip, in the input dtype."""
        packed, scale = self.quantize(values)
        return self.dequantize(packed, scale).to(values.dtype)

    def describe(self) -> dict[str, Any]:
        return {
            "scheme": "fp8_per_token_head",
            "bits": 8,
            "encoding": "e4m3fn (max normal 448)",
            "scale_granularity": "per (token, head), fp32, dynamic",
            "calibration": "none (online amax)",
        }


__all__ = ["E4M3_MAX", "SCALE_FLOOR", "Fp8PerTokenHeadSemantics"]
