# SPDX-License-Identifier: Apache-2.0
"""Layer 0 contract: cache-dtype literal -> quantization mode -> storage layout.

Pure Python, importable without torch.  Mirrors the reference contract
(``src/vllm_ascend_quantized_kv_cache/dtypes.py:15-94``): the enum values are
shared with the host, so they are kept identical.  Unknown literals fail
closed.
"""

from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum


class KVQuantMode(IntEnum):
    """Quantization modes; numeric values match the host's legacy enum."""

    NONE = 0
    INT8_PER_TENSOR = 8
    KIVI_INT4 = 9
    FP8_PER_TOKEN_HEAD = 10


_MODE_BY_LITERAL = {
    "int8": KVQuantMode.INT8_PER_TENSOR,
    "kivi_int4": KVQuantMode.KIVI_INT4,
    "fp8_per_token_head": KVQuantMode.FP8_PER_TOKEN_HEAD,
}


def get_kv_quant_mode(dtype: str) -> KVQuantMode:
    """Map a ``--kv-cache-dtype`` literal to its mode (``NONE`` if unknown)."""
    return _MODE_BY_LITERAL.get(dtype, KVQuantMode.NONE)


def is_quantized_kv_cache(dtype: str) -> bool:
    return get_kv_quant_mode(dtype) is not KVQuantMode.NONE


def int4_packed_dim(head_size: int) -> int:
    """Bytes per head row once two int4 codes share a byte."""
    if head_size <= 0 or head_size % 2:
        raise ValueError("INT4 head_size must be a positive even number")
    return head_size // 2


@dataclass(frozen=True)
class KVCacheLayout:
    """Resolved storage layout of one cache dtype (immutable)."""

    dtype: str
    head_size: int
    storage_dtype: str
    packed_last_dim: int
    quant_mode: KVQuantMode


def resolve_layout(dtype: str, head_size: int) -> KVCacheLayout:
    """Storage layout for a quantized cache literal; raises for anything else."""
    mode = get_kv_quant_mode(dtype)
    if mode is KVQuantMode.INT8_PER_TENSOR:
        if head_size <= 0:
            raise ValueError("head_size must be positive")
        return KVCacheLayout(dtype, head_size, "int8", head_size, mode)
    if mode is KVQuantMode.KIVI_INT4:
        return KVCacheLayout(dtype, head_size, "uint8", int4_packed_dim(head_size), mode)
    if mode is KVQuantMode.FP8_PER_TOKEN_HEAD:
        if head_size <= 0 or head_size % 4:
            raise ValueError(
                "fp8_per_token_head requires head_size positive and divisible "
                f"by 4 (fp32 scale alignment), got {head_size}"
            )
        return KVCacheLayout(dtype, head_size, "uint8", head_size, mode)
    raise ValueError(f"dtype is not a registered quantized KV layout: {dtype}")


__all__ = [
    "KVCacheLayout",
    "KVQuantMode",
    "get_kv_quant_mode",
    "int4_packed_dim",
    "is_quantized_kv_cache",
    "resolve_layout",
]
