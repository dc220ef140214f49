# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 byte-region layout: the host's two byte buffers as six views.

The host hands each attention layer two equal byte buffers (keys, values).
Each is cut, without copying, into ``[quant int32 | scale fp32 | min fp32]``
regions laid out back to back (not interleaved per page)::

    K: k_quant [NB, KVH, D, Bs/8] | k_scale [NB, KVH, D, Bs/G] | k_mn (same)
    V: v_quant [NB, Bs, KVH, D/8] | v_scale [NB, Bs, KVH, D/G] | v_mn (same)

so one token of one head costs ``S = D/2 + 8*D/G`` bytes per side.  The byte
format is the reference's (``pkg/methods/kivi_int4/byte_cache.py:32-223``),
kept identical because the host sizes its buffers from it and the MI355X
kernels read the same bytes; the error texts are the ones callers match.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import prod
from typing import Any

import torch

from ...ops.kivi_layout import _check_contiguous
from .geometry import validate_kivi_geometry

_LANES_PER_WORD = 8

Spec = tuple[tuple[int, ...], torch.dtype]


@dataclass(frozen=True)
class KiviByteCacheLayout:
    """Shape of one KIVI paged allocation and how its two buffers split."""

    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    group_size: int

    def __post_init__(self) -> None:
        if self.num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {self.num_blocks}")
        validate_kivi_geometry(
            head_size=self.head_size,
            group_size=self.group_size,
            residual_length=self.group_size,
            block_size=self.block_size,
        )

    def key_specs(self) -> tuple[Spec, ...]:
        nb, h, d, bs, g = (self.num_blocks, self.num_kv_heads, self.head_size,
                           self.block_size, self.group_size)
        return (
            ((nb, h, d, bs // _LANES_PER_WORD), torch.int32),
            ((nb, h, d, bs // g), torch.float32),
            ((nb, h, d, bs // g), torch.float32),
        )

    def value_specs(self) -> tuple[Spec, ...]:
        nb, h, d, bs, g = (self.num_blocks, self.num_kv_heads, self.head_size,
                           self.block_size, self.group_size)
        return (
            ((nb, bs, h, d // _LANES_PER_WORD), torch.int32),
            ((nb, bs, h, d // g), torch.float32),
            ((nb, bs, h, d // g), torch.float32),
        )

    @property
    def key_bytes(self) -> int:
        return _specs_bytes(self.key_specs())

    @property
    def value_bytes(self) -> int:
        return _specs_bytes(self.value_specs())

    @property
    def region_bytes(self) -> int:
        """Bytes of one buffer; both sides must match for two buffers to suffice."""
        if self.key_bytes != self.value_bytes:
            raise RuntimeError(
                "KIVI byte layout requires equal key/value regions, got "
                f"{self.key_bytes} vs {self.value_bytes}."
            )
        return self.key_bytes

    @property
    def bytes_per_token_head(self) -> int:
        """``S``: int4 data plus the amortised fp32 scale and min, one side."""
        return self.head_size // 2 + 8 * self.head_size // self.group_size

    @property
    def bytes_per_token(self) -> int:
        return 2 * self.num_kv_heads * self.bytes_per_token_head

    @property
    def page_size_bytes(self) -> int:
        """Both sides of one block: what the host budgets per page."""
        return 2 * self.block_size * self.num_kv_heads * self.bytes_per_token_head

    def compression_vs_fp16(self) -> float:
        return (2 * self.num_kv_heads * self.head_size * 2) / self.bytes_per_token

    def describe(self) -> dict[str, Any]:
        def summary(specs):
            return [{"shape": list(s), "dtype": str(t).replace("torch.", "")} for s, t in specs]

        return {
            "region_bytes": self.region_bytes,
            "bytes_per_token": self.bytes_per_token,
            "compression_vs_fp16": self.compression_vs_fp16(),
            "key": summary(self.key_specs()),
            "value": summary(self.value_specs()),
        }


def _specs_bytes(specs: tuple[Spec, ...]) -> int:
    return sum(prod(shape) * dtype.itemsize for shape, dtype in specs)


def kivi_byte_cache_layout(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    *,
    num_kv_heads: int,
    head_size: int,
    group_size: int,
) -> KiviByteCacheLayout:
    """Infer the page layout from the host's buffers (fails closed).

    ``block_size = bytes / (num_blocks * KVH * S)`` must come out whole.
    """
    _check_contiguous("key_cache", key_cache)
    _check_contiguous("value_cache", value_cache)
    if key_cache.device != value_cache.device:
        raise RuntimeError(
            f"KIVI key/value caches must share a device, got {key_cache.device} "
            f"and {value_cache.device}."
        )
    kb = key_cache.numel() * key_cache.element_size()
    vb = value_cache.numel() * value_cache.element_size()
    if kb != vb:
        raise RuntimeError(
            f"KIVI key cache holds {kb} bytes but value cache holds {vb}; "
            "the int4 layout needs equal regions."
        )
    nb = int(key_cache.shape[0])
    s = head_size // 2 + 8 * head_size // group_size
    stride = nb * num_kv_heads * s
    if stride <= 0 or kb % stride:
        raise RuntimeError(
            f"KIVI cache region of {kb} bytes is not a whole number of pages for "
            f"head_size={head_size}, group_size={group_size}, "
            f"num_kv_heads={num_kv_heads}, num_blocks={nb}."
        )
    return KiviByteCacheLayout(nb, kb // stride, num_kv_heads, head_size, group_size)


def _views_for_region(
    cache: torch.Tensor, specs: tuple[Spec, ...], region_bytes: int, name: str
) -> list[torch.Tensor]:
    if not cache.is_contiguous():
        raise RuntimeError(f"KIVI {name} cache must be contiguous.")
    have = cache.numel() * cache.element_size()
    if have != region_bytes:
        raise RuntimeError(f"KIVI {name} cache must hold {region_bytes} bytes, got {have}.")
    flat = cache.reshape(-1).view(torch.uint8)
    views, offset = [], 0
    for shape, dtype in specs:
        span = prod(shape) * dtype.itemsize
        views.append(flat.narrow(0, offset, span).view(dtype).view(shape))
        offset += span
    return views


def kivi_caches_from_byte_tensors(
    key_cache: torch.Tensor, value_cache: torch.Tensor, layout: KiviByteCacheLayout
) -> tuple[torch.Tensor, ...]:
    """Two host buffers -> ``(k_quant, k_scale, k_mn, v_quant, v_scale, v_mn)``."""
    region = layout.region_bytes
    return (
        *_views_for_region(key_cache, layout.key_specs(), region, "key"),
        *_views_for_region(value_cache, layout.value_specs(), region, "value"),
    )


__all__ = ["KiviByteCacheLayout", "kivi_byte_cache_layout", "kivi_caches_from_byte_tensors"]
