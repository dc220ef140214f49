# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head byte-region layout: the host's two byte buffers as four views.

As for KIVI, the host hands each layer two equal byte buffers and the plugin
cuts views out of them without copying; each side here has two regions, laid
out back to back::

    K: k_data uint8 [NB, Bs, KVH, D] | k_scale fp32 [NB, Bs, KVH, 1]
    V: v_data uint8 [NB, Bs, KVH, D] | v_scale fp32 [NB, Bs, KVH, 1]

so a (token, head) costs ``S = D + 4`` bytes per side, the host's page budget
for the literal (data ``2*Bs*KVH*D`` plus scales ``2*Bs*KVH*4`` per page).
The format and the error texts are the reference's
(``pkg/methods/fp8_per_token_head/byte_cache.py:13-197``): the host sizes its
buffers from it and the HIP store / gather kernels address the same bytes.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import prod
from typing import Any

import torch

from ...ops.kivi_layout import _check_contiguous

Spec = tuple[tuple[int, ...], torch.dtype]


@dataclass(frozen=True)
class Fp8PerTokenHeadLayout:
    """Shape of one fp8_per_token_head paged allocation and how it splits."""

    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int

    def __post_init__(self) -> None:
        if self.num_blocks <= 0:
            raise ValueError(f"num_blocks must be positive, got {self.num_blocks}")
        if self.head_size <= 0 or self.head_size % 4:
            raise ValueError(
                "fp8_per_token_head requires head_size positive and divisible "
                f"by 4, got {self.head_size}"
            )

    def side_specs(self) -> tuple[Spec, ...]:
        nb, bs, h, d = self.num_blocks, self.block_size, self.num_kv_heads, self.head_size
        return (((nb, bs, h, d), torch.uint8), ((nb, bs, h, 1), torch.float32))

    # keys and values split the same way, so the two host buffers are equal
    key_specs = side_specs
    value_specs = side_specs

    @property
    def bytes_per_token_head(self) -> int:
        """One side, one (token, head): E4M3 codes plus the fp32 scale."""
        return self.head_size + 4

    @property
    def region_bytes(self) -> int:
        """Bytes of one host buffer (the same for keys and values)."""
        return self.num_blocks * self.block_size * self.num_kv_heads * self.bytes_per_token_head

    def compression_vs_fp16(self) -> float:
        """One side's size against dense fp16 K or V."""
        return (2 * self.head_size) / self.bytes_per_token_head

    def describe(self) -> dict[str, Any]:
        return {
            "region_bytes": self.region_bytes,
            "bytes_per_token": 2 * self.num_kv_heads * self.bytes_per_token_head,
            "compression_vs_fp16": self.compression_vs_fp16(),
            "side": [
                {"shape": list(shape), "dtype": str(dtype).replace("torch.", "")}
                for shape, dtype in self.side_specs()
            ],
        }


def fp8_per_token_head_layout(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    *,
    num_kv_heads: int,
    head_size: int,
) -> Fp8PerTokenHeadLayout:
    """Infer the page layout from the host's buffers (fails closed).

    ``block_size = bytes / (num_blocks * KVH * (D + 4))`` must come out whole.
    """
    _check_contiguous("key_cache", key_cache)
    _check_contiguous("value_cache", value_cache)
    if key_cache.device != value_cache.device:
        raise RuntimeError(
            f"fp8_per_token_head key/value caches must share a device, got "
            f"{key_cache.device} and {value_cache.device}."
        )
    kb = key_cache.numel() * key_cache.element_size()
    vb = value_cache.numel() * value_cache.element_size()
    if kb != vb:
        raise RuntimeError(
            f"fp8_per_token_head key cache holds {kb} bytes but value "
            f"cache holds {vb}; the layout needs equal regions."
        )
    nb = int(key_cache.shape[0])
    stride = nb * num_kv_heads * (head_size + 4)
    if stride <= 0 or kb % stride:
        raise RuntimeError(
            f"fp8_per_token_head cache region of {kb} bytes is not a "
            f"whole number of pages for head_size={head_size}, "
            f"num_kv_heads={num_kv_heads}, num_blocks={nb}."
        )
    return Fp8PerTokenHeadLayout(nb, kb // stride, num_kv_heads, head_size)


def _views_for_region(
    cache: torch.Tensor, specs: tuple[Spec, ...], region_bytes: int, name: str
) -> list[torch.Tensor]:
    if not cache.is_contiguous():
        raise RuntimeError(f"fp8_per_token_head {name} cache must be contiguous.")
    have = cache.numel() * cache.element_size()
    if have != region_bytes:
        raise RuntimeError(
            f"fp8_per_token_head {name} cache must hold {region_bytes} bytes, got {have}."
        )
    flat = cache.reshape(-1).view(torch.uint8)
    views, offset = [], 0
    for shape, dtype in specs:
        span = prod(shape) * dtype.itemsize
        views.append(flat.narrow(0, offset, span).view(dtype).view(shape))
        offset += span
    if offset != flat.numel():
        raise RuntimeError(
            f"fp8_per_token_head {name} region bookkeeping error: {offset} vs "
            f"{flat.numel()} bytes."
        )
    return views


def fp8_caches_from_byte_tensors(
    key_cache: torch.Tensor, value_cache: torch.Tensor, layout: Fp8PerTokenHeadLayout
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Two host buffers -> ``(k_data, k_scale, v_data, v_scale)``."""
    region = layout.region_bytes
    return (
        *_views_for_region(key_cache, layout.key_specs(), region, "key"),
        *_views_for_region(value_cache, layout.value_specs(), region, "value"),
    )


__all__ = ["Fp8PerTokenHeadLayout", "fp8_caches_from_byte_tensors", "fp8_per_token_head_layout"]
