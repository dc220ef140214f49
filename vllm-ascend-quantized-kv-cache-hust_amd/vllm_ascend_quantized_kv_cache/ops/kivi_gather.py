# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 gather-dequant (HIP kernel ``kvq_kivi_gather_dequant``).

``kivi_dequant_gather_cache`` keeps the signature, validation and output
contract of ``pkg/ops/kivi_gather.py:36-156``: dense ``[sum L, KVH, D]`` in
``target_dtype``, request order, bit-identical dequant (``q*scale`` then
``+mn``, then a round-to-nearest-even cast).  ``gather_dequant_with_residual``
is the fused form the attention mixin uses: the residual tail overlay of
``pkg/methods/kivi_int4/attention_backend.py:889-923`` happens in the same
kernel.
"""

from __future__ import annotations

import torch

from . import _native
from .kivi_layout import (
    _check_contiguous,
    _check_dequant_gather_metadata,
    _check_key_cache_layout,
    _check_same_device,
    _check_value_cache_layout,
)


def gather_dequant_with_residual(
    caches: tuple[torch.Tensor, ...],
    block_table: torch.Tensor,
    cu_seqlens: torch.Tensor,
    total_tokens: int,
    target_dtype: torch.dtype,
    group_size: int,
    ring_meta: torch.Tensor | None = None,
    ring_k: torch.Tensor | None = None,
    ring_v: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Launch the gather (no validation beyond shapes); optional ring overlay.

    ``ring_meta`` is int32 ``[B, 5]`` = (row, k_first_lane, k_tail,
    v_first_lane, v_tail) on the device.
    """
    kq, ks, km, vq, vs, vm = caches
    nb, kvh, d, pbs = kq.shape
    batch, max_blocks = block_table.shape
    dev = kq.device
    out_k = torch.empty((total_tokens, kvh, d), dtype=target_dtype, device=dev)
    out_v = torch.empty((total_tokens, kvh, d), dtype=target_dtype, device=dev)
    if total_tokens == 0 or batch == 0:
        return out_k, out_v
    _native.require_gpu_tensors(
        "kivi_dequant_gather_cache", kq, ks, km, vq, vs, vm, block_table, cu_seqlens,
        ring_meta, ring_k, ring_v,
    )
    ring_len = ring_k.shape[1] if ring_k is not None else 0
    rc = _native.lib().kvq_kivi_gather_dequant(
        _native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq), _native.ptr(vs),
        _native.ptr(vm), nb, pbs * 8, kvh, d, group_size, _native.ptr(block_table),
        _native.index_code(block_table.dtype), max_blocks, _native.ptr(cu_seqlens), batch,
        _native.ptr(ring_meta), _native.ptr(ring_k), _native.ptr(ring_v),
        _native.dtype_code(ring_k.dtype) if ring_k is not None else 0, ring_len,
        _native.ptr(out_k), _native.ptr(out_v), _native.dtype_code(target_dtype),
        _native.stream_of(kq),
    )
    _native.check(rc, "kvq_kivi_gather_dequant")
    return out_k, out_v


def kivi_dequant_gather_cache(
    k_quant_cache: torch.Tensor,
    k_scale_cache: torch.Tensor,
    k_mn_cache: torch.Tensor,
    v_quant_cache: torch.Tensor,
    v_scale_cache: torch.Tensor,
    v_mn_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    target_dtype: torch.dtype,
    group_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gather the live tokens of the paged int4 history and dequantize them."""
    if block_table.shape[0] != seq_lens.numel():
        block_table = block_table[: seq_lens.numel()]
    for name, t in (
        ("k_quant_cache", k_quant_cache),
        ("k_scale_cache", k_scale_cache),
        ("k_mn_cache", k_mn_cache),
        ("v_quant_cache", v_quant_cache),
        ("v_scale_cache", v_scale_cache),
        ("v_mn_cache", v_mn_cache),
    ):
        _check_contiguous(name, t)
    for name, t in (
        ("k_scale_cache", k_scale_cache),
        ("k_mn_cache", k_mn_cache),
        ("v_quant_cache", v_quant_cache),
        ("v_scale_cache", v_scale_cache),
        ("v_mn_cache", v_mn_cache),
        ("block_table", block_table),
        ("seq_lens", seq_lens),
    ):
        _check_same_device(name, t, k_quant_cache)
    num_blocks, num_kv_heads, head_size, packed = k_quant_cache.shape
    block_size = packed * 8
    if group_size % 8 != 0:
        raise RuntimeError(
            f"KIVI INT4 dequant requires group_size ({group_size}) to be divisible by 8."
        )
    _check_key_cache_layout(
        k_quant_cache, k_scale_cache, k_mn_cache,
        num_kv_heads=num_kv_heads, head_size=head_size, group_size=group_size,
    )
    _check_value_cache_layout(
        v_quant_cache, v_scale_cache, v_mn_cache,
        num_kv_heads=num_kv_heads, head_size=head_size, group_size=group_size,
    )
    if v_quant_cache.shape[0] != num_blocks or v_quant_cache.shape[1] != block_size:
        raise RuntimeError(
            "KIVI key/value cache block layout mismatch: "
            f"key num_blocks={num_blocks}, block_size={block_size}; "
            f"value shape={tuple(v_quant_cache.shape)}."
        )
    cu, _, total = _check_dequant_gather_metadata(
        block_table, seq_lens, num_blocks=num_blocks, block_size=block_size
    )
    return gather_dequant_with_residual(
        (k_quant_cache, k_scale_cache, k_mn_cache, v_quant_cache, v_scale_cache, v_mn_cache),
        block_table.contiguous(),
        cu,
        total,
        target_dtype,
        group_size,
    )


__all__ = ["gather_dequant_with_residual", "kivi_dequant_gather_cache"]
