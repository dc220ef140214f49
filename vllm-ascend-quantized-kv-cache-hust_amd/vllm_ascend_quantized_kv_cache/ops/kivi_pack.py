# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 pack entry points (HIP kernels ``kvq_kivi_pack_key/value``).

``kivi_pack_key_cache`` / ``kivi_pack_value_cache`` keep the signatures and the
validation order of ``pkg/ops/triton/kivi_pack.py:229-348``; the mixin's
residual flushes use ``pack_key_rows`` / ``pack_value_rows``, which read token
rows through an index over two sources (the residual ring and the step's
input) so no staging copy is made.
"""

from __future__ import annotations

import torch

from . import _native
from .kivi_layout import (
    _check_contiguous,
    _check_key_cache_layout,
    _check_key_slot_groups,
    _check_same_device,
    _check_slot_mapping,
    _check_value_cache_layout,
)


def pack_key_rows(
    src_a: torch.Tensor,
    src_b: torch.Tensor | None,
    src_index: torch.Tensor | None,
    slots: torch.Tensor,
    k_quant: torch.Tensor,
    k_scale: torch.Tensor,
    k_mn: torch.Tensor,
    group_size: int,
) -> None:
    """Launch the key pack over ``slots.numel()`` tokens (no validation).

    Token ``t`` reads row ``src_index[t]`` (or ``t``) of ``src_a`` viewed as
    ``[n_a, KVH, D]``, rows past ``n_a`` continue into ``src_b``.
    """
    n = slots.numel()
    if n == 0:
        return
    _native.require_gpu_tensors("kivi_pack_key", src_a, src_b, src_index, slots, k_quant)
    nb, kvh, d, pbs = k_quant.shape
    n_a = src_a.numel() // (kvh * d)
    rc = _native.lib().kvq_kivi_pack_key(
        _native.ptr(src_a), n_a, _native.ptr(src_b), _native.ptr(src_index),
        _native.dtype_code(src_a.dtype), _native.ptr(slots), _native.index_code(slots.dtype),
        n, kvh, d, group_size, pbs * 8, _native.ptr(k_quant), _native.ptr(k_scale),
        _native.ptr(k_mn), _native.stream_of(k_quant),
    )
    _native.check(rc, "kvq_kivi_pack_key")


def pack_value_rows(
    src_a: torch.Tensor,
    src_b: torch.Tensor | None,
    src_index: torch.Tensor | None,
    slots: torch.Tensor,
    v_quant: torch.Tensor,
    v_scale: torch.Tensor,
    v_mn: torch.Tensor,
    group_size: int,
) -> None:
    """Launch the value pack over ``slots.numel()`` tokens (no validation)."""
    n = slots.numel()
    if n == 0:
        return
    _native.require_gpu_tensors("kivi_pack_value", src_a, src_b, src_index, slots, v_quant)
    nb, bs, kvh, words = v_quant.shape
    d = words * 8
    n_a = src_a.numel() // (kvh * d)
    rc = _native.lib().kvq_kivi_pack_value(
        _native.ptr(src_a), n_a, _native.ptr(src_b), _native.ptr(src_index),
        _native.dtype_code(src_a.dtype), _native.ptr(slots), _native.index_code(slots.dtype),
        n, kvh, d, group_size, bs, _native.ptr(v_quant), _native.ptr(v_scale),
        _native.ptr(v_mn), _native.stream_of(v_quant),
    )
    _native.check(rc, "kvq_kivi_pack_value")


def kivi_pack_value_cache(
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    v_quant_cache: torch.Tensor,
    v_scale_cache: torch.Tensor,
    v_mn_cache: torch.Tensor,
    group_size: int,
) -> None:
    """Pack ``value [T, KVH, D]`` into the paged int4 value cache (in place)."""
    num_tokens, num_kv_heads, head_size = value.shape
    if num_tokens == 0:
        return
    if group_size % 8 or head_size % group_size or head_size % 8:
        raise RuntimeError(
            f"KIVI value pack requires group_size % 8 == 0 and head_size % group_size == 0, "
            f"got head_size={head_size}, group_size={group_size}."
        )
    for name, t in (
        ("value", value),
        ("slot_mapping", slot_mapping),
        ("v_quant_cache", v_quant_cache),
        ("v_scale_cache", v_scale_cache),
        ("v_mn_cache", v_mn_cache),
    ):
        _check_contiguous(name, t)
    _check_same_device("slot_mapping", slot_mapping, value)
    _check_same_device("v_quant_cache", v_quant_cache, value)
    _check_same_device("v_scale_cache", v_scale_cache, value)
    _check_same_device("v_mn_cache", v_mn_cache, value)
    _check_slot_mapping(slot_mapping, num_tokens)
    _check_value_cache_layout(
        v_quant_cache, v_scale_cache, v_mn_cache,
        num_kv_heads=num_kv_heads, head_size=head_size, group_size=group_size,
    )
    pack_value_rows(
        value, None, None, slot_mapping, v_quant_cache, v_scale_cache, v_mn_cache, group_size
    )


def kivi_pack_key_cache(
    key: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_quant_cache: torch.Tensor,
    k_scale_cache: torch.Tensor,
    k_mn_cache: torch.Tensor,
    group_size: int,
) -> None:
    """Pack ``key [T, KVH, D]`` (T a multiple of ``group_size``) into the key cache."""
    num_tokens, num_kv_heads, head_size = key.shape
    if num_tokens == 0:
        return
    if group_size % 8 or num_tokens % group_size or head_size % 8:
        raise RuntimeError(
            "KIVI key pack requires group_size % 8 == 0, whole token groups and "
            f"head_size % 8 == 0, got T={num_tokens}, group_size={group_size}, "
            f"head_size={head_size}."
        )
    for name, t in (
        ("key", key),
        ("slot_mapping", slot_mapping),
        ("k_quant_cache", k_quant_cache),
        ("k_scale_cache", k_scale_cache),
        ("k_mn_cache", k_mn_cache),
    ):
        _check_contiguous(name, t)
    _check_same_device("slot_mapping", slot_mapping, key)
    _check_same_device("k_quant_cache", k_quant_cache, key)
    _check_same_device("k_scale_cache", k_scale_cache, key)
    _check_same_device("k_mn_cache", k_mn_cache, key)
    _check_slot_mapping(slot_mapping, num_tokens)
    block_size = _check_key_cache_layout(
        k_quant_cache, k_scale_cache, k_mn_cache,
        num_kv_heads=num_kv_heads, head_size=head_size, group_size=group_size,
    )
    _check_key_slot_groups(slot_mapping, block_size=block_size, group_size=group_size)
    pack_key_rows(
        key, None, None, slot_mapping, k_quant_cache, k_scale_cache, k_mn_cache, group_size
    )


def ring_write(
    ring: torch.Tensor,
    src: torch.Tensor,
    src_rows: torch.Tensor | None,
    dst_rows: torch.Tensor,
) -> None:
    """``ring.view(-1, KVH, D)[dst_rows[i]] = src[src_rows[i]]`` (dtype converted)."""
    n = dst_rows.numel()
    if n == 0:
        return
    _native.require_gpu_tensors("kivi ring write", ring, src, src_rows, dst_rows)
    row_elems = ring.shape[-1] * ring.shape[-2]
    rc = _native.lib().kvq_kivi_ring_write(
        _native.ptr(src.contiguous()), _native.dtype_code(src.dtype), _native.ptr(src_rows),
        _native.ptr(dst_rows), n, row_elems, _native.ptr(ring), _native.dtype_code(ring.dtype),
        _native.stream_of(ring),
    )
    _native.check(rc, "kvq_kivi_ring_write")


def store_one_launch_supported(head_size: int, group_size: int, dtype: torch.dtype) -> bool:
    """Geometries ``kvq_kivi_store`` runs (the others use the separate launches)."""
    return head_size == 128 and group_size in (64, 128) and dtype in (torch.bfloat16, torch.float16)


def kivi_store(
    key_input: torch.Tensor | None,
    value_input: torch.Tensor | None,
    ring_k: torch.Tensor,
    ring_v: torch.Tensor,
    jobs: torch.Tensor,
    counts: tuple[int, int, int, int],
    caches: tuple[torch.Tensor, ...],
    group_size: int,
) -> bool:
    """Key pack, value pack and both ring writes of a store batch in one launch.

    ``jobs`` (int64, on the device) and ``counts`` come from
    ``StorePlan.one_launch_jobs``; inputs are ``[n, KVH, D]`` contiguous in the
    ring dtype.  Returns False (nothing launched) for a geometry the one-launch
    kernel does not cover.
    """
    kq, ks, km, vq, vs, vm = caches
    nb, kvh, d, pbs = kq.shape
    if not store_one_launch_supported(d, group_size, ring_k.dtype):
        return False
    if sum(counts) == 0:
        return True
    _native.require_gpu_tensors("kivi store", ring_k, ring_v, jobs, kq, key_input, value_input)
    rc = _native.lib().kvq_kivi_store(
        _native.ptr(key_input), _native.ptr(value_input), _native.ptr(ring_k),
        _native.ptr(ring_v), ring_k.shape[0] * ring_k.shape[1], _native.dtype_code(ring_k.dtype),
        kvh, d, group_size, pbs * 8, _native.ptr(jobs), *counts,
        _native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq), _native.ptr(vs),
        _native.ptr(vm), _native.stream_of(ring_k),
    )
    _native.check(rc, "kvq_kivi_store")
    return True


__all__ = [
    "kivi_pack_key_cache",
    "kivi_pack_value_cache",
    "kivi_store",
    "pack_key_rows",
    "pack_value_rows",
    "ring_write",
    "store_one_launch_supported",
]
