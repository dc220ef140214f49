# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head kernels (``kvq_fp8_pth_*``): the store and the read path.

The store keeps the reference wrapper's contract
(``pkg/ops/triton/per_token_head_store.py:30-110,221-294``): the same
validator and error texts, the same ``QUANT_PARAMS`` table, no launch for an
empty batch, the fp8 views of the data regions handed to the launch.  The
arithmetic is the reference semantics (``pkg/methods/fp8_per_token_head/
semantics.py:52-65``) computed by the HIP kernel: IEEE ``x / scale`` and
gfx950's round-to-nearest-even E4M3 conversion.

The read path has no counterpart in the reference (its scheme stops at the
store): ``fp8_per_token_head_dequant_gather`` turns paged codes into dense
TND rows exactly as ``dequantize`` then ``.to(dtype)`` would, and
``fp8_per_token_head_attention`` runs the MFMA attention kernel over them.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native

#: quantization range by cache dtype (the host kernel's table); only the fp8
#: row is routed, the int8 row is kept for the table's sake as in the reference
QUANT_PARAMS: dict[torch.dtype, tuple[float, float]] = {
    torch.float8_e4m3fn: (448.0, -448.0),
    torch.int8: (127.0, -128.0),
}


def _check_contiguous(name: str, tensor: torch.Tensor) -> None:
    if not tensor.is_contiguous():
        raise RuntimeError(f"fp8_per_token_head {name} must be contiguous.")


def _check_same_device(name: str, a: torch.Tensor, b: torch.Tensor) -> None:
    if a.device != b.device:
        raise RuntimeError(
            f"fp8_per_token_head {name} must share a device with the KV "
            f"tensors, got {a.device} and {b.device}."
        )


def validate_store_args(
    key: torch.Tensor,
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
) -> None:
    """Every layout check before a launch (``per_token_head_store.py:53-109``)."""
    num_tokens, num_kv_heads, head_size = key.shape
    if value.shape[0] != num_tokens or value.shape[1] != num_kv_heads:
        raise RuntimeError(
            "fp8_per_token_head key/value token-head grids must match, got "
            f"key {tuple(key.shape)} vs value {tuple(value.shape)}."
        )
    if value.shape[2] != head_size:
        raise RuntimeError(
            "fp8_per_token_head requires equal key/value head sizes, got "
            f"{head_size} vs {value.shape[2]}."
        )
    if head_size % 4:
        raise RuntimeError(
            f"fp8_per_token_head requires head_size divisible by 4 (fp32 "
            f"scale alignment), got {head_size}."
        )
    if slot_mapping.shape != (num_tokens,):
        raise RuntimeError(
            f"fp8_per_token_head slot_mapping must be 1D of {num_tokens} "
            f"slots, got {tuple(slot_mapping.shape)}."
        )
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(
            f"fp8_per_token_head slot_mapping must be int32/int64, got {slot_mapping.dtype}."
        )
    expected_data = (k_data.shape[0], k_data.shape[1], num_kv_heads, head_size)
    for name, data, scale in (("key", k_data, k_scale), ("value", v_data, v_scale)):
        _check_contiguous(f"{name} data", data)
        _check_contiguous(f"{name} scale", scale)
        _check_same_device(f"{name} data", data, key)
        _check_same_device(f"{name} scale", scale, key)
        if data.shape != expected_data or data.dtype is not torch.uint8:
            raise RuntimeError(
                f"fp8_per_token_head {name} data cache must be uint8 "
                f"{expected_data}, got {tuple(data.shape)} / {data.dtype}."
            )
        expected_scale = (data.shape[0], data.shape[1], num_kv_heads, 1)
        if scale.shape != expected_scale or scale.dtype is not torch.float32:
            raise RuntimeError(
                f"fp8_per_token_head {name} scale cache must be float32 "
                f"{expected_scale}, got {tuple(scale.shape)} / {scale.dtype}."
            )


def _launch_kernel(
    key: torch.Tensor,
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_data_fp8: torch.Tensor,
    k_scale: torch.Tensor,
    v_data_fp8: torch.Tensor,
    v_scale: torch.Tensor,
    quant_max: float,
    quant_min: float,
    is_int_quant: bool,
) -> None:
    """The launch (``per_token_head_store.py:221-258``): one HIP kernel."""
    if is_int_quant or (quant_max, quant_min) != QUANT_PARAMS[torch.float8_e4m3fn]:
        raise NotImplementedError(
            "fp8_per_token_head: only the E4M3 (448, -448) store is built; the int8 "
            "variant of the parameter table is not routed."
        )
    _native.require_gpu_tensors(
        "fp8_per_token_head_store", key, value, slot_mapping, k_data_fp8, k_scale, v_data_fp8,
        v_scale,
    )
    num_tokens, kvh, d = key.shape
    nb, bs = k_data_fp8.shape[0], k_data_fp8.shape[1]
    value = value if value.dtype == key.dtype else value.to(key.dtype)
    rc = _native.lib().kvq_fp8_pth_store(
        _native.ptr(key), _native.ptr(value.contiguous()), _native.dtype_code(key.dtype),
        _native.ptr(slot_mapping), _native.index_code(slot_mapping.dtype), num_tokens, kvh, d,
        _native.ptr(k_data_fp8), _native.ptr(k_scale), _native.ptr(v_data_fp8),
        _native.ptr(v_scale), nb, bs, _native.stream_of(key),
    )
    _native.check(rc, "kvq_fp8_pth_store")


def fp8_per_token_head_store(
    key: torch.Tensor,
    value: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
) -> None:
    """Write ``[T, KVH, D]`` K/V into the paged E4M3 cache by slot.

    ``k_data/v_data [NB, Bs, KVH, D]`` uint8 and ``k_scale/v_scale
    [NB, Bs, KVH, 1]`` fp32 are the views of ``fp8_caches_from_byte_tensors``.
    Negative slots are padding and skipped (``per_token_head_store.py:261-294``).
    """
    if key.numel() == 0:
        return
    validate_store_args(key, value, slot_mapping, k_data, k_scale, v_data, v_scale)
    if not key.is_contiguous():
        key = key.contiguous()
    quant_max, quant_min = QUANT_PARAMS[torch.float8_e4m3fn]
    _launch_kernel(
        key,
        value,
        slot_mapping.contiguous(),
        k_data.view(torch.float8_e4m3fn),
        k_scale,
        v_data.view(torch.float8_e4m3fn),
        v_scale,
        quant_max,
        quant_min,
        is_int_quant=False,
    )


def _check_live_blocks(rows, lens: list[int], *, max_blocks: int, num_blocks: int,
                       block_size: int) -> None:
    """Every live position's page id lies in ``[0, num_blocks)`` (host lists)."""
    longest = max(lens, default=0)
    if longest > max_blocks * block_size:
        raise RuntimeError(
            "fp8_per_token_head block_table does not cover the longest sequence: "
            f"max_seq_len={longest}, max_blocks={max_blocks}, block_size={block_size}."
        )
    table = np.asarray(rows, dtype=np.int64).reshape(-1, max_blocks)[: len(lens)]
    need = -(-np.asarray(lens, dtype=np.int64) // block_size)
    live = np.arange(max_blocks)[None, :] < need[:, None]
    if ((table < 0) & live).any():
        raise RuntimeError(
            "fp8_per_token_head block_table has invalid block ids for live tokens.")
    if ((table >= num_blocks) & live).any():
        raise RuntimeError(
            "fp8_per_token_head block_table references blocks outside the cache.")


def fp8_per_token_head_dequant_gather(
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    target_dtype: torch.dtype,
    *,
    block_table_host=None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged E4M3 -> dense TND ``[sum seq_lens, KVH, D]`` in ``target_dtype``.

    Element ``(p, h, i)`` of request ``b`` is ``float(code) * scale`` in fp32,
    rounded to ``target_dtype``, read from slot ``block_table[b, p // Bs] * Bs
    + p % Bs``.  Live block ids are checked on the host (``block_table_host``,
    or the table read back once when only a device copy is given).
    """
    nb, bs, kvh, d = k_data.shape
    for name, t in (("key data", k_data), ("key scale", k_scale), ("value data", v_data),
                    ("value scale", v_scale)):
        _check_contiguous(name, t)
        _check_same_device(name, t, k_data)
    if v_data.shape != k_data.shape or k_scale.shape != (nb, bs, kvh, 1) or (
            v_scale.shape != k_scale.shape):
        raise RuntimeError(
            "fp8_per_token_head cache views disagree: "
            f"k_data {tuple(k_data.shape)}, k_scale {tuple(k_scale.shape)}, "
            f"v_data {tuple(v_data.shape)}, v_scale {tuple(v_scale.shape)}."
        )
    lens = [int(n) for n in seq_lens]
    if block_table.dim() != 2 or block_table.shape[0] < len(lens):
        raise RuntimeError(
            f"fp8_per_token_head block_table must be 2D with a row per request, got "
            f"{tuple(block_table.shape)} for {len(lens)} requests."
        )
    table = block_table[: len(lens)]
    rows = block_table_host if block_table_host is not None else table.cpu().numpy()
    _check_live_blocks(rows, lens, max_blocks=table.shape[1], num_blocks=nb, block_size=bs)
    dev = k_data.device
    total = sum(lens)
    out_k = torch.empty((total, kvh, d), dtype=target_dtype, device=dev)
    out_v = torch.empty_like(out_k)
    if total == 0:
        return out_k, out_v
    _native.require_gpu_tensors("fp8_per_token_head_dequant_gather", k_data, table)
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    cu_t = torch.tensor(cu, dtype=torch.int64).to(dev, non_blocking=True)
    table = table.contiguous()
    rc = _native.lib().kvq_fp8_pth_gather(
        _native.ptr(k_data), _native.ptr(k_scale), _native.ptr(v_data), _native.ptr(v_scale),
        nb, bs, kvh, d, _native.ptr(table), _native.index_code(table.dtype), table.shape[1],
        _native.ptr(cu_t), len(lens), _native.ptr(out_k), _native.ptr(out_v),
        _native.dtype_code(target_dtype), _native.stream_of(k_data),
    )
    _native.check(rc, "kvq_fp8_pth_gather")
    return out_k, out_v


def fp8_per_token_head_attention(
    query: torch.Tensor,
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    query_lens: list[int],
    scale: float,
    *,
    causal: bool = True,
    out: torch.Tensor | None = None,
    block_table_host=None,
) -> torch.Tensor:
    """Attention of TND ``query [sum query_lens, Hq, D]`` over the paged E4M3
    history: each request's rows are its last ``query_lens[b]`` positions of
    ``seq_lens[b]`` (decode: ``query_lens`` all 1)."""
    from .attention import prefill_attention

    key, value = fp8_per_token_head_dequant_gather(
        k_data, k_scale, v_data, v_scale, block_table, seq_lens, query.dtype,
        block_table_host=block_table_host,
    )
    return prefill_attention(query, key, value, list(query_lens), list(seq_lens), scale, causal,
                             out=out)


__all__ = [
    "QUANT_PARAMS",
    "fp8_per_token_head_attention",
    "fp8_per_token_head_dequant_gather",
    "fp8_per_token_head_store",
    "validate_store_args",
]
