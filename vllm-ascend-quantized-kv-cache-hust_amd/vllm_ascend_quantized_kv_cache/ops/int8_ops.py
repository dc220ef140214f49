# SPDX-License-Identifier: Apache-2.0
"""INT8 dynamic per-channel kernels (``kvq_int8_*``).

Scales, quantize+scatter, paged dequant and fused decode of
``pkg/methods/int8_dynamic/attention_backend.py:130-205,370-404``.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native

#: INT8 decode waves per CU the default plan aims at.  Up to 8 KV heads, the
#: kernel runs all heads of an item as one workgroup kept in step (one tile
#: buffer pair per head, 8 x 16 KB of LDS: one such workgroup per CU), so the
#: plan aims at one item per CU: on config 2 (64 x 4096 tokens, 8 KV heads)
#: items of 1024 positions decode in 101 us against 130 us for 2048 (two
#: rounds) and 246-288 us for 4096.  With more heads the kernel runs one wave
#: per head, and 4 waves per CU were best (2048-position items: 112 us, against
#: 119 us for 1024, 130 us for 1536 and 169 us for 4096).
INT8_DECODE_WAVES_PER_CU = 4
INT8_DECODE_WAVES_PER_CU_GROUPED = 8


def int8_split_tokens(total_positions: int, num_kv_heads: int, cu_count: int = 256,
                      seq_lens=None) -> int:
    """Positions per INT8 decode item: about INT8_DECODE_WAVES_PER_CU waves
    per CU (INT8_DECODE_WAVES_PER_CU_GROUPED for up to 8 KV heads, one
    workgroup per item), in [256, 4096], a multiple of 128.  With ``seq_lens``
    the split grows until the requests, each cut on its own, make no more
    items than that: a partial second round of workgroups costs more than
    longer items."""
    waves = INT8_DECODE_WAVES_PER_CU_GROUPED if num_kv_heads <= 8 else INT8_DECODE_WAVES_PER_CU
    target_items = max(1, (cu_count * waves) // max(1, num_kv_heads))
    per_item = -(-total_positions // target_items)
    per_item = int(min(4096, max(256, -(-per_item // 128) * 128)))
    if seq_lens is not None:
        while per_item < 4096 and sum(-(-int(n) // per_item) for n in seq_lens) > target_items:
            per_item += 128
    return per_item


def int8_calc_scales(key: torch.Tensor, value: torch.Tensor):
    """``(k_inv, v_inv, k_aq, v_aq)``: inv ``[1, KVH, D]``, aq ``[1, KVH, 1, D]``.

    Computed in ``key.dtype`` exactly as ``127.0 / amax`` and ``1.0 / inv``
    evaluate in torch (each step rounded to the dtype).
    """
    _native.require_gpu_tensors("int8_calc_scales", key, value)
    t = key.shape[0]
    kvh, d = key.shape[-2], key.shape[-1]
    c = kvh * d
    key = key.reshape(t, c).contiguous()
    value = value.reshape(t, c).contiguous().to(key.dtype)
    dev = key.device
    ws = torch.empty(2 * c, dtype=torch.int32, device=dev)
    k_inv = torch.empty(c, dtype=key.dtype, device=dev)
    v_inv = torch.empty_like(k_inv)
    k_aq = torch.empty_like(k_inv)
    v_aq = torch.empty_like(k_inv)
    rc = _native.lib().kvq_int8_calc_scales(
        _native.ptr(key), _native.ptr(value), _native.dtype_code(key.dtype), t, c,
        _native.ptr(ws), _native.ptr(k_inv), _native.ptr(v_inv), _native.ptr(k_aq),
        _native.ptr(v_aq), _native.stream_of(key),
    )
    _native.check(rc, "kvq_int8_calc_scales")
    return (
        k_inv.view(1, kvh, d),
        v_inv.view(1, kvh, d),
        k_aq.view(1, kvh, 1, d),
        v_aq.view(1, kvh, 1, d),
    )


def int8_quant_scatter(
    key: torch.Tensor,
    value: torch.Tensor,
    k_inv: torch.Tensor,
    v_inv: torch.Tensor,
    slot_mapping: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
) -> None:
    """Quantize ``[T, KVH, D]`` K/V and write them to the int8 pages by slot."""
    t = key.shape[0]
    if t == 0:
        return
    _native.require_gpu_tensors(
        "int8_quant_scatter", key, value, k_inv, slot_mapping, key_cache, value_cache
    )
    nb, bs, kvh, d = key_cache.shape
    rc = _native.lib().kvq_int8_quant_scatter(
        _native.ptr(key.contiguous()), _native.ptr(value.contiguous()),
        _native.dtype_code(key.dtype), _native.ptr(k_inv.contiguous()),
        _native.ptr(v_inv.contiguous()), _native.ptr(slot_mapping.contiguous()),
        _native.index_code(slot_mapping.dtype), t, kvh * d, _native.ptr(key_cache),
        _native.ptr(value_cache), nb, bs, _native.stream_of(key),
    )
    _native.check(rc, "kvq_int8_quant_scatter")


def int8_dequant_gather(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    target_dtype: torch.dtype,
    k_aq: torch.Tensor,
    v_aq: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged int8 -> dense TND ``[sum L, KVH, D]`` in ``target_dtype``."""
    nb, bs, kvh, d = key_cache.shape
    dev = key_cache.device
    total = int(sum(seq_lens))
    out_k = torch.empty((total, kvh, d), dtype=target_dtype, device=dev)
    out_v = torch.empty_like(out_k)
    if total == 0:
        return out_k, out_v
    _native.require_gpu_tensors("int8_dequant_gather", key_cache, value_cache, block_table)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(seq_lens)]), dtype=torch.int64, device=dev)
    bt = block_table.to(torch.int32).contiguous()
    rc = _native.lib().kvq_int8_dequant_gather(
        _native.ptr(key_cache), _native.ptr(value_cache), nb, bs, kvh, d,
        _native.ptr(k_aq.to(target_dtype).contiguous()),
        _native.ptr(v_aq.to(target_dtype).contiguous()), _native.dtype_code(target_dtype),
        _native.ptr(bt), bt.shape[1], _native.ptr(cu), len(seq_lens), _native.ptr(out_k),
        _native.ptr(out_v), _native.stream_of(key_cache),
    )
    _native.check(rc, "kvq_int8_dequant_gather")
    return out_k, out_v


def plan_int8_work(seq_lens: list[int], split_tokens: int) -> tuple[np.ndarray, np.ndarray]:
    """``(seq_meta int32 [B, 4], work int32 [W, 4])``; all positions are int8 (kind 0)."""
    meta = np.zeros((len(seq_lens), 4), dtype=np.int32)
    work: list[tuple[int, int, int, int]] = []
    for b, n in enumerate(seq_lens):
        first = len(work)
        p = 0
        while p < n:
            e = min(n, p + split_tokens)
            work.append((b, p, e, 0))
            p = e
        if n == 0:
            work.append((b, 0, 0, 1))
        meta[b] = (n, first, len(work) - first, 0)
    return meta, np.asarray(work, dtype=np.int32).reshape(-1, 4)


def int8_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    k_aq: torch.Tensor,
    v_aq: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    scale: float,
    out: torch.Tensor | None = None,
    split_tokens: int | None = None,
    plan: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """Paged int8 decode attention with per-channel antiquant (offset 0)."""
    batch, hq, d = query.shape
    nb, bs, kvh, _ = key_cache.shape
    if out is None:
        out = torch.empty_like(query)
    if batch == 0:
        return out
    bt = block_table.to(torch.int32).contiguous()
    if len(seq_lens) != batch or bt.shape[0] < batch:
        raise ValueError("int8_decode_attention: seq_lens / block_table rows != batch")
    if max(seq_lens) > bt.shape[1] * bs or min(seq_lens) < 0:
        raise ValueError(
            f"int8_decode_attention: a sequence length exceeds its block table "
            f"({max(seq_lens)} > {bt.shape[1]} x {bs})"
        )
    if plan is None:
        if split_tokens is None:
            split_tokens = int8_split_tokens(int(sum(seq_lens)), kvh, seq_lens=seq_lens)
        meta_np, work_np = plan_int8_work(seq_lens, split_tokens)
        meta = torch.from_numpy(meta_np).to(query.device)
        work = torch.from_numpy(work_np).to(query.device)
    else:
        meta, work = plan
    _native.require_gpu_tensors(
        "int8_decode_attention", query, key_cache, value_cache, bt, out, meta, work
    )
    lib = _native.lib()
    ws = torch.empty(
        (lib.kvq_int8_decode_workspace_bytes(work.shape[0], hq, d) + 3) // 4,
        dtype=torch.float32,
        device=query.device,
    )
    rc = lib.kvq_int8_decode_attn(
        _native.ptr(query), _native.dtype_code(query.dtype), batch, hq, kvh, d, float(scale),
        _native.ptr(key_cache), _native.ptr(value_cache), nb, bs,
        _native.ptr(k_aq.to(query.dtype).contiguous()),
        _native.ptr(v_aq.to(query.dtype).contiguous()), _native.ptr(bt), bt.shape[1],
        _native.ptr(meta), _native.ptr(work), work.shape[0], _native.ptr(ws), _native.ptr(out),
        _native.stream_of(query),
    )
    _native.check(rc, "kvq_int8_decode_attn")
    return out


def int8_quantize(x: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """Codes of ``x [T, KVH, D]`` through the quantize+scatter kernel (slot t -> row t)."""
    t = x.shape[0]
    kvh, d = inv.shape[-2], inv.shape[-1]
    codes = torch.empty((t, 1, kvh, d), dtype=torch.int8, device=x.device)
    if t == 0:
        return codes.view(x.shape)
    slots = torch.arange(t, dtype=torch.int64, device=x.device)
    xx = x.reshape(t, kvh, d)
    int8_quant_scatter(xx, xx, inv, inv, slots, codes, torch.empty_like(codes))
    return codes.view(x.shape)


def int8_dequantize(x: torch.Tensor, inv: torch.Tensor, target_dtype) -> torch.Tensor:
    """``(x - 0) * (1/inv)`` in ``target_dtype`` through the paged dequant kernel."""
    t = x.shape[0]
    kvh, d = inv.shape[-2], inv.shape[-1]
    aq = (1.0 / inv.to(target_dtype)).reshape(kvh * d)
    pages = x.reshape(t, 1, kvh, d).contiguous()
    table = torch.arange(t, dtype=torch.int32, device=x.device).view(1, t)
    dk, _ = int8_dequant_gather(pages, pages, table, [t], target_dtype, aq, aq)
    return dk.view(x.shape)


__all__ = [
    "INT8_DECODE_WAVES_PER_CU",
    "INT8_DECODE_WAVES_PER_CU_GROUPED",
    "int8_calc_scales",
    "int8_decode_attention",
    "int8_dequant_gather",
    "int8_dequantize",
    "int8_split_tokens",
    "int8_quant_scatter",
    "int8_quantize",
    "plan_int8_work",
]
