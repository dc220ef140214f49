# SPDX-License-Identifier: Apache-2.0
"""Fused KIVI INT4 decode attention (HIP kernel ``kvq_kivi_decode_attn``).

Replaces the gather + overlay + fused-attention sequence of
``pkg/methods/kivi_int4/attention_backend.py:849-935,1193-1230``: the kernel
reads the int4 pages and the residual ring directly.  The host builds a work
list from the request lengths and window states it already holds as Python
ints, so planning costs no device synchronisation.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import _native

#: positions per work item when the caller does not choose
DEFAULT_SPLIT_TOKENS = 1024
#: positions per generic (mixed-source) work item
TAIL_ITEM_TOKENS = 64


@dataclass(frozen=True)
class DecodeSeq:
    """One request's decode geometry.

    Positions ``< k_hist`` read int4 keys, the others ring lane
    ``(k_first + p - k_hist) % ring_len`` of row ``ring_row``; same for values.
    """

    seq_len: int
    k_hist: int
    v_hist: int
    ring_row: int = 0
    k_first: int = 0
    v_first: int = 0


def choose_split_tokens(total_positions: int, num_kv_heads: int, cu_count: int = 256) -> int:
    """Positions per work item: about 8 waves per CU, in [256, 4096], /128."""
    target_items = max(1, (cu_count * 8) // max(1, num_kv_heads))
    per_item = -(-total_positions // target_items)
    per_item = -(-per_item // 128) * 128
    return int(min(4096, max(256, per_item)))


def plan_decode_work(
    seqs: list[DecodeSeq], split_tokens: int
) -> tuple[np.ndarray, np.ndarray]:
    """``(seq_meta int32 [B, 8], work int32 [W, 4])`` for the decode kernel.

    Kind-0 items cover positions where both sides are int4 (split every
    ``split_tokens``); one kind-1 item covers the rest (at most two residual
    windows long).  Every request owns at least one item, contiguous in the list.
    """
    # kind-0 items start on 128-token boundaries: the MFMA kernel walks
    # page- and key-group-aligned tiles of up to 128 tokens
    split_tokens = max(128, -(-int(split_tokens) // 128) * 128)
    meta = np.zeros((len(seqs), 8), dtype=np.int32)
    work: list[tuple[int, int, int, int]] = []
    for b, s in enumerate(seqs):
        first = len(work)
        end_a = max(0, min(s.k_hist, s.v_hist, s.seq_len))
        p = 0
        while p < end_a:
            e = min(end_a, p + split_tokens)
            work.append((b, p, e, 0))
            p = e
        # the mixed-source tail (at most two residual windows) in 64-position
        # items, so tails of different requests and heads run side by side
        p = end_a
        while p < s.seq_len:
            e = min(s.seq_len, p + TAIL_ITEM_TOKENS)
            work.append((b, p, e, 1))
            p = e
        if s.seq_len == 0:
            work.append((b, 0, 0, 1))
        meta[b] = (
            s.seq_len, s.k_hist, s.v_hist, s.ring_row, s.k_first, s.v_first,
            first, len(work) - first,
        )
    return meta, np.asarray(work, dtype=np.int32).reshape(-1, 4)


def kivi_decode_attention(
    query: torch.Tensor,
    caches: tuple[torch.Tensor, ...],
    block_table: torch.Tensor,
    seqs: list[DecodeSeq],
    ring_k: torch.Tensor,
    ring_v: torch.Tensor,
    scale: float,
    group_size: int,
    out: torch.Tensor | None = None,
    split_tokens: int | None = None,
    plan: tuple[torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """``out[b] = softmax(q[b] K_b^T * scale) V_b`` over int4 history + ring.

    ``query`` is ``[B, Hq, D]``; ``block_table`` int32 ``[B, max_blocks]`` on
    the device; ``ring_k/ring_v`` ``[rows, R, KVH, D]``.  ``plan`` may carry a
    prebuilt ``(seq_meta, work)`` pair already on the device.
    """
    kq, ks, km, vq, vs, vm = caches
    batch, hq, d = query.shape
    nb, kvh, _, pbs = kq.shape
    if out is None:
        out = torch.empty_like(query)
    if batch == 0:
        return out
    if block_table.dtype != torch.int32:
        block_table = block_table.to(torch.int32)
    block_table = block_table.contiguous()
    if plan is None:
        if split_tokens is None:
            split_tokens = choose_split_tokens(sum(s.seq_len for s in seqs), kvh)
        meta_np, work_np = plan_decode_work(seqs, split_tokens)
        meta = torch.from_numpy(meta_np).to(query.device)
        work = torch.from_numpy(work_np).to(query.device)
    else:
        meta, work = plan
    _native.require_gpu_tensors(
        "kivi_decode_attention", query, kq, block_table, ring_k, ring_v, out, meta, work
    )
    lib = _native.lib()
    num_work = work.shape[0]
    ws = torch.empty(
        (lib.kvq_kivi_decode_workspace_bytes(num_work, hq, d) + 3) // 4,
        dtype=torch.float32,
        device=query.device,
    )
    rc = lib.kvq_kivi_decode_attn(
        _native.ptr(query), _native.dtype_code(query.dtype), batch, hq, kvh, d, float(scale),
        _native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq), _native.ptr(vs),
        _native.ptr(vm), nb, pbs * 8, group_size, _native.ptr(block_table),
        block_table.shape[1], _native.ptr(meta), _native.ptr(work), num_work,
        _native.ptr(ring_k), _native.ptr(ring_v), _native.dtype_code(ring_k.dtype),
        ring_k.shape[1], _native.ptr(ws), _native.ptr(out), _native.stream_of(query),
    )
    _native.check(rc, "kvq_kivi_decode_attn")
    return out


__all__ = [
    "DEFAULT_SPLIT_TOKENS",
    "DecodeSeq",
    "choose_split_tokens",
    "kivi_decode_attention",
    "plan_decode_work",
]
