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
import math

import numpy as np
import torch

from . import _native

#: positions per work item when the caller does not choose
DEFAULT_SPLIT_TOKENS = 1024
#: positions per generic (mixed-source) work item
TAIL_ITEM_TOKENS = 64
#: decode waves resident per CU (the MFMA kernel's LDS and register budget)
WAVES_PER_CU = 8
#: cost of one residual-window (tail) position against one int4 position
TAIL_POSITION_COST = 8.0
#: largest piece, in int4 positions: more work than one piece per wave slot
#: of this size runs as several rounds of pieces, dispatched as slots free
PIECE_MAX_COST = 4096.0


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
    seqs: list[DecodeSeq], split_tokens: int, paired: bool = False
) -> tuple[np.ndarray, np.ndarray]:
    """``(seq_meta int32 [B, 8], work int32 [W, 4])`` for the decode kernel.

    Kind-0 items cover positions where both sides are int4 (split every
    ``split_tokens``); kind-1 items cover the rest (at most two residual
    windows long).  Every request owns at least one item, contiguous in the
    list.  ``paired``: each int4 range of ``2 * split_tokens`` positions is
    two items, kind 2 (its even 64-position chunks) at an even index and kind
    3 (its odd chunks) right after, which the kernel runs side by side on one
    XCD so the two share every key line (a request that would start a pair at
    an odd index opens with an empty kind-1 item).
    """
    # int4 items start on 128-token boundaries, so paired items split on
    # 64-position chunks and the MFMA kernel's tiles stay inside pages and
    # key groups
    split_tokens = max(128, -(-int(split_tokens) // 128) * 128)
    meta = np.zeros((len(seqs), 8), dtype=np.int32)
    work: list[tuple[int, int, int, int]] = []
    for b, s in enumerate(seqs):
        first = len(work)
        end_a = max(0, min(s.k_hist, s.v_hist, s.seq_len))
        p = 0
        if paired and end_a > 0 and len(work) % 2:
            work.append((b, 0, 0, 1))
        while p < end_a:
            if paired:
                e = min(end_a, p + 2 * split_tokens)
                work.append((b, p, e, 2))
                work.append((b, p, e, 3))
            else:
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


def plan_decode_pieces(
    seqs: list[DecodeSeq],
    num_kv_heads: int,
    cu_count: int = 256,
    tail_cost: float = TAIL_POSITION_COST,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``(seq_meta, work, pieces)``: the work list cut into pieces of equal cost.

    Every request's positions, int4 part (in 64-position tiles) then tail
    (``tail_cost`` per position, in 32-position steps), are laid end to end
    and cut where the running cost crosses a multiple of ``total / n``.  ``n``
    is ``slots = cu_count * WAVES_PER_CU / num_kv_heads`` times the rounds
    needed to keep pieces under ``PIECE_MAX_COST``: one wave per (piece, kv
    head) then fills the chip a whole number of times and every wave of a
    round ends at about the same time.  A cut inside a request splits it into
    items (int4 items start on multiples of 64); ``pieces[k]`` is the first
    item of piece ``k``.  The items follow ``plan_decode_work``'s rules, so
    the list is valid with or without the pieces.
    """
    slots = max(1, cu_count * WAVES_PER_CU // max(1, num_kv_heads))
    spans = []
    total = 0.0
    for s in seqs:
        end_a = max(0, min(s.k_hist, s.v_hist, s.seq_len))
        spans.append(end_a)
        total += -(-end_a // 64) * 64 + (s.seq_len - end_a) * tail_cost
    slots *= max(1, math.ceil(total / (slots * PIECE_MAX_COST)))
    step = max(64.0, total / slots)
    meta = np.zeros((len(seqs), 8), dtype=np.int32)
    work: list[tuple[int, int, int, int]] = []
    pieces = [0]
    cum = 0.0
    cut = step

    def after(unit: float) -> None:  # close the piece once the cost reaches the cut
        nonlocal cut
        if cum >= cut - unit / 2 and len(pieces) < slots and len(work) > pieces[-1]:
            pieces.append(len(work))
            while cut - unit / 2 <= cum:
                cut += step

    for b, s in enumerate(seqs):
        first = len(work)
        end_a = spans[b]
        p = 0
        while p < end_a:
            tiles = max(1, int((cut - cum) / 64.0 + 0.5))
            e = min(end_a, p + 64 * tiles)
            work.append((b, p, e, 0))
            cum += -(-(e - p) // 64) * 64
            p = e
            after(64.0)
        p = end_a
        unit = 32 * tail_cost
        while p < s.seq_len:
            n = max(1, int((cut - cum) / unit + 0.5)) * 32
            e = min(s.seq_len, p + n)
            work.append((b, p, e, 1))
            cum += (e - p) * tail_cost
            p = e
            after(unit)
        if s.seq_len == 0:
            work.append((b, 0, 0, 1))
        meta[b] = (
            s.seq_len, s.k_hist, s.v_hist, s.ring_row, s.k_first, s.v_first,
            first, len(work) - first,
        )
    if len(work) > pieces[-1]:
        pieces.append(len(work))
    return (meta, np.asarray(work, dtype=np.int32).reshape(-1, 4),
            np.asarray(pieces, dtype=np.int32))


def plan_decode(
    seqs: list[DecodeSeq], num_kv_heads: int, cu_count: int = 256
) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """The default decode plan: ``(seq_meta, work, pieces or None)``.

    Work that fills the chip's wave slots once (pieces of at most
    ``PIECE_MAX_COST``) is cut into equal-cost pieces (``plan_decode_pieces``):
    with a single round, the wave that ends last sets the time, so every wave
    gets the same cost.  More work runs as items of ``choose_split_tokens``
    int4 positions per wave, in pairs that share their key lines, with the
    tail items last (``plan_decode_work(paired=True)``): over many rounds the
    hardware hands items to free slots, and the small tail items at the end
    fill the last round's gaps (measured on 256 x 32K tokens, unpaired: 2.63
    ms against 2.71 ms for pieces).
    """
    slots = max(1, cu_count * WAVES_PER_CU // max(1, num_kv_heads))
    total = 0.0
    for s in seqs:
        end_a = max(0, min(s.k_hist, s.v_hist, s.seq_len))
        total += -(-end_a // 64) * 64 + (s.seq_len - end_a) * TAIL_POSITION_COST
    if total <= slots * PIECE_MAX_COST:
        return plan_decode_pieces(seqs, num_kv_heads, cu_count)
    # paired items: each wave still takes split_tokens int4 positions
    meta, work = plan_decode_work(
        seqs, choose_split_tokens(sum(s.seq_len for s in seqs), num_kv_heads, cu_count),
        paired=True,
    )
    return meta, work, None


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
    the device; ``ring_k/ring_v`` ``[rows, R + 1, KVH, D]``.  ``plan`` may
    carry a prebuilt ``(seq_meta, work)`` pair or ``(seq_meta, work, pieces)``
    triple already on the device.  Without a plan the work is cut into
    default plan (``plan_decode``), or split every ``split_tokens`` positions
    when that is given (``plan_decode_work``).
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
    pieces = None
    if plan is None:
        if split_tokens is None:
            meta_np, work_np, pieces_np = plan_decode(seqs, kvh, _cu_count(query.device))
            if pieces_np is not None:
                pieces = torch.from_numpy(pieces_np).to(query.device)
        else:
            meta_np, work_np = plan_decode_work(seqs, split_tokens)
        meta = torch.from_numpy(meta_np).to(query.device)
        work = torch.from_numpy(work_np).to(query.device)
    elif len(plan) == 3:
        meta, work, pieces = plan
    else:
        meta, work = plan
    _native.require_gpu_tensors(
        "kivi_decode_attention", query, kq, block_table, ring_k, ring_v, out, meta, work, pieces
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
        _native.ptr(pieces), 0 if pieces is None else pieces.numel() - 1,
        _native.ptr(ring_k), _native.ptr(ring_v), _native.dtype_code(ring_k.dtype),
        ring_k.shape[1], _native.ptr(ws), _native.ptr(out), _native.stream_of(query),
    )
    _native.check(rc, "kvq_kivi_decode_attn")
    return out


_CU_COUNT: dict[int, int] = {}


def _cu_count(device) -> int:
    """Compute units of ``device`` (cached; the planner sizes pieces to it)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return _CU_COUNT[idx]


__all__ = [
    "DEFAULT_SPLIT_TOKENS",
    "DecodeSeq",
    "choose_split_tokens",
    "kivi_decode_attention",
    "plan_decode",
    "plan_decode_pieces",
    "plan_decode_work",
]
