# SPDX-License-Identifier: Apache-2.0
"""Fused KIVI INT4 decode attention (HIP kernel ``kvq_kivi_decode_attn``).

Replaces the gather + overlay + fused-attention sequence of
``pkg/methods/kivi_int4/attention_backend.py:849-935,1193-1230``: the kernel
reads the int4 pages and the residual ring directly.  The host builds a work
list from the request lengths and window states it already holds as Python
ints, so planning costs no device synchronisation.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _native

#: positions per work item when the caller does not choose
DEFAULT_SPLIT_TOKENS = 1024
#: positions per generic (mixed-source) work item
TAIL_ITEM_TOKENS = 64
#: decode waves resident per CU (the MFMA kernel's LDS and register budget)
WAVES_PER_CU = 8
#: cost of one residual-window (tail) position against one int4 position:
#: measured on config-3 decode, where 6 balances the pieces best (94.9 us,
#: against 97.3 at 8 and 97.1 at 5); a tail position moves 3.5x the bytes
#: of an int4 one and its item waits for memory about once per sub-tile
TAIL_POSITION_COST = 6.0
#: largest piece, in int4 positions: more work than one piece per wave slot
#: of this size runs as several rounds of pieces, dispatched as slots free
PIECE_MAX_COST = 4096.0
#: int4 tile of the pieces the page-streaming decode runs: whole pages, so no
#: two workgroups stream the same page
PAGE_TILE = 128


def page_streaming_applies(num_heads: int, num_kv_heads: int, head_size: int, block_size: int,
                           group_size: int, q_dtype: torch.dtype, ring_dtype: torch.dtype) -> bool:
    """The geometry the page-streaming decode covers (``kvq_kivi_decode_attn``
    given pieces: one workgroup per piece streams whole pages for all kv heads):
    8 kv heads, head size 128, block size 128, group 64 or 128, at most 16
    query heads per kv head, a 16-bit query shared with the ring.  Plans for
    it cut int4 items on page bounds (``PAGE_TILE``)."""
    return (num_kv_heads == 8 and head_size == 128 and block_size == 128
            and group_size in (64, 128) and num_heads % num_kv_heads == 0
            and num_heads // num_kv_heads <= 16
            and q_dtype in (torch.bfloat16, torch.float16) and ring_dtype == q_dtype)


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
    target_items = max(1, (cu_count * WAVES_PER_CU) // max(1, num_kv_heads))
    per_item = -(-total_positions // target_items)
    per_item = -(-per_item // 128) * 128
    return int(min(4096, max(256, per_item)))


def seq_array(seqs: list[DecodeSeq]) -> np.ndarray:
    """The planner's request geometry, int32 ``[B, 6]``."""
    out = np.empty((len(seqs), 6), dtype=np.int32)
    for i, s in enumerate(seqs):
        out[i] = (s.seq_len, s.k_hist, s.v_hist, s.ring_row, s.k_first, s.v_first)
    return out


def work_capacity(batch: int, num_kv_heads: int, cu_count: int, total_positions: int) -> int:
    """An upper bound on the items any plan of a batch can hold."""
    slots = max(1, cu_count * WAVES_PER_CU // max(1, num_kv_heads))
    rounds = 1 + total_positions // (slots * int(PIECE_MAX_COST)) + 1
    # pieces cut a request at most once per piece boundary; split plans make
    # at most two items per 128 int4 positions (pairs) and a tail item per 64
    # positions, plus up to three per request at range ends
    return 2 * slots * rounds + 3 * batch + 2 * (total_positions // 64) + 8


def plan_into(seqs: np.ndarray, num_kv_heads: int, cu_count: int, mode: int, *,
              split_tokens: int = 0, tail_cost: float = TAIL_POSITION_COST,
              meta: np.ndarray, work: np.ndarray, pieces: np.ndarray | None) -> tuple[int, int]:
    """Run the native planner into caller arrays; ``(num_work, num_pieces)``.

    ``seqs`` int32 ``[B, 6]``; ``meta`` int32 ``[B, 8]``; ``work`` int32
    ``[cap, 4]``; ``pieces`` int32 ``[cap_p + 1]`` (pinned views let the
    caller copy the plan to the device without a synchronisation).
    """
    npieces = ctypes.c_int64(0)
    n = _native.lib().kvq_plan_kivi_decode(
        seqs.ctypes.data, seqs.shape[0], num_kv_heads, cu_count, mode, int(split_tokens),
        float(tail_cost), meta.ctypes.data, work.ctypes.data, work.shape[0],
        None if pieces is None else pieces.ctypes.data,
        0 if pieces is None else pieces.shape[0] - 1, ctypes.byref(npieces),
    )
    _native.check(int(n) if n < 0 else 0, "kvq_plan_kivi_decode")
    return int(n), int(npieces.value)


def _plan(seqs: list[DecodeSeq], num_kv_heads: int, cu_count: int, mode: int,
          split_tokens: int = 0, tail_cost: float = TAIL_POSITION_COST):
    arr = seq_array(seqs)
    cap = work_capacity(len(seqs), num_kv_heads, cu_count, int(arr[:, 0].sum()) if len(seqs) else 0)
    meta = np.zeros((len(seqs), 8), dtype=np.int32)
    work = np.zeros((cap, 4), dtype=np.int32)
    pieces = np.zeros(cap + 1, dtype=np.int32)
    n, npc = plan_into(arr, num_kv_heads, cu_count, mode, split_tokens=split_tokens,
                       tail_cost=tail_cost, meta=meta, work=work, pieces=pieces)
    return meta, work[:n].copy(), (pieces[: npc + 1].copy() if npc else None)


def plan_decode_work(
    seqs: list[DecodeSeq], split_tokens: int, paired: bool = False
) -> tuple[np.ndarray, np.ndarray]:
    """``(seq_meta int32 [B, 8], work int32 [W, 4])`` for the decode kernel.

    Kind-0 items cover positions where both sides are int4 (split every
    ``split_tokens``, rounded up to a multiple of 128); kind-1 items cover the
    rest in 64-position items.  Every request owns at least one item,
    contiguous in the list.  ``paired``: each int4 range of ``2 *
    split_tokens`` positions is two items, kind 2 (its even 64-position
    chunks) at an even index and kind 3 (its odd chunks) right after, which
    the kernel runs side by side on one XCD so the two share every key line
    (a request that would start a pair at an odd index opens with an empty
    kind-1 item).  Planned natively (``kvq_plan_kivi_decode``).
    """
    mode = _native.KVQ_PLAN_SPLIT_PAIRED if paired else _native.KVQ_PLAN_SPLIT
    meta, work, _ = _plan(seqs, 1, 1, mode, split_tokens=split_tokens)
    return meta, work


def plan_decode_pieces(
    seqs: list[DecodeSeq],
    num_kv_heads: int,
    cu_count: int = 256,
    tail_cost: float = TAIL_POSITION_COST,
    tile: int = 64,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """``(seq_meta, work, pieces)``: the work list cut into cost-balanced pieces.

    Every request's positions, int4 part (in 64-position tiles) then tail
    (``tail_cost`` per position, in 32-position steps), are laid end to end
    and cut where the running cost crosses a multiple of ``total / n``.  ``n``
    is ``slots = cu_count * WAVES_PER_CU / num_kv_heads`` times the rounds
    needed to keep pieces under ``PIECE_MAX_COST``: one wave per (piece, kv
    head) then fills the chip a whole number of times and every wave of a
    round ends at about the same time (in a one-round plan with ``tile`` =
    ``PAGE_TILE`` and one piece per CU, the first half of the pieces, which the
    hardware dispatches first on their CUs and whose waves the arbiter then
    favours, carry 1.4 times the cost of the second half, so that the two
    workgroups sharing a CU finish together).  A cut inside a request splits it into
    items (int4 items start on multiples of ``tile``, 64 or ``PAGE_TILE``);
    ``pieces[k]`` is the first item of piece ``k``.  Planned natively
    (``kvq_plan_kivi_decode``).
    """
    meta, work, pieces = _plan(seqs, num_kv_heads, cu_count, _native.KVQ_PLAN_PIECES,
                               split_tokens=tile, tail_cost=tail_cost)
    return meta, work, (pieces if pieces is not None else np.zeros(1, dtype=np.int32))


def plan_decode(
    seqs: list[DecodeSeq], num_kv_heads: int, cu_count: int = 256, *,
    page_streaming: bool = False,
) -> tuple[np.ndarray, np.ndarray, np.ndarray | None]:
    """The default decode plan: ``(seq_meta, work, pieces or None)``.

    ``page_streaming`` (the layer is one ``page_streaming_applies`` accepts):
    pieces on page bounds, any amount of work -- a workgroup per piece streams
    its pages at the memory's pace, and many rounds of equal pieces keep every
    CU busy to the end.  Otherwise:

    Work that fills the chip's wave slots once (pieces of at most
    ``PIECE_MAX_COST``) is cut into equal-cost pieces (``plan_decode_pieces``):
    with a single round, the wave that ends last sets the time, so every wave
    gets the same cost.  More work runs as items of up to 8192 int4 positions
    per wave, with the tail items last (``plan_decode_work``): over many rounds
    the hardware hands items to free slots, and the small tail items at the end
    fill the last round's gaps (measured on 256 x 32K tokens: 2.53 ms, against
    2.60 ms for pairs of 4096-position half items).
    """
    if page_streaming:
        return _plan(seqs, num_kv_heads, cu_count, _native.KVQ_PLAN_PIECES, split_tokens=PAGE_TILE)
    return _plan(seqs, num_kv_heads, cu_count, _native.KVQ_PLAN_DEFAULT)


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
            paged = page_streaming_applies(hq, kvh, d, pbs * 8, group_size, query.dtype,
                                           ring_k.dtype)
            meta_np, work_np, pieces_np = plan_decode(seqs, kvh, _cu_count(query.device),
                                                      page_streaming=paged)
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
    "page_streaming_applies",
    "plan_decode",
    "plan_decode_pieces",
    "plan_decode_work",
]
