# SPDX-License-Identifier: Apache-2.0
"""Layout and metadata validators shared by the pack and gather entry points.

Same rules and message texts as ``pkg/ops/kivi_layout.py:13-238`` (callers
match on them), so a bad layout fails before any kernel is launched.
"""

from __future__ import annotations

import numpy as np
import torch


def _check_same_device(name: str, tensor: torch.Tensor, ref: torch.Tensor) -> None:
    if tensor.device != ref.device:
        raise RuntimeError(f"{name} must be on device {ref.device}, got {tensor.device}.")


def _check_contiguous(name: str, tensor: torch.Tensor) -> None:
    if not tensor.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous.")


def _check_4d(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if t.ndim != 4:
            raise RuntimeError(f"{name} must be 4D, got shape={tuple(t.shape)}.")


def _check_value_cache_layout(
    v_quant_cache: torch.Tensor,
    v_scale_cache: torch.Tensor,
    v_mn_cache: torch.Tensor,
    *,
    num_kv_heads: int,
    head_size: int,
    group_size: int,
) -> None:
    """``v_quant [NB,Bs,KVH,D/8]`` int32 and ``v_scale/v_mn [NB,Bs,KVH,D/G]``."""
    _check_4d("v_quant_cache", v_quant_cache)
    if v_scale_cache.ndim != 4 or v_mn_cache.ndim != 4:
        raise RuntimeError(
            "v_scale_cache and v_mn_cache must be 4D, got "
            f"{tuple(v_scale_cache.shape)} and {tuple(v_mn_cache.shape)}."
        )
    nb, bs = v_quant_cache.shape[:2]
    want_q = (nb, bs, num_kv_heads, head_size // 8)
    want_s = (nb, bs, num_kv_heads, head_size // group_size)
    for name, t, want in (
        ("v_quant_cache", v_quant_cache, want_q),
        ("v_scale_cache", v_scale_cache, want_s),
        ("v_mn_cache", v_mn_cache, want_s),
    ):
        if tuple(t.shape) != want:
            raise RuntimeError(
                f"{name} layout mismatch: got {tuple(t.shape)}, expected {want}."
            )


def _check_key_cache_layout(
    k_quant_cache: torch.Tensor,
    k_scale_cache: torch.Tensor,
    k_mn_cache: torch.Tensor,
    *,
    num_kv_heads: int,
    head_size: int,
    group_size: int,
) -> int:
    """``k_quant [NB,KVH,D,Bs/8]`` int32 and ``k_scale/k_mn [NB,KVH,D,Bs/G]``.

    Returns the block size.
    """
    _check_4d("k_quant_cache", k_quant_cache)
    if k_scale_cache.ndim != 4 or k_mn_cache.ndim != 4:
        raise RuntimeError(
            "k_scale_cache and k_mn_cache must be 4D, got "
            f"{tuple(k_scale_cache.shape)} and {tuple(k_mn_cache.shape)}."
        )
    nb = k_quant_cache.shape[0]
    bs = k_quant_cache.shape[3] * 8
    want_q = (nb, num_kv_heads, head_size, bs // 8)
    want_s = (nb, num_kv_heads, head_size, bs // group_size)
    for name, t, want in (
        ("k_quant_cache", k_quant_cache, want_q),
        ("k_scale_cache", k_scale_cache, want_s),
        ("k_mn_cache", k_mn_cache, want_s),
    ):
        if tuple(t.shape) != want:
            raise RuntimeError(
                f"{name} layout mismatch: got {tuple(t.shape)}, expected {want}."
            )
    return bs


def _check_slot_mapping(slot_mapping: torch.Tensor, num_tokens: int) -> None:
    if slot_mapping.ndim != 1:
        raise RuntimeError(
            f"slot_mapping must be 1D, got shape={tuple(slot_mapping.shape)}."
        )
    if slot_mapping.numel() != num_tokens:
        raise RuntimeError(
            "slot_mapping length must match num_tokens, got "
            f"{slot_mapping.numel()} vs {num_tokens}."
        )
    if slot_mapping.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f"slot_mapping must be int32/int64, got {slot_mapping.dtype}.")


def key_slot_groups_error(slots: list[int], *, block_size: int, group_size: int) -> str | None:
    """Host-side form of the key-flush gate; ``None`` when the window passes.

    Each group of ``group_size`` slots must be valid, contiguous, start
    group-aligned and stay inside one cache block, so every packed word has a
    single writer.
    """
    if any(s < 0 for s in slots):
        return "kivi_pack_key_cache requires all slot_mapping entries to be valid."
    for start in range(0, len(slots), group_size):
        grp = slots[start : start + group_size]
        if grp != list(range(grp[0], grp[0] + group_size)):
            return (
                "kivi_pack_key_cache requires each token group to map to contiguous slots."
            )
    for start in range(0, len(slots), group_size):
        if slots[start] % group_size:
            return "kivi_pack_key_cache requires each token group to be group-size aligned."
    for start in range(0, len(slots), group_size):
        if slots[start] // block_size != slots[start + group_size - 1] // block_size:
            return (
                "kivi_pack_key_cache requires each token group to stay within one cache block."
            )
    return None


def _check_key_slot_groups(
    slot_mapping: torch.Tensor, *, block_size: int, group_size: int
) -> None:
    """Kernel-side gate of a key flush (``pkg/ops/kivi_layout.py:127-163``)."""
    slots = [int(s) for s in slot_mapping.tolist()]
    if len(slots) % group_size:
        raise RuntimeError(
            "kivi_pack_key_cache requires whole token groups, got "
            f"{len(slots)} slots for group_size={group_size}."
        )
    err = key_slot_groups_error(slots, block_size=block_size, group_size=group_size)
    if err is not None:
        raise RuntimeError(err)


def _check_block_table(block_table: torch.Tensor) -> None:
    if block_table.ndim != 2:
        raise RuntimeError(f"block_table must be 2D, got shape={tuple(block_table.shape)}.")
    if block_table.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f"block_table must be int32/int64, got {block_table.dtype}.")


def _check_seq_lens(seq_lens: torch.Tensor, batch_size: int) -> None:
    if seq_lens.ndim != 1:
        raise RuntimeError(f"seq_lens must be 1D, got shape={tuple(seq_lens.shape)}.")
    if seq_lens.numel() != batch_size:
        raise RuntimeError(
            f"seq_lens length must match batch size, got {seq_lens.numel()} vs {batch_size}."
        )
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise RuntimeError(f"seq_lens must be int32/int64, got {seq_lens.dtype}.")


def check_gather_metadata_host(
    block_table_rows: list[list[int]] | np.ndarray | None,
    seq_lens: list[int],
    *,
    max_blocks: int,
    num_blocks: int,
    block_size: int,
) -> None:
    """Coverage and live-block checks on host lists (no device sync)."""
    longest = max(seq_lens, default=0)
    if longest > max_blocks * block_size:
        raise RuntimeError(
            "block_table does not cover the longest KIVI sequence: "
            f"max_seq_len={longest}, max_blocks={max_blocks}, block_size={block_size}."
        )
    if block_table_rows is None:
        return
    try:
        table = np.asarray(block_table_rows, dtype=np.int64)
    except ValueError:  # ragged rows
        table = None
    if table is None or table.ndim != 2:
        for row, length in zip(block_table_rows, seq_lens):
            live = row[: -(-length // block_size)] if length > 0 else []
            if any(b < 0 for b in live):
                raise RuntimeError("KIVI block_table has invalid block ids for live tokens.")
            if any(b >= num_blocks for b in live):
                raise RuntimeError("KIVI block_table references blocks outside the int4 cache.")
        return
    n = min(table.shape[0], len(seq_lens))
    lens = np.asarray(seq_lens[:n], dtype=np.int64)
    live = np.arange(table.shape[1])[None, :] < -(-lens // block_size)[:, None]
    neg = ((table[:n] < 0) & live).any(axis=1)
    out = ((table[:n] >= num_blocks) & live).any(axis=1)
    bad = np.flatnonzero(neg | out)
    if bad.size:  # the first offending request, checked as the reference checks it
        if neg[bad[0]]:
            raise RuntimeError("KIVI block_table has invalid block ids for live tokens.")
        raise RuntimeError("KIVI block_table references blocks outside the int4 cache.")


def _check_dequant_gather_metadata(
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    num_blocks: int,
    block_size: int,
) -> tuple[torch.Tensor, int, int]:
    """Metadata gate of the gather (``pkg/ops/kivi_layout.py:205-238``).

    Returns ``(cu_seq_lens int64 [B+1] on the table's device, batch, total)``.
    """
    batch = int(seq_lens.numel())
    _check_block_table(block_table)
    _check_seq_lens(seq_lens, batch)
    _check_contiguous("block_table", block_table)
    _check_contiguous("seq_lens", seq_lens)
    if block_table.shape[0] != batch:
        raise RuntimeError(
            f"block_table batch size must match seq_lens, got {block_table.shape[0]} vs {batch}."
        )
    lens = [int(x) for x in seq_lens.tolist()]
    check_gather_metadata_host(
        [[int(b) for b in r] for r in block_table.tolist()],
        lens,
        max_blocks=block_table.shape[1],
        num_blocks=num_blocks,
        block_size=block_size,
    )
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    cu_t = torch.tensor(cu, dtype=torch.int64, device=block_table.device)
    return cu_t, batch, cu[-1]


__all__ = [
    "_check_block_table",
    "_check_contiguous",
    "_check_dequant_gather_metadata",
    "_check_key_cache_layout",
    "_check_key_slot_groups",
    "_check_same_device",
    "_check_seq_lens",
    "_check_slot_mapping",
    "_check_value_cache_layout",
    "check_gather_metadata_host",
    "key_slot_groups_error",
]
