# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 scheme object: geometry, window bookkeeping, self-description.

The reference's semantics object (``pkg/methods/kivi_int4/semantics.py:40-310``)
also carries a torch restatement of the quantization math for CPU testing.
In this build the math lives only in the HIP kernels (``ops.kivi_pack`` /
``ops.kivi_gather``); the CPU restatement that checks them is test
infrastructure outside the package.  What stays here is host bookkeeping the
attention mixin needs, with the reference's names and behaviour:

* ``ordered_slots``: per-request absolute slot lists from a block table;
* ``is_aligned_key_window``: the state machine's key-flush gate;
* ``cu_seqlens_to_seq_lens`` and ``build_causal_mask`` (metadata only).
"""

from __future__ import annotations

from types import SimpleNamespace
from typing import Any

import torch

from .geometry import validate_kivi_config

BITS = 4


def _normalize_config(config: Any) -> Any:
    if hasattr(config, "group_size"):
        return config
    return SimpleNamespace(
        head_size=config.head_size,
        group_size=config.kivi_group_size,
        residual_length=config.kivi_residual_length,
        block_size=getattr(config, "block_size", None),
    )


class KiviInt4Semantics:
    """Geometry and window bookkeeping of the KIVI INT4 scheme."""

    def __init__(self, config: Any) -> None:
        validate_kivi_config(config)
        self.config = _normalize_config(config)

    @property
    def group_size(self) -> int:
        return self.config.group_size

    @property
    def bits(self) -> int:
        return BITS

    def packed_key_last_dim(self) -> int:
        """int32 words per token row: head_size / 8."""
        return self.config.head_size // 8

    @staticmethod
    def cu_seqlens_to_seq_lens(cu_seqlens: Any) -> list[int]:
        if isinstance(cu_seqlens, torch.Tensor):
            cu_seqlens = cu_seqlens.tolist()
        out, prev = [], 0
        for end in cu_seqlens:
            out.append(int(end) - prev)
            prev = int(end)
        return out

    @staticmethod
    def ordered_slots(block_table: Any, seq_lens: list[int], block_size: int) -> list[list[int]]:
        """Absolute slot of every position, per request, skipping unallocated blocks.

        ``slot = block_id * block_size + offset``; a negative block id gives a
        negative slot, so filtering ``slot >= 0`` drops exactly the positions
        in unallocated blocks (``semantics.py:224-252``).  One host copy of the
        table, no per-position device reads.
        """
        if isinstance(block_table, torch.Tensor):
            rows = block_table.to("cpu", torch.long).tolist()
        else:
            rows = [list(r) for r in block_table]
        out: list[list[int]] = []
        for req, n in enumerate(seq_lens):
            row = rows[req] if req < len(rows) else []
            slots = []
            for pos in range(int(n)):
                blk = int(row[pos // block_size])
                if blk >= 0:
                    slots.append(blk * block_size + pos % block_size)
            out.append(slots)
        return out

    def is_aligned_key_window(self, window_slots: list[int], block_size: int) -> bool:
        """Every group contiguous, group aligned and inside one block."""
        if not window_slots:
            return False
        g = self.group_size
        if len(window_slots) % g:
            return False
        for start in range(0, len(window_slots), g):
            grp = [int(s) for s in window_slots[start : start + g]]
            first = grp[0]
            if first % block_size % g:
                return False
            if grp[-1] // block_size != first // block_size:
                return False
            if grp != list(range(first, first + g)):
                return False
        return True

    def build_causal_mask(self, q_len: int, kv_seq_len: int, dtype: Any, device: Any) -> Any:
        """Additive mask, ``finfo.min`` where ``kv_pos > q_pos`` (metadata only).

        The HIP attention kernels apply this rule themselves; the tensor form
        is kept for callers that pass an explicit mask.
        """
        q_pos = torch.arange(kv_seq_len - q_len, kv_seq_len, device=device)
        kv_pos = torch.arange(kv_seq_len, device=device)
        masked = kv_pos.unsqueeze(0) > q_pos.unsqueeze(1)
        zero = torch.zeros((), dtype=dtype, device=device)
        neg = torch.full((), torch.finfo(dtype).min, dtype=dtype, device=device)
        return torch.where(masked, neg, zero).unsqueeze(0)

    def describe(self) -> dict[str, Any]:
        return {
            "scheme": "kivi_int4",
            "bits": self.bits,
            "group_size": self.group_size,
            "residual_length": self.config.residual_length,
            "key_grouping": "token groups (residual window flushed whole)",
            "value_grouping": "head-dim groups (per token)",
            "kernels": "HIP gfx950 (pack, gather-dequant, fused decode, MFMA prefill)",
        }


__all__ = ["KiviInt4Semantics"]
