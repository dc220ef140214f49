# SPDX-License-Identifier: Apache-2.0
"""Shared builders for the tests: seeded synthetic K/V and empty KIVI caches."""

from __future__ import annotations

import torch


def make_kv(t: int, kvh: int, d: int, *, dtype=torch.bfloat16, seed: int = 0, outliers=True):
    """K/V ~ N(0,1); keys scaled per (head, dim) channel by exp(N(0,1))."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(t, kvh, d, generator=g)
    v = torch.randn(t, kvh, d, generator=g)
    if outliers:
        k = k * torch.exp(torch.randn(kvh, d, generator=g))
    return k.to(dtype), v.to(dtype)


def empty_kivi_caches(nb: int, bs: int, kvh: int, d: int, g: int, device="cpu", fill=0):
    """The six KIVI tensors (filled with ``fill`` so stale reads are visible)."""
    kq = torch.full((nb, kvh, d, bs // 8), fill, dtype=torch.int32, device=device)
    ks = torch.full((nb, kvh, d, bs // g), float(fill), dtype=torch.float32, device=device)
    km = torch.full_like(ks, float(fill))
    vq = torch.full((nb, bs, kvh, d // 8), fill, dtype=torch.int32, device=device)
    vs = torch.full((nb, bs, kvh, d // g), float(fill), dtype=torch.float32, device=device)
    vm = torch.full_like(vs, float(fill))
    return kq, ks, km, vq, vs, vm


def shuffled_table(batch: int, blocks_per_seq: int, num_blocks: int, seed: int = 0):
    """A random permutation of the block pool laid out as a block table."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=g)[: batch * blocks_per_seq]
    return perm.view(batch, blocks_per_seq).to(torch.int32)


def slots_for(table_row: torch.Tensor, positions: range, bs: int) -> torch.Tensor:
    pos = torch.tensor(list(positions), dtype=torch.int64)
    return table_row.to(torch.int64)[pos // bs] * bs + pos % bs


def to_dev(tensors, device):
    return tuple(t.to(device) for t in tensors)
