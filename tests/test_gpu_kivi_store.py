# SPDX-License-Identifier: Apache-2.0
"""One-launch store (``kvq_kivi_store``) against the separate launches and
against the oracle.

The key pack, value pack and ring-write entry points are each pinned to the
oracle elsewhere; here one batch of all four kinds of work is applied once
through ``kvq_kivi_store`` and once through the three separate entry points,
from identical starting state, and every output tensor (codes, scales, mins,
both rings, untouched entries included) must be bit-identical.  Pack sources
mix ring rows and input rows; the value rows end mid-wave and include a
skipped (negative) slot; ring writes never target a row the batch packs (the
kernel's precondition).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._util import empty_kivi_caches
from vllm_ascend_quantized_kv_cache.ops.kivi_pack import (
    kivi_store,
    pack_key_rows,
    pack_value_rows,
    ring_write,
)

pytestmark = pytest.mark.gpu

KVH, D, BS, NB, ROWS, CAP, N_IN = 8, 128, 128, 16, 6, 129, 300


def _batch(g, segments, seed):
    gen = torch.Generator().manual_seed(seed)
    n_ring = ROWS * CAP
    perm = torch.randperm(n_ring, generator=gen).tolist()
    inp = torch.randperm(N_IN, generator=gen).tolist()
    used = 0

    def ring_rows(n):
        nonlocal used
        out = perm[used : used + n]
        used += n
        return out

    kp_src, kp_slot = [], []
    if segments == "all":
        # two key groups: one read from ring rows, one from input rows; the
        # first lands at a non-zero group offset of its block when g < BS
        kp_src = ring_rows(g) + [n_ring + x for x in inp[:g]]
        kp_slot = [3 * BS + (BS - g) + i for i in range(g)] + [9 * BS + i for i in range(g)]
    vp_src, vp_slot = [], []
    if segments in ("all", "decode"):
        n = 37  # 37 * 8 rows: the last wave is partly past the end
        vp_src = ring_rows(20) + [n_ring + x for x in inp[g : g + 17]]
        slots = torch.randperm(NB * BS, generator=gen)[:n].tolist()
        slots[5] = -1  # skipped token
        vp_slot = slots
    kr_dst = ring_rows(5)
    kr_src = inp[:5]
    vr_dst = ring_rows(7)
    vr_src = inp[5:12]
    jobs = kp_src + kp_slot + vp_src + vp_slot + kr_src + kr_dst + vr_src + vr_dst
    counts = (len(kp_src), len(vp_src), len(kr_dst), len(vr_dst))
    parts = dict(kp_src=kp_src, kp_slot=kp_slot, vp_src=vp_src, vp_slot=vp_slot,
                 kr_src=kr_src, kr_dst=kr_dst, vr_src=vr_src, vr_dst=vr_dst)
    return jobs, counts, parts


@pytest.mark.parametrize("segments", ["all", "decode", "ring_only"])
@pytest.mark.parametrize("g", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_store_one_launch_matches_separate_launches(gpu_device, segments, g, dtype):
    dev = gpu_device
    gen = torch.Generator().manual_seed(11 + g)
    chan = torch.exp(torch.randn(KVH, D, generator=gen))
    ring_k0 = (torch.randn(ROWS, CAP, KVH, D, generator=gen) * chan).to(dtype)
    ring_v0 = torch.randn(ROWS, CAP, KVH, D, generator=gen).to(dtype)
    in_k = (torch.randn(N_IN, KVH, D, generator=gen) * chan).to(dtype).to(dev)
    in_v = torch.randn(N_IN, KVH, D, generator=gen).to(dtype).to(dev)
    jobs, counts, p = _batch(g, segments, seed=g + len(segments))
    print(f"store case: segments={segments} g={g} dtype={dtype} counts={counts}", flush=True)

    def i64(x):
        return torch.tensor(x, dtype=torch.int64, device=dev)

    # separate launches (packs first, then ring writes)
    caches_a = tuple(t.to(dev) for t in empty_kivi_caches(NB, BS, KVH, D, g, fill=7))
    rk_a, rv_a = ring_k0.to(dev), ring_v0.to(dev)
    if counts[0]:
        pack_key_rows(rk_a.view(-1, KVH, D), in_k, i64(p["kp_src"]), i64(p["kp_slot"]),
                      *caches_a[:3], g)
    if counts[1]:
        pack_value_rows(rv_a.view(-1, KVH, D), in_v, i64(p["vp_src"]), i64(p["vp_slot"]),
                        *caches_a[3:], g)
    ring_write(rk_a, in_k, i64(p["kr_src"]), i64(p["kr_dst"]))
    ring_write(rv_a, in_v, i64(p["vr_src"]), i64(p["vr_dst"]))

    # one launch
    caches_b = tuple(t.to(dev) for t in empty_kivi_caches(NB, BS, KVH, D, g, fill=7))
    rk_b, rv_b = ring_k0.to(dev), ring_v0.to(dev)
    assert kivi_store(in_k, in_v, rk_b, rv_b, i64(jobs), counts, caches_b, g)
    torch.cuda.synchronize()

    names = ("k_quant", "k_scale", "k_mn", "v_quant", "v_scale", "v_mn")
    for name, a, b in zip(names, caches_a, caches_b):
        assert torch.equal(a, b), f"{name} differs"
    assert torch.equal(rk_a, rk_b), "key ring differs"
    assert torch.equal(rv_a, rv_b), "value ring differs"
    # the batch really wrote something in every segment it carries
    assert not torch.equal(rk_b.cpu(), ring_k0) and not torch.equal(rv_b.cpu(), ring_v0)
    if counts[0]:
        assert (caches_b[0] != 7).any()
    if counts[1]:
        assert (caches_b[3] != 7).any()


@pytest.mark.parametrize("g", [64, 128])
def test_store_large_batch_matches_oracle(gpu_device, g):
    """A store batch large enough that each wave of the one-launch kernel
    takes several units (two and four per wave: the counted-wait pipeline),
    its pack sources scattered over ring rows and input rows, checked bit for
    bit against the oracle's packs of the same source rows."""
    dev = gpu_device
    dtype = torch.bfloat16
    nb, rows, cap = 512, 8, 129
    for n_groups, n_val in ((60, 1500), (200, 6000)):
        gen = torch.Generator().manual_seed(5 * g + n_groups)
        chan = torch.exp(torch.randn(KVH, D, generator=gen))
        n_in = n_groups * g + 64
        ring_k = (torch.randn(rows, cap, KVH, D, generator=gen) * chan).to(dtype)
        ring_v = torch.randn(rows, cap, KVH, D, generator=gen).to(dtype)
        in_k = (torch.randn(n_in, KVH, D, generator=gen) * chan).to(dtype)
        in_v = torch.randn(n_in, KVH, D, generator=gen).to(dtype)
        n_ring = rows * cap
        src_k = torch.cat([ring_k.view(-1, KVH, D), in_k])
        src_v = torch.cat([ring_v.view(-1, KVH, D), in_v])
        # key groups: sources anywhere in [ring ; input], whole groups at
        # group-aligned offsets of shuffled blocks
        kp_src = torch.randint(0, n_ring + n_in, (n_groups * g,), generator=gen)
        gpb = BS // g
        blocks = torch.randperm(nb // 2, generator=gen)
        kp_slot = torch.cat([blocks[i // gpb] * BS + (i % gpb) * g + torch.arange(g)
                             for i in range(n_groups)])
        # value rows: distinct slots in the other half of the pool, a few skipped
        vp_src = torch.randint(0, n_ring + n_in, (n_val,), generator=gen)
        vp_slot = nb // 2 * BS + torch.randperm(nb // 2 * BS, generator=gen)[:n_val]
        vp_slot[::97] = -1
        print(f"large store case: g={g} groups={n_groups} values={n_val}", flush=True)
        want = empty_kivi_caches(nb, BS, KVH, D, g, fill=7)
        ref.pack_key_cache(src_k[kp_src], kp_slot, want[0], want[1], want[2], g)
        ref.pack_value_cache(src_v[vp_src], vp_slot, want[3], want[4], want[5], g)
        got = tuple(t.to(dev) for t in empty_kivi_caches(nb, BS, KVH, D, g, fill=7))
        jobs = torch.cat([kp_src, kp_slot, vp_src, vp_slot]).to(torch.int64).to(dev)
        assert kivi_store(in_k.to(dev), in_v.to(dev), ring_k.to(dev), ring_v.to(dev), jobs,
                          (n_groups * g, n_val, 0, 0), got, g)
        torch.cuda.synchronize()
        names = ("k_quant", "k_scale", "k_mn", "v_quant", "v_scale", "v_mn")
        for name, a, b in zip(names, want, got):
            assert torch.equal(a.view(torch.int32), b.cpu().view(torch.int32)), f"{name} differs"
