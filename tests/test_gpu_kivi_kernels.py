# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the KIVI INT4 HIP kernels against the CPU oracle.

Codes, scales and mins must be bit-exact; gathered K/V bit-exact after the
round-to-nearest-even cast; fused decode attention within atol/rtol 1e-2 of
the oracle's dequant followed by fp32 SDPA.
"""

from __future__ import annotations

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._util import empty_kivi_caches, make_kv, shuffled_table, slots_for, to_dev

pytestmark = pytest.mark.gpu

# (head_size, kv_heads, group_size, block_size) -- the reference's geometry sweep
GEOMS = [(32, 2, 8, 16), (64, 4, 16, 32), (128, 8, 128, 128), (128, 4, 32, 64), (256, 2, 64, 64),
         (256, 1, 128, 128), (128, 8, 64, 128)]


def _packs(dev, d, kvh, g, bs, dtype, seed, n_groups=5):
    from vllm_ascend_quantized_kv_cache.ops.kivi_pack import (
        kivi_pack_key_cache,
        kivi_pack_value_cache,
    )

    nb = n_groups * g // bs + 3
    t = n_groups * g
    key, value = make_kv(t, kvh, d, dtype=dtype, seed=seed)
    # groups land in shuffled blocks, group-aligned inside each block
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    gpb = bs // g
    slots = []
    for gi in range(n_groups):
        blk = int(perm[gi // gpb])
        off = (gi % gpb) * g
        slots.extend(range(blk * bs + off, blk * bs + off + g))
    slots = torch.tensor(slots, dtype=torch.int64)
    vslots = slots.clone()
    vslots[3] = -1  # value padding token must be skipped
    cpu = empty_kivi_caches(nb, bs, kvh, d, g, fill=7)
    gpu = to_dev(cpu, dev)
    ref.pack_key_cache(key, slots, cpu[0], cpu[1], cpu[2], g)
    ref.pack_value_cache(value, vslots, cpu[3], cpu[4], cpu[5], g)
    kivi_pack_key_cache(key.to(dev), slots.to(dev), gpu[0], gpu[1], gpu[2], g)
    kivi_pack_value_cache(value.to(dev), vslots.to(torch.int32).to(dev), gpu[3], gpu[4], gpu[5], g)
    return cpu, gpu


@pytest.mark.parametrize("d,kvh,g,bs", GEOMS)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_pack_bit_exact(gpu_device, d, kvh, g, bs, dtype):
    cpu, gpu = _packs(gpu_device, d, kvh, g, bs, dtype, seed=d + g + bs)
    torch.cuda.synchronize()
    for name, a, b in zip(("kq", "ks", "km", "vq", "vs", "vm"), cpu, gpu):
        b = b.cpu()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"{name} differs"


def test_pack_config1_bit_exact(gpu_device):
    """896 packed tokens, 8 heads, D=G=Bs=128."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_pack import (
        kivi_pack_key_cache,
        kivi_pack_value_cache,
    )

    d, kvh, g, bs, nb = 128, 8, 128, 128, 8
    key, value = make_kv(1024, kvh, d, seed=0)
    table = torch.arange(nb, dtype=torch.int32)
    slots = slots_for(table, range(896), bs)
    cpu = empty_kivi_caches(nb, bs, kvh, d, g)
    gpu = to_dev(cpu, gpu_device)
    ref.pack_key_cache(key[:896], slots, *cpu[:3], g)
    ref.pack_value_cache(value[:896], slots, *cpu[3:], g)
    kivi_pack_key_cache(key[:896].to(gpu_device), slots.to(gpu_device), *gpu[:3], g)
    kivi_pack_value_cache(value[:896].to(gpu_device), slots.to(gpu_device), *gpu[3:], g)
    torch.cuda.synchronize()
    for a, b in zip(cpu, gpu):
        assert torch.equal(a.view(torch.int32), b.cpu().view(torch.int32))


def _boundary_values(shape, group_axis_len, seed):
    """fp32 values whose KIVI quotients sit on the x.5 rounding boundaries.

    Every group of ``group_axis_len`` entries along the last axis holds its
    min, its max = min + 15 s, and entries min + (k + 0.5) s nudged by -1, 0
    or +1 ulp, so (x - mn) / scale + 0.5 falls within a few ulps of an integer
    (the cases the reciprocal fast path hands to the exact division).
    """
    import numpy as np

    rng = np.random.default_rng(seed)
    x = np.empty(shape, dtype=np.float32)
    flat = x.reshape(-1, group_axis_len)
    for row in flat:
        mn = np.float32(rng.normal())
        s = np.float32(np.exp(rng.normal()) * 0.1)
        k = rng.integers(0, 15, group_axis_len).astype(np.float32)
        v = (mn + (k + np.float32(0.5)) * s).astype(np.float32)
        nudge = rng.integers(-1, 2, group_axis_len)
        v = np.where(nudge < 0, np.nextafter(v, np.float32(-np.inf)), v)
        v = np.where(nudge > 0, np.nextafter(v, np.float32(np.inf)), v).astype(np.float32)
        v[0] = mn
        v[-1] = np.float32(mn + np.float32(15) * s)
        row[:] = v
    return torch.from_numpy(x)


@pytest.mark.parametrize("d,kvh,g,bs", [(128, 8, 128, 128), (128, 4, 32, 64), (64, 2, 16, 32)])
def test_pack_boundary_quotients_bit_exact(gpu_device, d, kvh, g, bs):
    from vllm_ascend_quantized_kv_cache.ops.kivi_pack import (
        kivi_pack_key_cache,
        kivi_pack_value_cache,
    )

    n_groups = 4
    t = n_groups * g
    nb = t // bs + 2
    # keys group over tokens: build [kvh, d, t] and move tokens first
    key = _boundary_values((kvh, d, t), g, seed=d + g).permute(2, 0, 1).contiguous()
    value = _boundary_values((t, kvh, d), g, seed=d + g + 1)
    table = torch.randperm(nb, generator=torch.Generator().manual_seed(g)).to(torch.int32)
    slots = slots_for(table, range(t), bs)
    cpu = empty_kivi_caches(nb, bs, kvh, d, g)
    gpu = to_dev(cpu, gpu_device)
    ref.pack_key_cache(key, slots, *cpu[:3], g)
    ref.pack_value_cache(value, slots, *cpu[3:], g)
    kivi_pack_key_cache(key.to(gpu_device), slots.to(gpu_device), *gpu[:3], g)
    kivi_pack_value_cache(value.to(gpu_device), slots.to(gpu_device), *gpu[3:], g)
    torch.cuda.synchronize()
    for name, a, b in zip(("kq", "ks", "km", "vq", "vs", "vm"), cpu, gpu):
        assert torch.equal(a.view(torch.int32), b.cpu().view(torch.int32)), f"{name} differs"


@pytest.mark.parametrize("d,kvh,g,bs", GEOMS)
def test_gather_bit_exact(gpu_device, d, kvh, g, bs):
    from vllm_ascend_quantized_kv_cache.ops.kivi_gather import kivi_dequant_gather_cache

    cpu, gpu = _packs(gpu_device, d, kvh, g, bs, torch.bfloat16, seed=11 + d, n_groups=8)
    nb = cpu[0].shape[0]
    # three ragged requests over a shuffled table; unused columns hold -1
    maxb = 4
    table = torch.full((3, maxb), -1, dtype=torch.int32)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(5))
    lens = [min(maxb * bs, 3 * bs + 5), bs - 3, 1]
    used = 0
    for r, n in enumerate(lens):
        nblk = -(-n // bs)
        table[r, :nblk] = perm[used : used + nblk]
        used += nblk
    seq = torch.tensor(lens, dtype=torch.int64)
    for out_dtype in (torch.bfloat16, torch.float32, torch.float16):
        want_k, want_v = ref.dequant_gather(*cpu, table, seq, out_dtype, g)
        got_k, got_v = kivi_dequant_gather_cache(
            *gpu, table.to(gpu_device), seq.to(gpu_device), out_dtype, g
        )
        assert torch.equal(want_k, got_k.cpu()), out_dtype
        assert torch.equal(want_v, got_v.cpu()), out_dtype


def _ring_case(dev, d, kvh, g, bs, r_len, lens, seed, ring_dtype=torch.float32, split=None,
               stale=False, make=None):
    """Packed history for several requests plus residual rings (FIFO, wrapped).

    ``split(n) -> (hist_k, hist_v)``: the int4 history of each side (default:
    the incremental rule, ``ref.incremental_split``).  ``stale``: the bytes no
    pack writes hold NaN scales and minima and nonzero codes, as a reused
    page would, so a read past a request's int4 history shows.  ``make(n, kvh,
    d, seed) -> (key, value)``: the request's K/V (default ``make_kv``)."""
    nb = sum(-(-n // bs) for n in lens) + 2
    maxb = max(-(-n // bs) for n in lens)
    table = torch.full((len(lens), maxb), -1, dtype=torch.int32)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    used = 0
    for r, n in enumerate(lens):
        nblk = -(-n // bs)
        table[r, :nblk] = perm[used : used + nblk]
        used += nblk
    cpu = empty_kivi_caches(nb, bs, kvh, d, g)
    if stale:
        for t in (cpu[1], cpu[2], cpu[4], cpu[5]):
            t.fill_(float("nan"))
        cpu[0].fill_(0x77777777)
        cpu[3].fill_(0x77777777)
    ring_k = torch.zeros(len(lens) + 1, r_len, kvh, d, dtype=ring_dtype)
    ring_v = torch.zeros_like(ring_k)
    seqs, windows_k, windows_v, keys, values = [], [], [], [], []
    gen = torch.Generator().manual_seed(seed + 1)
    for b, n in enumerate(lens):
        key, value = (make or (lambda n_, h_, d_, sd: make_kv(n_, h_, d_, seed=sd)))(
            n, kvh, d, seed * 31 + b)
        keys.append(key)
        values.append(value)
        hk, hv = split(n) if split else ref.incremental_split(n, r_len)
        slots = slots_for(table[b], range(n), bs)
        if hk:
            ref.pack_key_cache(key[:hk], slots[:hk], *cpu[:3], g)
        if hv:
            ref.pack_value_cache(value[:hv], slots[:hv], *cpu[3:], g)
        row = len(lens) - b  # rows need not follow request order
        ks_ = int(torch.randint(0, r_len, (1,), generator=gen))  # ring start
        vs_ = int(torch.randint(0, r_len, (1,), generator=gen))
        tk, tv = n - hk, n - hv
        for i in range(tk):
            ring_k[row, (ks_ + i) % r_len] = key[hk + i].to(ring_dtype)
        for i in range(tv):
            ring_v[row, (vs_ + i) % r_len] = value[hv + i].to(ring_dtype)
        seqs.append((n, hk, hv, row, ks_, vs_))
        windows_k.append(key[hk:])
        windows_v.append(value[hv:])
    return cpu, table, ring_k, ring_v, seqs, windows_k, windows_v, keys, values


@pytest.mark.parametrize("d,kvh,g,bs", GEOMS)
def test_gather_with_residual_overlay(gpu_device, d, kvh, g, bs):
    from vllm_ascend_quantized_kv_cache.ops.kivi_gather import gather_dequant_with_residual

    r_len = max(g, 2 * g if g <= 64 else g)
    lens = [r_len * 3 + 5, r_len // 2, r_len + 1, 2 * r_len]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=3
    )
    seq_t = torch.tensor(lens)
    want_k, want_v = ref.dequant_gather(*cpu, table, seq_t, torch.bfloat16, g)
    want_k = ref.overlay_residual(want_k, lens, wk)
    want_v = ref.overlay_residual(want_v, lens, wv)
    meta = torch.tensor(
        [[row, ks_, n - hk, vs_, n - hv] for (n, hk, hv, row, ks_, vs_) in seqs],
        dtype=torch.int32,
    )
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int64)
    got_k, got_v = gather_dequant_with_residual(
        to_dev(cpu, gpu_device), table.to(gpu_device), cu.to(gpu_device), sum(lens),
        torch.bfloat16, g, meta.to(gpu_device), ring_k.to(gpu_device), ring_v.to(gpu_device),
    )
    assert torch.equal(want_k, got_k.cpu())
    assert torch.equal(want_v, got_v.cpu())


@pytest.mark.parametrize("g,bs,kvh,index_dtype", [(64, 128, 8, torch.int32),
                                                   (128, 128, 8, torch.int64),
                                                   (64, 64, 4, torch.int32)])
def test_gather_of_many_pages_matches_oracle(gpu_device, g, bs, kvh, index_dtype):
    """Thousands of (page, head) units of the d = 128 gather: more workgroups
    than the device holds at once, units past a request's end (a ragged batch
    over a wide table), and requests whose tails come from the rings (none,
    part of a page, more than a page, the whole request).  Pages hold random
    codes, scales and minima."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_gather import gather_dequant_with_residual

    d = 128
    lens = [20000, 7001, 15000, 129]
    tails = [(128, 5), (0, 0), (77, 128), (1, 129)]  # (k_tail, v_tail) rows from the rings
    r_len = 256
    gen = torch.Generator().manual_seed(17)
    nblk = [-(-n // bs) for n in lens]
    nb = sum(nblk) + 3
    maxb = max(nblk)
    table = torch.full((len(lens), maxb), -1, dtype=index_dtype)
    perm = torch.randperm(nb, generator=gen)
    used = 0
    for r, n in enumerate(nblk):
        table[r, :n] = perm[used : used + n].to(index_dtype)
        used += n
    kq = torch.randint(-2**31, 2**31, (nb, kvh, d, bs // 8), generator=gen, dtype=torch.int64)
    vq = torch.randint(-2**31, 2**31, (nb, bs, kvh, d // 8), generator=gen, dtype=torch.int64)
    kq, vq = kq.to(torch.int32), vq.to(torch.int32)
    ks = torch.rand((nb, kvh, d, bs // g), generator=gen) + 0.01
    km = torch.randn((nb, kvh, d, bs // g), generator=gen)
    vs = torch.rand((nb, bs, kvh, d // g), generator=gen) + 0.01
    vm = torch.randn((nb, bs, kvh, d // g), generator=gen)
    cpu = (kq, ks, km, vq, vs, vm)
    ring_k = torch.randn((len(lens), r_len, kvh, d), generator=gen).to(torch.bfloat16)
    ring_v = torch.randn((len(lens), r_len, kvh, d), generator=gen).to(torch.bfloat16)
    meta, wk, wv = [], [], []
    for b, (kt, vt) in enumerate(tails):
        row = len(lens) - 1 - b
        kf, vf = (37 * b + 11) % r_len, (53 * b + 200) % r_len
        meta.append([row, kf, kt, vf, vt])
        wk.append(ring_k[row, [(kf + i) % r_len for i in range(kt)]])
        wv.append(ring_v[row, [(vf + i) % r_len for i in range(vt)]])
    meta = torch.tensor(meta, dtype=torch.int32)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int64)
    for out_dtype in (torch.bfloat16, torch.float32):
        want_k, want_v = ref.dequant_gather(*cpu, table, torch.tensor(lens), out_dtype, g)
        want_k = ref.overlay_residual(want_k, lens, wk)
        want_v = ref.overlay_residual(want_v, lens, wv)
        got_k, got_v = gather_dequant_with_residual(
            to_dev(cpu, gpu_device), table.to(gpu_device), cu.to(gpu_device), sum(lens),
            out_dtype, g, meta.to(gpu_device), ring_k.to(gpu_device), ring_v.to(gpu_device),
        )
        assert torch.equal(want_k, got_k.cpu()), out_dtype
        assert torch.equal(want_v, got_v.cpu()), out_dtype


@pytest.mark.parametrize("d,kvh,g,bs", GEOMS)
@pytest.mark.parametrize("rep", [1, 5])
def test_decode_attention_matches_oracle(gpu_device, d, kvh, g, bs, rep):
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, kivi_decode_attention

    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 4 + 7, r_len + 1, 5, 3 * r_len, r_len * 6]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=9, ring_dtype=torch.bfloat16
    )
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    scale = d ** -0.5
    # the reference gather in fp32 (its exact dequant values), then fp32 SDPA;
    # a bf16 target would add the reference's own intermediate rounding
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    for split in (None, 64, 256):
        got = kivi_decode_attention(
            q.to(gpu_device), to_dev(cpu, gpu_device), table.to(gpu_device), dseqs,
            ring_k.to(gpu_device), ring_v.to(gpu_device), scale, g, split_tokens=split,
        )
        torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("kvh,g,bs,rep", [
    (8, 32, 64, 8),     # 32-token tiles, 4 value groups per token
    (16, 64, 128, 2),   # two value groups per head, key scales gathered per tile
    (8, 128, 256, 7),   # one value group per head; two key groups per page
    (8, 128, 128, 12),  # GQA group above 8 (two score MFMAs); one key group per page
    (4, 64, 128, 8),    # kv heads not a multiple of 8
])
def test_decode_head_group_geometries(gpu_device, kvh, g, bs, rep):
    """Decode across the kernel's tile forms: tile size, value groups per
    head, key-scale DMA form, folded and unfolded score MFMAs."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, kivi_decode_attention

    d = 128
    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 9 + 3, r_len + 5, r_len * 5]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=21, ring_dtype=torch.bfloat16
    )
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    for split in (None, 256):
        got = kivi_decode_attention(
            q.to(gpu_device), to_dev(cpu, gpu_device), table.to(gpu_device), dseqs,
            ring_k.to(gpu_device), ring_v.to(gpu_device), scale, g, split_tokens=split,
        )
        torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("kvh,g,bs,rep", [(8, 128, 128, 5), (8, 32, 64, 4), (4, 64, 256, 8)])
def test_decode_tail_int4_values_match_oracle(gpu_device, kvh, g, bs, rep):
    """Tails whose values are int4: the key window reaches further back than the
    value window (hist_k < hist_v), so the tail's first positions pair ring keys
    with int4 values; tails start off the 32-position grid and cross pages."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        plan_decode_pieces,
    )

    d = 128
    r_len = 3 * g

    def split(n):  # keys: whole groups, at least g + 1 in the ring; values: 0-9 in the ring
        hk = max(0, (n - g - 1) // g * g)
        return hk, max(hk, n - n % 10)

    lens = [5 * g + 37, 2 * g + 1, 3 * g - 11, 7 * g + 64, 41]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=33, ring_dtype=torch.bfloat16, split=split
    )
    assert any(hv > hk for (_, hk, hv, *_r) in seqs)
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    plans = [None, 64]
    for split_tokens in plans:
        got = kivi_decode_attention(
            q.to(gpu_device), to_dev(cpu, gpu_device), table.to(gpu_device), dseqs,
            ring_k.to(gpu_device), ring_v.to(gpu_device), scale, g, split_tokens=split_tokens,
        )
        torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)
    # pieces cut on few CUs: a wave walks several tail items of several requests
    meta, work, pieces = plan_decode_pieces(dseqs, kvh, cu_count=3)
    plan = tuple(torch.from_numpy(x).to(gpu_device) for x in (meta, work, pieces))
    got = kivi_decode_attention(
        q.to(gpu_device), to_dev(cpu, gpu_device), table.to(gpu_device), dseqs,
        ring_k.to(gpu_device), ring_v.to(gpu_device), scale, g, plan=plan,
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("kvh,g,bs,rep", [(8, 128, 128, 5), (8, 64, 128, 8), (4, 32, 64, 4)])
@pytest.mark.parametrize("cu_count", [1, 3, 256])
def test_decode_pieces_match_oracle(gpu_device, kvh, g, bs, rep, cu_count):
    """Equal-cost pieces: one wave per (piece, kv head) walks several items of
    several requests, int4 and tail alike (few CUs: many items per piece; int4
    items that start mid key group), in the kernel's single pass."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        plan_decode_pieces,
    )

    d = 128
    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 9 + 3, 1, r_len + 5, 0, r_len * 5 + 64, 77]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=33, ring_dtype=torch.bfloat16
    )
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    meta, work, pieces = plan_decode_pieces(dseqs, kvh, cu_count)
    print(f"pieces case kvh={kvh} g={g} cu={cu_count}: {len(work)} items, "
          f"{len(pieces) - 1} pieces", flush=True)
    dev = gpu_device
    got = kivi_decode_attention(
        q.to(dev), to_dev(cpu, dev), table.to(dev), dseqs, ring_k.to(dev), ring_v.to(dev),
        scale, g, plan=(torch.from_numpy(meta).to(dev), torch.from_numpy(work).to(dev),
                        torch.from_numpy(pieces).to(dev)),
    )
    # rows of empty requests are the empty sum (zeros) in both
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("g,rep,dtype", [(128, 5, torch.bfloat16), (64, 8, torch.float16),
                                         (64, 16, torch.bfloat16), (128, 12, torch.float16)])
@pytest.mark.parametrize("tile,cu_count", [(128, 256), (128, 1), (64, 3)])
def test_page_streaming_decode_matches_oracle(gpu_device, g, rep, dtype, tile, cu_count):
    """The page-streaming decode (8 kv heads, block 128, head size 128): one
    workgroup per piece streams whole pages for all heads.  Pieces on page
    bounds (tile 128) and on 64-position bounds (items that start and end
    mid-page), a single piece holding every item (the stage stream crosses
    requests), folded (<= 8) and unfolded GQA groups up to 16, both 16-bit
    dtypes, and NaN scales in every byte past the int4 histories, which the
    masked positions of a page must not reach."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        plan_decode_pieces,
    )

    d, kvh, bs = 128, 8, 128
    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 9 + 3, 1, 700, 0, r_len * 5 + 64, 77, 2 * bs + 1, 3 * bs]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=41, ring_dtype=dtype, stale=True
    )
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(8)).to(dtype)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q.float(), dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    meta, work, pieces = plan_decode_pieces(dseqs, kvh, cu_count, tile=tile)
    print(f"page-streaming case g={g} rep={rep} {dtype} tile={tile} cu={cu_count}: "
          f"{len(work)} items, {len(pieces) - 1} pieces", flush=True)
    dev = gpu_device
    got = kivi_decode_attention(
        q.to(dev), to_dev(cpu, dev), table.to(dev), dseqs, ring_k.to(dev), ring_v.to(dev),
        scale, g, plan=(torch.from_numpy(meta).to(dev), torch.from_numpy(work).to(dev),
                        torch.from_numpy(pieces).to(dev)),
    ).float().cpu()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("d,kvh,g,bs", [(128, 8, 128, 128), (128, 8, 64, 128), (128, 4, 32, 64),
                                         (64, 4, 16, 32)])
@pytest.mark.parametrize("split", [128, 256])
def test_decode_paired_items_match_oracle(gpu_device, d, kvh, g, bs, split):
    """Paired int4 items (even / odd 64-position chunks of one range, on one
    XCD) through the MFMA kernel, 32-token tiles included, and through the
    generic kernel (D = 64)."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        plan_decode_work,
    )

    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 9 + 3, 1, r_len + 5, 0, r_len * 5 + 64, 77, 700]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=41, ring_dtype=torch.bfloat16
    )
    rep = 5
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    meta, work = plan_decode_work(dseqs, split, paired=True)
    print(f"paired case d={d} g={g} split={split}: {len(work)} items", flush=True)
    dev = gpu_device
    got = kivi_decode_attention(
        q.to(dev), to_dev(cpu, dev), table.to(dev), dseqs, ring_k.to(dev), ring_v.to(dev),
        scale, g, plan=(torch.from_numpy(meta).to(dev), torch.from_numpy(work).to(dev)),
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


def test_mfma_lane_layout(gpu_device):
    """The 16x16x32 f16 MFMA lane mapping the decode kernels assume."""
    from vllm_ascend_quantized_kv_cache.ops import _native

    g = torch.Generator().manual_seed(0)
    a = torch.randint(-4, 5, (16, 32), generator=g).to(torch.float16)
    b = torch.randint(-4, 5, (32, 16), generator=g).to(torch.float16)
    da, db = a.to(gpu_device), b.to(gpu_device)
    d = torch.empty(16, 16, dtype=torch.float32, device=gpu_device)
    rc = _native.lib().kvq_selftest_mfma_f16(
        da.data_ptr(), db.data_ptr(), d.data_ptr(), _native.stream_of(d)
    )
    _native.check(rc, "kvq_selftest_mfma_f16")
    assert torch.equal(d.cpu(), a.float() @ b.float())


def test_lane_reductions(gpu_device):
    """The permlane / DPP reductions the kernels use: the four-row max and sum
    (the sum in the shuffle form's order, bit for bit), the whole-wave max and
    sum (every lane the same value), and the paired four-row max."""
    from vllm_ascend_quantized_kv_cache.ops import _native

    g = torch.Generator().manual_seed(6)
    x = (torch.rand(16, 64, generator=g, dtype=torch.float64) - 0.5) * 2.0 ** torch.randint(
        -20, 20, (16, 64), generator=g, dtype=torch.int64).double()
    x = x.float()
    x[3, 17] = float("-inf")  # a masked score
    dx = x.to(gpu_device).contiguous()
    out = torch.empty(16, 64, 6, dtype=torch.float32, device=gpu_device)
    rc = _native.lib().kvq_selftest_lane_reductions(dx.data_ptr(), out.data_ptr(),
                                                    _native.stream_of(out))
    _native.check(rc, "kvq_selftest_lane_reductions")
    out = out.cpu()
    lanes = torch.arange(64)

    def max4(v):
        return torch.maximum(torch.maximum(v, v[lanes ^ 16]), torch.maximum(v[lanes ^ 32], v[lanes ^ 48]))

    for t in range(16):
        v = x[t]
        m4 = max4(v)
        s1 = v + v[lanes ^ 16]  # float32 adds, the shuffle form's order
        s4 = s1 + s1[lanes ^ 32]
        assert torch.equal(out[t, :, 0], m4), t
        # the paired form: each value gets its own four-row max, not the other's
        assert torch.equal(out[t, :, 4], m4), t
        assert torch.equal(out[t, :, 5], max4(x[(t + 1) % 16])), t
        assert torch.equal(out[t, :, 1], s4), t
        assert torch.equal(out[t, :, 2], torch.full((64,), float(v.max()))), t
        ws = out[t, :, 3]
        assert torch.equal(ws, ws[:1].expand(64)), t
        exact = float(v.double().sum())
        if torch.isfinite(v).all():
            assert abs(float(ws[0]) - exact) <= 1e-5 * float(v.double().abs().sum()), t
        else:
            assert float(ws[0]) == exact, t


def test_lds_dma_lane_layout(gpu_device):
    """global_load_lds writes lane i's bytes at LDS base + size * i (16 B and 4 B lanes)."""
    from vllm_ascend_quantized_kv_cache.ops import _native

    src = torch.randint(0, 2**31 - 1, (320,), dtype=torch.int32,
                        generator=torch.Generator().manual_seed(4))
    dsrc = src.to(gpu_device)
    dst = torch.zeros(320, dtype=torch.int32, device=gpu_device)
    rc = _native.lib().kvq_selftest_lds_dma(dsrc.data_ptr(), dst.data_ptr(),
                                            _native.stream_of(dst))
    _native.check(rc, "kvq_selftest_lds_dma")
    assert torch.equal(dst.cpu(), src)


@pytest.mark.parametrize("kvh,g,bs,rep,dtype",
                         [(8, 128, 128, 5, torch.bfloat16), (8, 64, 128, 8, torch.float16),
                          (4, 32, 64, 4, torch.bfloat16)])
def test_decode_with_row_maxima_growing_every_page(gpu_device, kvh, g, bs, rep, dtype):
    """Keys along one direction per kv head with a magnitude that grows with
    the position (even heads) or shrinks (odd heads), queries along it: every
    page and tail tile raises the even heads' running maximum, so the softmax
    rescales at each one, in the page-streaming decode (8 kv heads) and the
    per-wave one (4), int4 pages and tails alike."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        page_streaming_applies,
    )

    d = 128
    r_len = 2 * g if g <= 64 else g
    lens = [r_len * 7 + 3, r_len * 2 + 64, 700]
    u = torch.randn(kvh, d, generator=torch.Generator().manual_seed(17))
    u = u / u.norm(dim=1, keepdim=True)
    sign = torch.tensor([1.0 if h % 2 == 0 else -1.0 for h in range(kvh)])

    def make(n, h_, d_, sd):
        gen = torch.Generator().manual_seed(sd)
        pos = torch.arange(n, dtype=torch.float32)
        key = u[None] * (sign[None, :, None] * 0.05 * pos[:, None, None]) + 0.05 * torch.randn(
            n, h_, d_, generator=gen)
        value = torch.randn(n, h_, d_, generator=gen)
        return key.to(dtype), value.to(dtype)

    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=51, ring_dtype=dtype, make=make
    )
    hq = kvh * rep
    q = (8.0 * u.repeat_interleave(rep, dim=0)[None].expand(len(lens), hq, d)
         + 0.05 * torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(9)))
    q = q.to(dtype)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    assert page_streaming_applies(hq, kvh, d, bs, g, dtype, dtype) == (kvh == 8)
    dev = gpu_device
    # the default plan: pieces on page bounds for the page-streaming decode
    got = kivi_decode_attention(
        q.to(dev), to_dev(cpu, dev), table.to(dev), dseqs, ring_k.to(dev), ring_v.to(dev),
        scale, g,
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


def test_decode_combine_of_many_items_per_request(gpu_device):
    """Split plans of 128 positions: one request in 158 items (the
    combine's (m, l) pass and weighted sum run in three 64-item chunks), one
    in 17 (one past the rows the combine preloads), one in 16, and a short
    one, against the oracle."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        kivi_decode_attention,
        plan_decode_work,
    )

    d, kvh, g, bs, rep = 128, 8, 128, 128, 5
    r_len = g
    # int4 items of 128 up to min(k_hist, v_hist), then two 64-position tail items
    lens = [20005, 15 * 128 + 10, 14 * 128 + 8, 70]
    cpu, table, ring_k, ring_v, seqs, wk, wv, _, _ = _ring_case(
        gpu_device, d, kvh, g, bs, r_len, lens, seed=61, ring_dtype=torch.bfloat16
    )
    dseqs = [DecodeSeq(n, hk, hv, row, ks_, vs_) for (n, hk, hv, row, ks_, vs_) in seqs]
    meta, _ = plan_decode_work(dseqs, 128)
    items = meta[:, 7].tolist()
    assert items[0] > 128 and items[1] == 17 and items[2] == 16, items
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    scale = d ** -0.5
    dk, dv = ref.dequant_gather(*cpu, table, torch.tensor(lens), torch.float32, g)
    dk = ref.overlay_residual(dk, lens, wk)
    dv = ref.overlay_residual(dv, lens, wv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    got = kivi_decode_attention(
        q.to(gpu_device), to_dev(cpu, gpu_device), table.to(gpu_device), dseqs,
        ring_k.to(gpu_device), ring_v.to(gpu_device), scale, g, split_tokens=128,
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)
