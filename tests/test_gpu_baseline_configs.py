# SPDX-License-Identifier: Apache-2.0
"""GPU parity at the BASELINE workloads' full sizes.

Each test builds its configuration's real state on the GPU through the
attention mixins -- KIVI bound to the host's two byte buffers, which the
mixin slices into its six views, as a vLLM-HUST host hands them over
(reference ``tests/test_kivi_int4.py:1396-1481``) -- runs one step of the
configuration's path through ``forward`` and compares with the oracle on the
CPU on the same inputs:

* packed int4 pages (codes, fp32 scales and minima), int8 pages, INT8 scales,
  residual rings and gathered dense K/V: bit-exact;
* attention outputs: within atol/rtol 1e-2 of the oracle's fp32 attention
  over the reference dequant.

Sizes are the configurations' own (configs 1-5); where the CPU oracle would
take minutes, a stated subset of requests or heads is compared (config 5:
4 of 256 requests; config 4 and config 2's prefill: 2 requests, KV heads 0
and 7 with their query heads), while the GPU still runs the whole batch, so
the planner takes the paths it takes at full size.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import kvq_oracle as ref
from vllm_ascend_quantized_kv_cache.methods.int8_dynamic.attention_backend import (
    AscendInt8AttentionBackendMixin,
)
from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import attention_backend as ab
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.byte_cache import (
    KiviByteCacheLayout,
    kivi_caches_from_byte_tensors,
)

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-2, rtol=1e-2)


# ---------------------------------------------------------------------------
# builders
# ---------------------------------------------------------------------------


def _kivi_on_bytes(device, *, hq, kvh, d, g, r, nb, bs, rows):
    """A KIVI mixin bound to two zeroed uint8 page buffers ``(NB, Bs, KVH, S)``."""

    class Impl(ab.AscendKiviInt4AttentionBackendMixin):
        pass

    impl = Impl()
    impl.num_heads, impl.num_kv_heads, impl.head_size = hq, kvh, d
    impl.scale = d ** -0.5
    impl._init_kivi_state(None)
    impl.enable_kivi = True
    impl.kivi_group_size, impl.kivi_residual_length = g, r
    impl.kivi_max_num_seqs = rows
    layout = KiviByteCacheLayout(nb, bs, kvh, d, g)
    kbuf = torch.zeros((nb, bs, kvh, layout.bytes_per_token_head), dtype=torch.uint8,
                       device=device)
    vbuf = torch.zeros_like(kbuf)
    impl._bind_kivi_cache((kbuf, vbuf))
    return impl, kbuf, vbuf, layout


def _md(state, **kw):
    base = dict(attn_state=SimpleNamespace(name=state), causal=True, finished_req_ids=None)
    base.update(kw)
    return SimpleNamespace(**base)


def _table(nblk: list[int], nb: int, seed: int) -> torch.Tensor:
    """Block table over a random permutation of the pool (padding block 0)."""
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    table = torch.zeros((len(nblk), max(nblk)), dtype=torch.int64)
    used = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[used:used + n]
        used += n
    return table


def _slots(row: torch.Tensor, p0: int, p1: int, bs: int) -> torch.Tensor:
    pos = torch.arange(p0, p1)
    return row[pos // bs] * bs + pos % bs


def _rand_kv(device, n, kvh, d, seed, key_scales):
    """Seeded N(0,1) K/V in bf16 on the GPU; keys times per-channel scales."""
    gen = torch.Generator(device=device).manual_seed(seed)
    k = (torch.randn((n, kvh, d), generator=gen, device=device)
         * key_scales.to(device)).to(torch.bfloat16)
    v = torch.randn((n, kvh, d), generator=gen, device=device).to(torch.bfloat16)
    return k, v


def _oracle_pages(layout, seqs, g):
    """Zeroed CPU byte buffers with every request's history packed by the oracle.

    ``seqs``: ``(keys, values, slots, hist_k, hist_v)`` per request.
    """
    kbuf = torch.zeros((layout.num_blocks, layout.block_size, layout.num_kv_heads,
                        layout.bytes_per_token_head), dtype=torch.uint8)
    vbuf = torch.zeros_like(kbuf)
    views = kivi_caches_from_byte_tensors(kbuf, vbuf, layout)
    for k, v, slots, hk, hv in seqs:
        ref.pack_key_cache(k[:hk], slots[:hk], *views[:3], g)
        ref.pack_value_cache(v[:hv], slots[:hv], *views[3:], g)
    return kbuf, vbuf, views


def _ring_rows(impl, req: str, is_key: bool) -> torch.Tensor:
    ring = impl._kivi_ring
    row = impl._get_kivi_residual_row(req, create=False)
    return ring.tensor(is_key)[row, ring.lanes(row, is_key=is_key)].cpu()


def _incremental(n: int, r: int) -> tuple[int, int]:
    """``(hist_k, hist_v)`` after ``n`` tokens written one step at a time."""
    return ((n - 1) // r) * r if n else 0, max(0, n - r)


# ---------------------------------------------------------------------------
# config 1: KIVI round trip, 1 x 1024 tokens
# ---------------------------------------------------------------------------


def test_config1_pack_and_gather_round_trip_full_size(gpu_device):
    kvh, d, g, r, bs, n = 8, 128, 128, 128, 128, 1024
    nb = n // bs
    gen = torch.Generator().manual_seed(0)
    key_scales = torch.exp(torch.randn((kvh, d), generator=gen))
    table = _table([nb], nb, seed=1)  # pages 0..7, shuffled
    impl, kbuf, vbuf, layout = _kivi_on_bytes(gpu_device, hq=kvh, kvh=kvh, d=d, g=g, r=r,
                                             nb=nb, bs=bs, rows=1)
    k, v = _rand_kv(gpu_device, n, kvh, d, 7, key_scales)
    slots = _slots(table[0], 0, n, bs)
    impl._write_kivi_cache(k, v, slots.to(gpu_device), ["r"], [n])
    hk, hv = _incremental(n, r)
    assert (hk, hv) == (896, 896)
    kc, vc = k.cpu(), v.cpu()
    want_k, want_v, views = _oracle_pages(layout, [(kc, vc, slots, hk, hv)], g)
    assert torch.equal(kbuf.cpu(), want_k) and torch.equal(vbuf.cpu(), want_v)
    assert torch.equal(_ring_rows(impl, "r", True), kc[hk:])
    assert torch.equal(_ring_rows(impl, "r", False), vc[hv:])
    gk, gv = impl._gather_dequant_kivi_paged_cache(table.to(gpu_device), [n], torch.bfloat16,
                                                   ["r"])
    dk, dv = ref.dequant_gather(*views, table, torch.tensor([n]), torch.bfloat16, g)
    assert torch.equal(gk.cpu(), ref.overlay_residual(dk, [n], [kc[hk:]]))
    assert torch.equal(gv.cpu(), ref.overlay_residual(dv, [n], [vc[hv:]]))


# ---------------------------------------------------------------------------
# configs 3 and 5: KIVI INT4 decode step (store + fused decode)
# ---------------------------------------------------------------------------


def _kivi_decode_step(device, *, b, hq, kvh, d, g, r, bs, lens, check, seed):
    """Write every request's context through the mixin, run one DecodeOnly step
    for the whole batch, and compare the requests in ``check`` with the oracle."""
    nblk = [-(-(n + 1) // bs) for n in lens]
    nb = sum(nblk) + 8
    gen = torch.Generator().manual_seed(seed)
    key_scales = torch.exp(torch.randn((kvh, d), generator=gen))
    table = _table(nblk, nb, seed=seed + 1)
    impl, kbuf, vbuf, layout = _kivi_on_bytes(device, hq=hq, kvh=kvh, d=d, g=g, r=r, nb=nb,
                                             bs=bs, rows=b)
    reqs = [f"r{i}" for i in range(b)]
    new_k, new_v, kept = [], [], {}
    for i, n in enumerate(lens):
        k, v = _rand_kv(device, n + 1, kvh, d, seed + 100 + i, key_scales)
        impl._write_kivi_cache(k[:n], v[:n], _slots(table[i], 0, n, bs).to(device), [reqs[i]],
                               [n])
        new_k.append(k[n].clone())
        new_v.append(v[n].clone())
        if i in check:
            kept[i] = (k.cpu(), v.cpu())
        del k, v
    q = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16)
    new_slots = torch.stack([_slots(table[i], n, n + 1, bs)[0] for i, n in enumerate(lens)])
    lens1 = [n + 1 for n in lens]
    out = torch.zeros((b, hq, d), dtype=torch.bfloat16, device=device)
    md = _md("DecodeOnly", seq_lens_list=lens1, slot_mapping=new_slots.to(device),
             block_tables=table.to(device), req_ids=reqs, num_actual_tokens=b)
    impl.forward(None, q.to(device), torch.stack(new_k), torch.stack(new_v), (kbuf, vbuf), md,
                 out)
    torch.cuda.synchronize()

    # the checked requests' pages: copy them out under renumbered block ids
    rows = sorted(check)
    sub_blocks = torch.cat([table[i, :nblk[i]] for i in rows])
    remap = torch.full((nb,), -1, dtype=torch.int64)
    remap[sub_blocks] = torch.arange(sub_blocks.numel())
    sub_table = torch.stack([torch.cat([remap[table[i, :nblk[i]]],
                                        torch.zeros(max(nblk) - nblk[i], dtype=torch.int64)])
                             for i in rows])
    sub_layout = KiviByteCacheLayout(sub_blocks.numel(), bs, kvh, d, g)
    idx = sub_blocks.to(device)
    # the six views span the whole buffer ([quant | scale | mn]), so pages
    # are picked per view
    got = [t.index_select(0, idx).cpu() for t in impl._kivi_caches()]
    seqs, win_k, win_v = [], [], []
    for j, i in enumerate(rows):
        kc, vc = kept[i]
        hk, hv = _incremental(lens1[i], r)
        seqs.append((kc, vc, _slots(sub_table[j], 0, lens1[i], bs), hk, hv))
        win_k.append(kc[hk:])
        win_v.append(vc[hv:])
        assert torch.equal(_ring_rows(impl, reqs[i], True), kc[hk:]), f"key ring {i}"
        assert torch.equal(_ring_rows(impl, reqs[i], False), vc[hv:]), f"value ring {i}"
    _, _, views = _oracle_pages(sub_layout, seqs, g)
    for name, a, w in zip(("k_quant", "k_scale", "k_mn", "v_quant", "v_scale", "v_mn"), got,
                          views):
        assert torch.equal(a, w), f"{name} pages differ from the oracle"
    sub_lens = [lens1[i] for i in rows]
    # the fused decode is held to the reference gather's exact (fp32) dequant
    # values followed by fp32 attention
    dk, dv = ref.dequant_gather(*views, sub_table, torch.tensor(sub_lens), torch.float32, g)
    dk = ref.overlay_residual(dk, sub_lens, win_k)
    dv = ref.overlay_residual(dv, sub_lens, win_v)
    want = ref.attention(q[rows], dk, dv, [1] * len(rows), sub_lens, d ** -0.5, causal=True)
    torch.testing.assert_close(out.cpu()[rows].float(), want, **TOL)
    return kbuf


def test_config3_decode_step_full_batch(gpu_device):
    """Config 3: 32 requests, L ~ U[2048, 16384] (seed 0), Hq 40, G = R = Bs =
    128; all 32 requests checked (one round of equal-cost pieces)."""
    b = 32
    lens = torch.randint(2048, 16385, (b,), generator=torch.Generator().manual_seed(0)).tolist()
    _kivi_decode_step(gpu_device, b=b, hq=40, kvh=8, d=128, g=128, r=128, bs=128, lens=lens,
                      check=set(range(b)), seed=0)


def test_config5_decode_step_full_batch(gpu_device):
    """Config 5: 256 x 32768 tokens, Hq 64, G 64 (S = 80 B), 65,800 shuffled
    pages (10.8 GB, past 2^31 bytes per side); the whole batch runs through
    forward() on the page-streaming decode (eight rounds of pieces, then the
    last round in pieces of half the cost), and requests 0, 85, 170 and 255
    (the last pieces) are compared with the oracle."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, plan_decode

    b, n = 256, 32768
    seqs = [DecodeSeq(n + 1, *_incremental(n + 1, 128))] * b
    # without page streaming the plan at this size is split items, no pieces
    assert plan_decode(seqs, 8)[2] is None
    pieces = plan_decode(seqs, 8, page_streaming=True)[2]
    assert pieces is not None and len(pieces) - 1 == 256 * 8 + 512
    kbuf = _kivi_decode_step(gpu_device, b=b, hq=64, kvh=8, d=128, g=64, r=128, bs=128,
                             lens=[n] * b, check={0, 85, 170, 255}, seed=5)
    assert kbuf.numel() > 2 ** 31


# ---------------------------------------------------------------------------
# config 4: KIVI chunked prefill over an int4 prefix (the fall-through path)
# ---------------------------------------------------------------------------


def test_config4_chunk_over_int4_prefix_full_size(gpu_device):
    """8 requests of an 8192-token int4-cached prefix plus a 2048-token chunk:
    the chunk's store (window flushes into int4), the gather of 8 x 10240
    tokens with the residual overlay (bit-exact), and causal attention of the
    chunk over them (requests 0 and 7, KV heads 0 and 7 with their query
    heads)."""
    _kivi_chunk_over_prefix(gpu_device, b=8, hq=40, kvh=8, d=128, g=128, r=128, bs=128,
                            prefix=8192, chunk=2048)


def _kivi_chunk_over_prefix(dev, *, b, hq, kvh, d, g, r, bs, prefix, chunk):
    n = prefix + chunk
    nblk = [n // bs] * b
    nb = sum(nblk) + 8
    gen = torch.Generator().manual_seed(4)
    key_scales = torch.exp(torch.randn((kvh, d), generator=gen))
    table = _table(nblk, nb, seed=41)
    impl, kbuf, vbuf, layout = _kivi_on_bytes(dev, hq=hq, kvh=kvh, d=d, g=g, r=r, nb=nb, bs=bs,
                                             rows=b)
    reqs = [f"r{i}" for i in range(b)]
    ks, vs = [], []
    for i in range(b):
        k, v = _rand_kv(dev, n, kvh, d, 400 + i, key_scales)
        impl._write_kivi_cache(k[:prefix], v[:prefix], _slots(table[i], 0, prefix, bs).to(dev),
                               [reqs[i]], [prefix])
        ks.append(k)
        vs.append(v)
    qgen = torch.Generator(device=dev).manual_seed(44)
    q = torch.randn((b * chunk, hq, d), generator=qgen, device=dev).to(torch.bfloat16)
    slots = torch.cat([_slots(table[i], prefix, n, bs) for i in range(b)])
    out = torch.zeros((b * chunk, hq, d), dtype=torch.bfloat16, device=dev)
    md = _md("PrefillCacheHit", actual_seq_lengths_q=[chunk * (i + 1) for i in range(b)],
             seq_lens_list=[n] * b, slot_mapping=slots.to(dev), block_tables=table.to(dev),
             req_ids=reqs, num_actual_tokens=b * chunk)
    impl.forward(None, q, torch.cat([k[prefix:] for k in ks]),
                 torch.cat([v[prefix:] for v in vs]), (kbuf, vbuf), md, out)
    gk, gv = impl._gather_dequant_kivi_paged_cache(table.to(dev), [n] * b, torch.bfloat16, reqs)
    torch.cuda.synchronize()
    hk, hv = _incremental(n, r)
    kc = [k.cpu() for k in ks]
    vc = [v.cpu() for v in vs]
    del ks, vs
    seqs = [(kc[i], vc[i], _slots(table[i], 0, n, bs), hk, hv) for i in range(b)]
    want_k, want_v, views = _oracle_pages(layout, seqs, g)
    assert torch.equal(kbuf.cpu(), want_k), "int4 key pages differ from the oracle"
    assert torch.equal(vbuf.cpu(), want_v), "int4 value pages differ from the oracle"
    dk, dv = ref.dequant_gather(*views, table, torch.tensor([n] * b), torch.bfloat16, g)
    dk = ref.overlay_residual(dk, [n] * b, [x[hk:] for x in kc])
    dv = ref.overlay_residual(dv, [n] * b, [x[hv:] for x in vc])
    assert torch.equal(gk.cpu(), dk) and torch.equal(gv.cpu(), dv)
    rep = hq // kvh
    for i in (0, b - 1):
        qi = q[i * chunk:(i + 1) * chunk].cpu()
        oi = out[i * chunk:(i + 1) * chunk].cpu().float()
        for h in (0, kvh - 1):
            heads = slice(h * rep, (h + 1) * rep)
            want = ref.attention(qi[:, heads], dk[i * n:(i + 1) * n, h:h + 1],
                                 dv[i * n:(i + 1) * n, h:h + 1], [chunk], [n], d ** -0.5, True)
            torch.testing.assert_close(oi[:, heads], want, **TOL)


# ---------------------------------------------------------------------------
# config 2: INT8 dynamic per-channel, 64 x 4096 tokens, Llama-3-8B geometry
# ---------------------------------------------------------------------------


def test_config2_int8_prefill_and_decode_full_batch(gpu_device):
    """Scales from the whole first K/V, quantize + scatter of 64 x 4096 tokens
    into 2,112 shuffled pages, prefill attention (requests 0 and 63, KV heads
    0 and 7), then one decode step of the whole batch checked for all 64."""
    _int8_prefill_then_decode(gpu_device, b=64, hq=32, kvh=8, d=128, bs=128, n=4096)


def _int8_prefill_then_decode(dev, *, b, hq, kvh, d, bs, n):
    nblk = [n // bs + 1] * b
    nb = sum(nblk)
    table = _table(nblk, nb, seed=21)
    gen = torch.Generator().manual_seed(2)
    key_scales = torch.exp(torch.randn((kvh, d), generator=gen))
    k, v = _rand_kv(dev, b * (n + 1), kvh, d, 22, key_scales)
    k = k.view(b, n + 1, kvh, d)
    v = v.view(b, n + 1, kvh, d)
    pk, pv = k[:, :n].reshape(-1, kvh, d), v[:, :n].reshape(-1, kvh, d)
    qgen = torch.Generator(device=dev).manual_seed(23)
    q = torch.randn((b * n, hq, d), generator=qgen, device=dev).to(torch.bfloat16)

    class Impl(AscendInt8AttentionBackendMixin):
        num_heads, num_kv_heads, head_size, scale = hq, kvh, d, d ** -0.5

    impl = Impl()
    layer = SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)
    cache = torch.zeros(2, nb, bs, kvh, d, dtype=torch.int8, device=dev)
    slots = torch.cat([_slots(table[i], 0, n, bs) for i in range(b)])
    out = torch.zeros((b * n, hq, d), dtype=torch.bfloat16, device=dev)
    md = SimpleNamespace(attn_state=SimpleNamespace(name="PrefillNoCache"),
                         model_runner_type="generate", causal=True,
                         slot_mapping=slots.to(dev), num_actual_tokens=b * n,
                         actual_seq_lengths_q=[n * (i + 1) for i in range(b)],
                         seq_lens_list=[n] * b, block_tables=table.to(dev))
    impl.forward(layer, q, pk, pv, cache, md, out)
    torch.cuda.synchronize()
    pkc, pvc = pk.cpu(), pv.cpu()
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(pkc, pvc)
    assert torch.equal(layer._int8_k_inv_scale.cpu(), k_inv)
    assert torch.equal(layer._int8_v_inv_scale.cpu(), v_inv)
    assert torch.equal(layer._int8_k_aq_scale.cpu().flatten(), k_aq.flatten())
    assert torch.equal(layer._int8_v_aq_scale.cpu().flatten(), v_aq.flatten())
    want_cache = torch.zeros(2, nb, bs, kvh, d, dtype=torch.int8)
    ref.int8_reshape_and_cache(pkc, pvc, k_inv, v_inv, slots, want_cache[0], want_cache[1])
    assert torch.equal(cache.cpu(), want_cache), "int8 pages differ after the prefill"
    rep = hq // kvh
    for i in (0, b - 1):
        rows = slice(i * n, (i + 1) * n)
        qi, oi = q[rows].cpu(), out[rows].cpu().float()
        for h in (0, kvh - 1):
            heads = slice(h * rep, (h + 1) * rep)
            want = ref.attention(qi[:, heads], pkc[rows, h:h + 1], pvc[rows, h:h + 1], [n], [n],
                                 d ** -0.5, True)
            torch.testing.assert_close(oi[:, heads], want, **TOL)
    del q, out, pkc, pvc
    # one decode step for all 64 requests
    kd, vd = k[:, n].contiguous(), v[:, n].contiguous()
    qd = torch.randn((b, hq, d), generator=gen).to(torch.bfloat16)
    new = torch.stack([_slots(table[i], n, n + 1, bs)[0] for i in range(b)])
    lens = [n + 1] * b
    md = SimpleNamespace(attn_state=SimpleNamespace(name="DecodeOnly"),
                         model_runner_type="generate", causal=True, slot_mapping=new.to(dev),
                         num_actual_tokens=b, seq_lens_list=lens, block_tables=table.to(dev))
    out = torch.zeros((b, hq, d), dtype=torch.bfloat16, device=dev)
    impl.forward(layer, qd.to(dev), kd, vd, cache, md, out)
    torch.cuda.synchronize()
    ref.int8_reshape_and_cache(kd.cpu(), vd.cpu(), k_inv, v_inv, new, want_cache[0],
                               want_cache[1])
    assert torch.equal(cache.cpu(), want_cache), "int8 pages differ after the decode step"
    dk, dv = ref.int8_paged_dequant(want_cache[0], want_cache[1], table, lens, torch.float32,
                                    k_inv, v_inv)
    want = ref.attention(qd, dk, dv, [1] * b, lens, d ** -0.5, True)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)
