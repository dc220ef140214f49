# SPDX-License-Identifier: Apache-2.0
"""Pins the CPU oracle before anything is checked against it (no GPU).

Each check is chosen so that a plausible slip in the oracle (a swapped lane
order, a dropped floor, ties rounded the wrong way, a transposed key layout, a
missing GQA repeat) fails at least one of them:

* the reference's own known-answer tests (``tests/test_kivi_int4.py``);
* an independent scalar C restatement (``oracle/kvq_ref.c``), bit for bit;
* hand-computed words for tiny inputs;
* closed forms and brute force (float64 loops) for attention and INT8;
* the incremental residual rule's closed form over several geometries.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from oracle import kvq_oracle as ref
from tests import _cpu_kernels as ck
from tests._util import empty_kivi_caches, make_kv, shuffled_table, slots_for

# ---------------------------------------------------------------------------
# a3: scalar math, reference known answers (tests/test_kivi_int4.py:1140-1171)
# ---------------------------------------------------------------------------


def test_group_scale_floor_applies_to_scale_not_range():
    zero = torch.tensor(0.0)
    floor = torch.tensor(1e-6).item()  # fp32(1e-6)
    assert ref.group_scale(zero, torch.tensor(3e-7)).item() == floor
    assert ref.group_scale(zero, torch.tensor(1e-9)).item() == floor
    # above the floor the scale is the plain fp32 quotient
    got = ref.group_scale(torch.tensor(-1.0), torch.tensor(2.0))
    assert got.item() == torch.tensor(3.0 / 15.0, dtype=torch.float32).item()


def test_quantize_ties_round_half_up_and_clamps():
    one, zero = torch.tensor(1.0), torch.tensor(0.0)
    q = ref.quantize_group(torch.tensor([2.5, 3.5, 99.0, -4.0, 0.49, 14.5]), zero, one)
    assert q.dtype == torch.int32
    assert q.tolist() == [3, 4, 15, 0, 0, 15]


def test_pack_int4_lane_order_hand_computed():
    # lane L at bits 4L..4L+3 (semantics.py:76-83)
    word = ref.pack_int4(torch.tensor([[1, 2, 3, 4, 5, 6, 7, 8]]))
    assert word.dtype == torch.int32
    assert word.item() == 0x87654321 - 2**32  # sign bit set by lane 7 = 8
    assert ref.pack_int4(torch.tensor([[15, 0, 0, 0, 0, 0, 0, 0]])).item() == 15
    assert ref.pack_int4(torch.tensor([[0] * 7 + [15]])).item() == -(2**28)


def test_pack_unpack_round_trip():
    g = torch.Generator().manual_seed(1)
    q = torch.randint(0, 16, (64, 8), generator=g, dtype=torch.int32)
    assert torch.equal(ref.unpack_int4(ref.pack_int4(q)), q.float())


def test_key_pack_hand_computed_codes():
    # one head, one dim, G = 8 tokens 0..7: mn 0, mx 7, scale 7/15;
    # codes floor(t*15/7 + 0.5) = 0,2,4,6,9,11,13,15 with lanes along tokens
    key = torch.arange(8, dtype=torch.float32).view(8, 1, 1).expand(8, 1, 8).contiguous()
    kq, ks, km, vq, vs, vm = empty_kivi_caches(1, 8, 1, 8, 8)
    ref.pack_key_cache(key, torch.arange(8), kq, ks, km, 8)
    want = 0xFDB96420 - 2**32
    assert kq[0, 0, :, 0].tolist() == [want] * 8
    assert ks[0, 0, 0, 0].item() == torch.tensor(7.0 / 15.0).item()
    assert km[0, 0, 0, 0].item() == 0.0
    # values: lanes along head_dim; the same ramp across dims gives the same word
    ref.pack_value_cache(key.transpose(0, 2).contiguous(), torch.arange(8), vq, vs, vm, 8)
    assert vq[0, 0, 0, 0].item() == want


# ---------------------------------------------------------------------------
# a4 / a5 / a7: torch oracle vs the scalar C restatement, bit for bit
# ---------------------------------------------------------------------------

GEOMETRIES = [  # (D, G, Bs, KVH, NB) -- the reference's page round-trip set
    (128, 128, 128, 8, 7),
    (32, 8, 16, 2, 3),
    (64, 32, 256, 4, 2),
    (128, 64, 128, 2, 4),
]


@pytest.mark.parametrize("d,g,bs,kvh,nb", GEOMETRIES)
def test_pack_matches_c_restatement(d, g, bs, kvh, nb):
    t = nb * bs
    key, value = make_kv(t, kvh, d, dtype=torch.float32, seed=d + g)
    table = shuffled_table(1, nb, nb, seed=g)[0]
    slots = slots_for(table, range(t), bs)
    torch_caches = empty_kivi_caches(nb, bs, kvh, d, g, fill=7)
    c_caches = empty_kivi_caches(nb, bs, kvh, d, g, fill=7)
    ref.pack_key_cache(key, slots, *torch_caches[:3], g)
    ref.pack_value_cache(value, slots, *torch_caches[3:], g)
    ck.c_pack_key(key, slots, c_caches[:3], g, bs)
    ck.c_pack_value(value, slots, c_caches[3:], g, bs)
    for a, b in zip(torch_caches, c_caches):
        assert torch.equal(a, b)


def test_pack_skips_negative_slots_like_c():
    d, g, bs, kvh, nb = 32, 8, 16, 2, 3
    key, value = make_kv(2 * bs, kvh, d, dtype=torch.float32, seed=5)
    slots = torch.arange(2 * bs, dtype=torch.int64)
    slots[8:16] = -1  # one key group and eight value tokens are padding
    a = empty_kivi_caches(nb, bs, kvh, d, g, fill=3)
    b = empty_kivi_caches(nb, bs, kvh, d, g, fill=3)
    ref.pack_key_cache(key, slots, *a[:3], g)
    ref.pack_value_cache(value, slots, *a[3:], g)
    ck.c_pack_key(key, slots, b[:3], g, bs)
    ck.c_pack_value(value, slots, b[3:], g, bs)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert (a[0][0, :, :, 1] == 3).all()  # untouched words of the skipped group


@pytest.mark.parametrize("d,g,bs,kvh,nb", GEOMETRIES)
def test_gather_matches_c_restatement(d, g, bs, kvh, nb):
    key, value = make_kv(nb * bs, kvh, d, dtype=torch.float32, seed=11)
    table = shuffled_table(1, nb, nb, seed=3)
    slots = slots_for(table[0], range(nb * bs), bs)
    caches = empty_kivi_caches(nb, bs, kvh, d, g)
    ref.pack_key_cache(key, slots, *caches[:3], g)
    ref.pack_value_cache(value, slots, *caches[3:], g)
    # two requests over the same pages, ragged lengths, a negative id past the end
    bt = torch.cat([table, table.flip(1)]).to(torch.int64)
    bt = torch.cat([bt, torch.full((2, 1), -1, dtype=torch.int64)], dim=1)
    lens = torch.tensor([nb * bs - 3, bs // 2 + 1], dtype=torch.int64)
    dk, dv = ref.dequant_gather(*caches, bt, lens, torch.float32, g)
    ck_, cv_ = ck.c_gather(caches, bs, kvh, d, g, bt.contiguous(), lens)
    assert torch.equal(dk, ck_) and torch.equal(dv, cv_)


@pytest.mark.parametrize("g", [8, 32, 128])
def test_gather_of_pack_equals_fake_quant(g):
    """Gather(pack(x)) == fake_quant(x) (tests/test_kivi_int4.py:561-694)."""
    d, bs, kvh = 128, 128, 2
    t = 2 * bs
    key, value = make_kv(t, kvh, d, dtype=torch.float32, seed=g)
    caches = empty_kivi_caches(2, bs, kvh, d, g)
    slots = torch.arange(t)
    ref.pack_key_cache(key, slots, *caches[:3], g)
    ref.pack_value_cache(value, slots, *caches[3:], g)
    dk, dv = ref.dequant_gather(*caches, torch.tensor([[0, 1]]), torch.tensor([t]),
                                torch.float32, g)
    assert torch.equal(dk, ref.fake_quant_key(key, g))
    assert torch.equal(dv, ref.fake_quant_value(value, g))
    # reconstruction error is bounded by half a quantization step
    step = (key.view(-1, g, kvh, d).amax(1) - key.view(-1, g, kvh, d).amin(1)) / 15
    err = (dk - key).abs().view(-1, g, kvh, d).amax(1)
    assert (err <= step * 0.5 + 1e-5).all()


def test_overlay_replaces_last_rows_fifo():
    dense = torch.zeros(10, 1, 2)
    win_a = torch.arange(6, dtype=torch.float32).view(3, 1, 2)  # longer than request
    win_b = torch.full((2, 1, 2), 9.0)
    out = ref.overlay_residual(dense, [2, 8], [win_a, win_b])
    assert out[:2].flatten().tolist() == [2, 3, 4, 5]
    assert (out[2:8] == 0).all() and (out[8:] == 9).all()


# ---------------------------------------------------------------------------
# attention: brute force in float64 and torch SDPA
# ---------------------------------------------------------------------------


def _attention_f64(q, k, v, q_lens, kv_lens, scale, causal):
    hq, kvh = q.shape[1], k.shape[1]
    out = torch.zeros(q.shape, dtype=torch.float64)
    qs = ks = 0
    for ql, kl in zip(q_lens, kv_lens):
        for i in range(ql):
            qpos = kl - ql + i
            for h in range(hq):
                kh = h // (hq // kvh)
                lim = qpos + 1 if causal else kl
                s = [float((q[qs + i, h].double() * k[ks + j, kh].double()).sum()) * scale
                     for j in range(lim)]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                tot = sum(w)
                acc = sum(w[j] / tot * v[ks + j, kh].double() for j in range(lim))
                out[qs + i, h] = acc
        qs += ql
        ks += kl
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_attention_matches_float64_brute_force(causal):
    g = torch.Generator().manual_seed(2)
    hq, kvh, d = 4, 2, 8
    q_lens, kv_lens = [1, 3, 2], [4, 3, 6]
    q = torch.randn(sum(q_lens), hq, d, generator=g)
    k = torch.randn(sum(kv_lens), kvh, d, generator=g)
    v = torch.randn(sum(kv_lens), kvh, d, generator=g)
    got = ref.attention(q, k, v, q_lens, kv_lens, 0.3, causal)
    want = _attention_f64(q, k, v, q_lens, kv_lens, 0.3, causal)
    torch.testing.assert_close(got.double(), want, atol=1e-5, rtol=1e-5)


def test_attention_matches_sdpa_gqa():
    g = torch.Generator().manual_seed(4)
    hq, kvh, d, n = 8, 2, 16, 12
    q = torch.randn(n, hq, d, generator=g)
    k = torch.randn(n, kvh, d, generator=g)
    v = torch.randn(n, kvh, d, generator=g)
    got = ref.attention(q, k, v, [n], [n], d ** -0.5, True)
    kk = k.repeat_interleave(hq // kvh, 1).transpose(0, 1)
    vv = v.repeat_interleave(hq // kvh, 1).transpose(0, 1)
    want = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(0, 1), kk, vv, is_causal=True).transpose(0, 1)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# INT8: C restatement (explicit bf16 RNE), closed forms, rounding
# ---------------------------------------------------------------------------


def test_int8_scales_bf16_match_c_restatement():
    key, value = make_kv(257, 8, 128, dtype=torch.bfloat16, seed=9)
    key[:, 0, 0] = 0  # an all-zero channel exercises the 1e-12 floor
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(key, value)
    for x, inv, aq in ((key, k_inv, k_aq), (value, v_inv, v_aq)):
        c_inv, c_aq = ck.c_int8_scales_bf16(x.float().reshape(x.shape[0], -1).contiguous())
        assert inv.dtype == torch.bfloat16
        assert torch.equal(inv.float().flatten(), c_inv)
        assert torch.equal(aq.float().flatten(), c_aq)


def test_int8_quantize_bf16_matches_c_and_rounds_half_even():
    key, _ = make_kv(64, 8, 128, dtype=torch.bfloat16, seed=10)
    k_inv, _, _, _ = ref.int8_calc_scales(key, key)
    codes = ref.int8_quantize(key, k_inv)
    c_codes = ck.c_int8_quant_bf16(key.float().reshape(64, -1).contiguous(),
                                   k_inv.float().flatten().contiguous())
    assert torch.equal(codes.reshape(64, -1), c_codes)
    inv = torch.ones(4, dtype=torch.bfloat16)
    x = torch.tensor([2.5, -2.5, 300.0, -300.0], dtype=torch.bfloat16)
    assert ref.int8_quantize(x, inv).tolist() == [2, -2, 127, -128]


@pytest.mark.parametrize("bs,nb", [(16, 7), (128, 5)])
def test_int8_reshape_and_cache_matches_per_slot_loop(bs, nb):
    """The scatter half of ``int8_reshape_and_cache`` (the host
    ``reshape_and_cache``, ``i8ab.py:86-88``), pinned by a per-slot loop.

    The codes come from the independent C restatement (bf16 product, then
    round half to even, then the clamp); the loop writes token ``i`` to page
    ``s // Bs``, row ``s % Bs`` for every slot ``s >= 0`` and skips padding.
    Slots cover a shuffled pool, the pool's last row and negative padding;
    every byte the loop does not write must keep its sentinel, on both sides.
    """
    kvh, d = 2, 16
    g = torch.Generator().manual_seed(21)
    pool = torch.randperm(nb * bs, generator=g)[: nb * bs // 2].tolist()
    slots = pool + [nb * bs - 1, -1, -7, 0]
    slots = list(dict.fromkeys(slots))  # distinct live slots; padding may repeat
    n = len(slots)
    key, value = make_kv(n, kvh, d, dtype=torch.bfloat16, seed=22)
    key[3] *= 400  # codes that clamp at both ends
    key[4] *= -400
    k_inv, v_inv, _, _ = ref.int8_calc_scales(key, value)
    sentinel = 77
    kc = torch.full((nb, bs, kvh, d), sentinel, dtype=torch.int8)
    vc = torch.full_like(kc, sentinel)
    ref.int8_reshape_and_cache(key, value, k_inv, v_inv, torch.tensor(slots), kc, vc)

    want_k = torch.full_like(kc, sentinel)
    want_v = torch.full_like(vc, sentinel)
    codes_k = ck.c_int8_quant_bf16(key.float().reshape(n, -1).contiguous(),
                                   k_inv.float().flatten().contiguous()).reshape(n, kvh, d)
    codes_v = ck.c_int8_quant_bf16(value.float().reshape(n, -1).contiguous(),
                                   v_inv.float().flatten().contiguous()).reshape(n, kvh, d)
    assert codes_k.max() == 127 and codes_k.min() == -128
    for i, s in enumerate(slots):
        if s < 0:
            continue
        for h in range(kvh):
            for c in range(d):
                want_k[s // bs, s % bs, h, c] = codes_k[i, h, c]
                want_v[s // bs, s % bs, h, c] = codes_v[i, h, c]
    assert torch.equal(kc, want_k)
    assert torch.equal(vc, want_v)
    assert int((kc != sentinel).any(dim=(2, 3)).sum()) == len([s for s in slots if s >= 0])


def test_int8_scales_closed_form_fp32():
    x = torch.tensor([[0.5, -4.0, 0.0], [-1.0, 2.0, 0.0]])
    k_inv, _, k_aq, _ = ref.int8_calc_scales(x, x)
    assert k_inv.flatten().tolist() == pytest.approx([127.0, 127 / 4, 127e12], rel=1e-6)
    assert torch.equal(k_aq, 1.0 / k_inv)


def test_int8_scales_two_rounding_steps_over_every_bf16_amax():
    """``127.0 / amax`` in bf16 is reciprocal then multiply, each rounded to
    bf16 (torch's ``__rdiv__``); a single rounded division differs on some
    amax values, so this pins the order of the two roundings."""
    bits = torch.arange(0x2B8D, 0x7F80, dtype=torch.int32).to(torch.int16)  # bf16(1e-12) .. inf
    amax = bits.view(torch.bfloat16)
    x = torch.stack([amax, -amax])  # one channel per amax value
    k_inv, _, k_aq, _ = ref.int8_calc_scales(x, x)
    two_step = (amax.float().reciprocal().to(torch.bfloat16).float() * 127).to(torch.bfloat16)
    one_step = (127.0 / amax.float()).to(torch.bfloat16)
    assert torch.equal(k_inv.flatten(), two_step)
    assert not torch.equal(two_step, one_step)
    assert torch.equal(k_aq.flatten(), (1.0 / two_step.float()).to(torch.bfloat16))


def test_int8_paged_dequant_brute_force():
    g = torch.Generator().manual_seed(6)
    nb, bs, kvh, d = 5, 4, 2, 8
    kc = torch.randint(-128, 128, (nb, bs, kvh, d), generator=g, dtype=torch.int8)
    vc = torch.randint(-128, 128, (nb, bs, kvh, d), generator=g, dtype=torch.int8)
    inv = torch.rand(1, kvh, d, generator=g) * 100 + 1
    table = torch.tensor([[3, 1], [0, 4]])
    dk, dv = ref.int8_paged_dequant(kc, vc, table, [6, 3], torch.float32, inv, inv)
    rows_k, rows_v = [], []
    for b, n in enumerate([6, 3]):
        for p in range(n):
            blk = int(table[b, p // bs])
            rows_k.append(kc[blk, p % bs].float() * (1.0 / inv[0]))
            rows_v.append(vc[blk, p % bs].float() * (1.0 / inv[0]))
    assert torch.equal(dk, torch.stack(rows_k)) and torch.equal(dv, torch.stack(rows_v))


# ---------------------------------------------------------------------------
# a6: residual window model vs the incremental rule's closed form
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("r", [8, 16, 32, 64, 128])
def test_window_model_matches_incremental_closed_form(r):
    m = ref.KiviWindowModel(r)
    rows = torch.zeros(1, 1, 1)
    for length in range(1, 3 * r + 5):
        m.write(rows, rows, [length - 1])
        hk, hv = ref.incremental_split(length, r)
        assert (len(m.history[True]), len(m.history[False])) == (hk, hv), length
        assert len(m.win[True]) == length - hk and len(m.win[False]) == length - hv
    # the flushed keys are whole, in order
    assert [s for s, _ in m.history[True]] == list(range(len(m.history[True])))


def test_window_model_overwrite_does_not_evict_and_bulk_flushes():
    m = ref.KiviWindowModel(4)
    one = torch.ones(1, 1, 1)
    for s in range(4):
        m.write(one * s, one * s, [s])
    m.write(one * 9, one * 9, [2])  # overwrite of a held slot
    assert [s for s, _ in m.win[True]] == [0, 1, 2, 3] and not m.history[True]
    assert m.win[True][2][1].item() == 9
    m.write(one, one, [4])  # full: keys flush all 4, values evict 1
    assert len(m.history[True]) == 4 and len(m.history[False]) == 1
    assert [s for s, _ in m.win[False]] == [1, 2, 3, 4]
    bulk = ref.KiviWindowModel(4)
    rows = torch.zeros(10, 1, 1)
    bulk.write_prefill(rows, rows, list(range(10)))
    assert len(bulk.history[True]) == 8 and len(bulk.win[True]) == 2


def test_algorithmic_bytes_formula():
    # D=128, G=128 -> S=72; one token of history on each side, nothing resident
    b = ref.algorithmic_bytes_int4_decode(128, 128, 0, 0, 8, 128, 128, 40, 128)
    assert b == 256 * 8 * 72 + 2 * 40 * 128 * 2 + 4
    # per-token slope 1152 B (S=72, KVH=8, both sides)
    hk, hv = ref.incremental_split(9216, 128)
    b1 = ref.algorithmic_bytes_int4_decode(hk, hv, 9216 - hk, 9216 - hv, 8, 128, 128, 40, 128)
    hk2, hv2 = ref.incremental_split(9216 + 128, 128)
    b2 = ref.algorithmic_bytes_int4_decode(hk2, hv2, 9216 + 128 - hk2, 9216 + 128 - hv2,
                                           8, 128, 128, 40, 128)
    assert b2 - b1 == 128 * 1152 + 4


def test_oracle_is_deterministic_under_shuffle():
    """Packing in any slot order gives the same caches (per-group independence)."""
    d, g, bs, kvh, nb = 32, 8, 16, 2, 4
    key, value = make_kv(nb * bs, kvh, d, dtype=torch.float32, seed=12)
    slots = torch.arange(nb * bs)
    a = empty_kivi_caches(nb, bs, kvh, d, g)
    ref.pack_value_cache(value, slots, *a[3:], g)
    perm = list(range(nb * bs))
    random.Random(0).shuffle(perm)
    b = empty_kivi_caches(nb, bs, kvh, d, g)
    ref.pack_value_cache(value[perm], slots[perm], *b[3:], g)
    for x, y in zip(a[3:], b[3:]):
        assert torch.equal(x, y)


def test_int8_antiquant_keeps_bf16_scale_in_fp32_product():
    """Decode antiquant: code * bf16(1/inv), product in fp32 (no bf16 rounding of K)."""
    g = torch.Generator().manual_seed(13)
    kc = torch.randint(-128, 128, (2, 4, 1, 8), generator=g, dtype=torch.int8)
    inv = (torch.rand(1, 1, 8, generator=g) * 300 + 1).to(torch.bfloat16)
    dk, _ = ref.int8_paged_dequant(kc, kc, torch.tensor([[1, 0]]), [7], torch.float32, inv, inv)
    aq = (1.0 / inv).to(torch.bfloat16).float()[0]  # the scale itself is a bf16 value
    rows = [kc[[1, 0][p // 4], p % 4].float() * aq for p in range(7)]
    assert dk.dtype == torch.float32 and torch.equal(dk, torch.stack(rows))
    dense, _ = ref.int8_paged_dequant(kc, kc, torch.tensor([[1, 0]]), [7], torch.bfloat16, inv,
                                      inv)
    assert torch.equal(dense, dk.to(torch.bfloat16))  # dense prefill path rounds once more
