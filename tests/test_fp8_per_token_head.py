# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head on the CPU: the oracle pinned, and the host-side contract.

Oracle pins (a slip in any of them -- a wrong rounding, a reciprocal in place
of the division, a dropped clamp or floor, a wrong scatter index -- fails at
least one check):

* the 256 E4M3 codes decoded from the OCP e4m3fn definition (sign, 4-bit
  exponent with bias 7, 3-bit mantissa, subnormals, one NaN per sign) and
  torch's e4m3fn cast checked against an independent nearest-even encoder at
  every rounding boundary (each midpoint and the fp32 neighbours on both
  sides) and on random values;
* the reference's known answers (``tests/test_fp8_per_token_head.py``): the
  1e-6 floor, the page budget, the fake-quant error bound, outlier
  independence, all-zero rows, the byte round trip through the views;
* closed forms: a power-of-two scale makes the quotient exact, so codes are
  the encoder's codes of ``x / 2^k``; negating the input flips only the sign
  bit; values on the grid survive a round trip unchanged;
* the division rule: rows built so that ``x / scale`` and ``x * (1/scale)``
  round to different codes follow the division;
* the paged store and gather against a brute-force per-slot loop.

Host contract (mirrors the reference's tests of the same names): layout
literal, method discovery failing closed, region budget, views aliasing the
host buffers, layout inference, validators, launch contract.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kvq_oracle as ref
from vllm_ascend_quantized_kv_cache.dtypes import KVCacheLayout, KVQuantMode, resolve_layout
from vllm_ascend_quantized_kv_cache.methods.fp8_per_token_head.byte_cache import (
    Fp8PerTokenHeadLayout,
    fp8_caches_from_byte_tensors,
    fp8_per_token_head_layout,
)
from vllm_ascend_quantized_kv_cache.methods.registry import get_method
from vllm_ascend_quantized_kv_cache.ops import fp8_ops

HEAD = 128
KVH = 2
BLOCK = 128
NB = 4


# ---------------------------------------------------------------------------
# an independent E4M3 (OCP e4m3fn) encoder
# ---------------------------------------------------------------------------


def e4m3_values() -> np.ndarray:
    """float64 value of each of the 256 codes, from the format's definition."""
    vals = np.empty(256, dtype=np.float64)
    for c in range(256):
        sign = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 0x7
        if e == 15 and m == 7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = sign * m * 2.0 ** -9
        else:
            vals[c] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3 = e4m3_values()
POS = E4M3[:127]  # codes 0x00..0x7E: 0 .. 448, ascending


def encode_rne(x: np.ndarray) -> np.ndarray:
    """Nearest E4M3 code of fp32 values with |x| <= 448, ties to the even code.

    Distances are exact in float64 (fp32 values, codes and midpoints all are).
    """
    x = np.asarray(x, dtype=np.float32)
    mag = np.abs(x).astype(np.float64)
    assert (mag <= 448.0).all()
    hi = np.clip(np.searchsorted(POS, mag, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    d_lo, d_hi = mag - POS[lo], POS[hi] - mag
    pick = np.where(d_lo < d_hi, lo, hi)
    tie = d_lo == d_hi
    pick = np.where(tie, np.where(lo % 2 == 0, lo, hi), pick)
    pick = np.where(mag == POS[hi], hi, pick)
    return (pick | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)


def boundary_points() -> np.ndarray:
    """Every rounding boundary of [0, 448] with its fp32 neighbours, both signs."""
    mids = (POS[:-1] + POS[1:]) / 2
    pts = [0.0, 448.0, 2.0 ** -10, 2.0 ** -11]
    for v in np.concatenate([mids, POS]):
        f = np.float32(v)
        pts += [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(0))]
    pts = np.asarray(pts, dtype=np.float32)
    pts = pts[np.abs(pts) <= 448.0]
    return np.concatenate([pts, -pts])


def test_e4m3_code_table_matches_the_format():
    got = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float64)
    want = torch.from_numpy(E4M3)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan) and nan.sum() == 2  # 0x7F and 0xFF
    assert torch.equal(got[~nan], want[~nan])
    assert E4M3[0x7E] == 448.0 and E4M3[0x01] == 2.0 ** -9 and E4M3[0x08] == 2.0 ** -6
    assert E4M3[0x38] == 1.0 and E4M3[0x80] == 0.0 and np.signbit(E4M3[0x80])
    assert (np.diff(POS) > 0).all()


def test_torch_e4m3_cast_is_round_to_nearest_even():
    pts = boundary_points()
    got = torch.from_numpy(pts).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, encode_rne(pts))
    # midpoints themselves go to the even code, the fp32 neighbours to the nearest
    mid = np.float32((POS[9] + POS[10]) / 2)  # between codes 9 and 10
    assert encode_rne(np.array([mid]))[0] == 10
    assert encode_rne(np.array([np.nextafter(mid, np.float32(0))]))[0] == 9
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-12, 6, 1 << 16))).astype(np.float32)
    x = np.clip(x, -448, 448).astype(np.float32)
    got = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, encode_rne(x))


# ---------------------------------------------------------------------------
# oracle: the reference's known answers (tests/test_fp8_per_token_head.py)
# ---------------------------------------------------------------------------


def test_scale_floor_matches_host_kernel():
    scale = ref.fp8_pth_scale(torch.zeros(1, 1, HEAD))
    assert float(scale[0, 0, 0]) == torch.tensor(1e-6).item()


def test_fake_quant_error_bounded_by_e4m3_precision():
    torch.manual_seed(5)
    x = torch.randn(8, KVH, HEAD)
    codes, scale = ref.fp8_pth_quantize(x)
    assert scale.shape == (8, KVH, 1)
    fq = ref.fp8_pth_dequantize(codes, scale)
    err = (fq - x).abs()
    assert (err <= 0.07 * x.abs() + scale * 2 ** -8).all()


def test_per_token_head_scale_is_independent():
    torch.manual_seed(6)
    x = torch.randn(2, KVH, HEAD)
    x[0, 0, 0] = 1.0e4
    fq = ref.fp8_pth_dequantize(*ref.fp8_pth_quantize(x))
    rel = (fq[1, 0] - x[1, 0]).abs() / x[1, 0].abs().clamp(min=1e-3)
    assert rel.max() < 0.07 and torch.isfinite(fq).all()
    scales = ref.fp8_pth_scale(x)
    assert scales[0, 0, 0] > scales[1, 0, 0] * 100


def test_zero_rows_do_not_divide_by_zero():
    codes, scale = ref.fp8_pth_quantize(torch.zeros(3, 1, HEAD))
    fq = ref.fp8_pth_dequantize(codes, scale)
    assert torch.isfinite(fq).all() and (fq == 0).all() and (codes == 0).all()


def test_byte_level_roundtrip_through_views():
    torch.manual_seed(7)
    layout = Fp8PerTokenHeadLayout(NB, BLOCK, KVH, HEAD)
    key_buf = torch.zeros(NB, BLOCK, KVH, layout.bytes_per_token_head, dtype=torch.uint8)
    k_data, k_scale, _, _ = fp8_caches_from_byte_tensors(key_buf, torch.zeros_like(key_buf),
                                                         layout)
    x = torch.randn(32, KVH, HEAD)
    codes, scale = ref.fp8_pth_quantize(x)
    k_data[0, :32] = codes
    k_scale[0, :32, :, 0] = scale[:, :, 0]
    back = ref.fp8_pth_dequantize(k_data[0, :32], k_scale[0, :32])
    assert torch.equal(back, ref.fp8_pth_dequantize(codes, scale))
    # the bytes really are in the host buffer: data first, then the scales
    assert torch.equal(key_buf.view(-1)[: 32 * KVH * HEAD].view(32, KVH, HEAD), codes)


# ---------------------------------------------------------------------------
# oracle: closed forms and the division rule
# ---------------------------------------------------------------------------


def test_power_of_two_scale_gives_exact_quotients():
    rng = np.random.default_rng(1)
    for k in (-15, -3, 0, 5):  # 2^-15 is above the 1e-6 floor
        x = rng.uniform(-448, 448, (4, 3, 64)).astype(np.float32)
        x[:, :, 0] = 448.0  # amax = 448 -> scale 1
        x = (x * np.float32(2.0 ** k)).astype(np.float32)  # exact
        codes, scale = ref.fp8_pth_quantize(torch.from_numpy(x))
        assert (scale == 2.0 ** k).all()
        want = encode_rne((x / np.float32(2.0 ** k)).astype(np.float32))
        np.testing.assert_array_equal(codes.numpy(), want)


def test_negation_flips_only_the_sign_bit():
    torch.manual_seed(2)
    x = torch.randn(5, 2, 32) * 3
    c, s = ref.fp8_pth_quantize(x)
    cn, sn = ref.fp8_pth_quantize(-x)
    assert torch.equal(s, sn)
    assert torch.equal(cn, c ^ 0x80)


def test_grid_values_round_trip_unchanged():
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 127, (6, 2, 64)).astype(np.uint8)
    codes |= (rng.integers(0, 2, codes.shape) * 0x80).astype(np.uint8)
    codes[:, :, 0] = 0x7E  # 448: scale 1
    x = torch.from_numpy(E4M3[codes].astype(np.float32))
    c, s = ref.fp8_pth_quantize(x)
    assert (s == 1.0).all()
    back = ref.fp8_pth_dequantize(c, s)
    assert torch.equal(back, x)  # -0 codes come back as -0 (equal to 0)


def division_rows(n: int, seed: int = 0):
    """Rows ``[amax, x]`` where ``x / scale`` and ``x * (1/scale)`` give
    different codes (scale = fp32(amax / 448)); returns (rows, div codes)."""
    rng = np.random.default_rng(seed)
    found_x, found_a = [], []
    mids = ((POS[:-1] + POS[1:]) / 2)[8:]  # normal midpoints
    while len(found_x) < n:
        amax = np.float32(rng.uniform(1e-3, 1e3))
        s = np.float32(amax / np.float32(448.0))
        m = mids[rng.integers(0, mids.size, 4096)]
        x = (m * np.float64(s)).astype(np.float32)
        for cand in (x, np.nextafter(x, np.float32(np.inf)), np.nextafter(x, np.float32(0))):
            ok = np.abs(cand) <= amax
            q_div = (cand / s).astype(np.float32)
            q_rcp = (cand * np.float32(np.float32(1.0) / s)).astype(np.float32)
            diff = ok & (encode_rne(np.clip(q_div, -448, 448)) !=
                         encode_rne(np.clip(q_rcp, -448, 448)))
            for v in cand[diff][: n - len(found_x)]:
                found_x.append(v)
                found_a.append(amax)
    rows = np.zeros((n, 1, 8), dtype=np.float32)
    rows[:, 0, 0] = found_a
    rows[:, 0, 1] = found_x
    s = (np.asarray(found_a, dtype=np.float32) / np.float32(448.0)).astype(np.float32)
    want = encode_rne(np.clip((np.asarray(found_x, np.float32) / s).astype(np.float32),
                              -448, 448))
    return rows, want


def test_quotient_is_a_division_not_a_reciprocal_product():
    rows, want = division_rows(64)
    codes, _ = ref.fp8_pth_quantize(torch.from_numpy(rows))
    np.testing.assert_array_equal(codes[:, 0, 1].numpy(), want)


# ---------------------------------------------------------------------------
# oracle: paged store and gather against a per-slot loop
# ---------------------------------------------------------------------------


def test_store_and_gather_match_a_per_slot_loop():
    torch.manual_seed(4)
    nb, bs, kvh, d = 6, 16, 2, 32
    t = 40
    k = torch.randn(t, kvh, d).to(torch.bfloat16)
    v = torch.randn(t, kvh, d).to(torch.bfloat16)
    slots = torch.randperm(nb * bs)[:t]
    slots[3] = -1  # padding
    views = [torch.zeros(nb, bs, kvh, d, dtype=torch.uint8),
             torch.zeros(nb, bs, kvh, 1), torch.zeros(nb, bs, kvh, d, dtype=torch.uint8),
             torch.zeros(nb, bs, kvh, 1)]
    ref.fp8_pth_store(k, v, slots, *views)
    for i in range(t):
        s = int(slots[i])
        if s < 0:
            continue
        for x, data, scale in ((k, views[0], views[1]), (v, views[2], views[3])):
            row = x[i].float()
            for h in range(kvh):
                amax = row[h].abs().max()
                sc = torch.clamp(amax / 448.0, min=1e-6)
                assert scale[s // bs, s % bs, h, 0] == sc
                q = torch.clamp(row[h] / sc, -448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
                assert torch.equal(data[s // bs, s % bs, h], q)
    # gather: positions of two requests over a table with an unallocated tail
    table = torch.tensor([[2, 0, -1], [5, 1, 3]])
    lens = [20, 41]
    dk, dv = ref.fp8_pth_gather(*views, table, lens, torch.bfloat16)
    assert dk.shape == (61, kvh, d) and dk.dtype == torch.bfloat16
    row = 0
    for b, n in enumerate(lens):
        for p in range(n):
            blk = int(table[b, p // bs])
            want = (views[0][blk, p % bs].view(torch.float8_e4m3fn).float() *
                    views[1][blk, p % bs]).to(torch.bfloat16)
            assert torch.equal(dk[row], want)
            row += 1


# ---------------------------------------------------------------------------
# host contract (the reference's tests of the same names)
# ---------------------------------------------------------------------------


def test_layout_contract():
    layout = resolve_layout("fp8_per_token_head", HEAD)
    assert isinstance(layout, KVCacheLayout)
    assert layout.storage_dtype == "uint8" and layout.packed_last_dim == HEAD
    assert layout.quant_mode is KVQuantMode.FP8_PER_TOKEN_HEAD
    with pytest.raises(ValueError, match="divisible by 4"):
        resolve_layout("fp8_per_token_head", 126)


def test_method_discovery_and_fail_closed_adapter():
    method = get_method("fp8_per_token_head", head_size=HEAD, num_kv_heads=KVH)
    assert method.spec.dtype == "fp8_per_token_head"
    assert method.spec.requires_gpu_kernels
    assert method.resolve_layout().quant_mode is KVQuantMode.FP8_PER_TOKEN_HEAD
    with pytest.raises(ValueError, match="no adapter wired"):
        method.host_adapter("vllm_ascend_hust")
    with pytest.raises(ValueError, match="divisible by 4"):
        get_method("fp8_per_token_head", head_size=126)
    assert method.semantics.describe()["encoding"] == "e4m3fn (max normal 448)"


def test_region_budget_matches_host_page_size():
    layout = Fp8PerTokenHeadLayout(NB, BLOCK, KVH, HEAD)
    assert layout.bytes_per_token_head == HEAD + 4
    host_page = 2 * BLOCK * KVH * HEAD + 2 * BLOCK * KVH * 4
    assert 2 * layout.region_bytes == NB * host_page
    assert layout.compression_vs_fp16() == pytest.approx(256 / 132)
    assert layout.describe()["bytes_per_token"] == 2 * KVH * (HEAD + 4)


def test_views_alias_host_buffers():
    layout = Fp8PerTokenHeadLayout(NB, BLOCK, KVH, HEAD)
    key_buf = torch.zeros(NB, BLOCK, KVH, layout.bytes_per_token_head, dtype=torch.uint8)
    value_buf = torch.zeros_like(key_buf)
    k_data, k_scale, v_data, v_scale = fp8_caches_from_byte_tensors(key_buf, value_buf, layout)
    assert k_data.shape == (NB, BLOCK, KVH, HEAD) and k_data.dtype is torch.uint8
    assert k_scale.shape == (NB, BLOCK, KVH, 1) and k_scale.dtype is torch.float32
    assert v_data.shape == k_data.shape and v_scale.shape == k_scale.shape
    data_bytes = NB * BLOCK * KVH * HEAD
    key_buf.reshape(-1).view(torch.float32)[data_bytes // 4] = 2.5
    assert float(k_scale[0, 0, 0, 0]) == 2.5
    value_buf.reshape(-1).view(torch.float32)[data_bytes // 4] = -0.75
    assert float(v_scale[0, 0, 0, 0]) == -0.75


def test_layout_derivation_and_fail_closed():
    s = HEAD + 4
    key_buf = torch.zeros(NB, BLOCK, KVH, s, dtype=torch.uint8)
    layout = fp8_per_token_head_layout(key_buf, torch.zeros_like(key_buf), num_kv_heads=KVH,
                                       head_size=HEAD)
    assert (layout.num_blocks, layout.block_size) == (NB, BLOCK)
    with pytest.raises(RuntimeError, match="equal regions"):
        fp8_per_token_head_layout(key_buf, key_buf[:, :, :, : s - 8].contiguous(),
                                  num_kv_heads=KVH, head_size=HEAD)
    short = key_buf[:, :, :, : s - 4].contiguous()
    with pytest.raises(RuntimeError, match="whole number of pages"):
        fp8_per_token_head_layout(short, short.clone(), num_kv_heads=KVH, head_size=HEAD)


def test_quant_params_match_host_kernel():
    assert fp8_ops.QUANT_PARAMS[torch.float8_e4m3fn] == (448.0, -448.0)
    assert fp8_ops.QUANT_PARAMS[torch.int8] == (127.0, -128.0)


def _store_views():
    layout = Fp8PerTokenHeadLayout(NB, BLOCK, KVH, HEAD)
    key_buf = torch.zeros(NB, BLOCK, KVH, layout.bytes_per_token_head, dtype=torch.uint8)
    return fp8_caches_from_byte_tensors(key_buf, torch.zeros_like(key_buf), layout)


def test_store_validators_fail_closed():
    k_data, k_scale, v_data, v_scale = _store_views()
    key = torch.randn(4, KVH, HEAD)
    value = torch.randn(4, KVH, HEAD)
    slots = torch.arange(4, dtype=torch.long)

    def expect_reject(match, **overrides):
        args = dict(key=key, value=value, slot_mapping=slots, k_data=k_data, k_scale=k_scale,
                    v_data=v_data, v_scale=v_scale)
        args.update(overrides)
        with pytest.raises(RuntimeError, match=match):
            fp8_ops.validate_store_args(**args)

    expect_reject("token-head grids", value=torch.randn(4, KVH + 1, HEAD))
    expect_reject("equal key/value head", value=torch.randn(4, KVH, HEAD + 8))
    expect_reject("divisible by 4", key=torch.randn(4, KVH, 126), value=torch.randn(4, KVH, 126))
    expect_reject("1D of 4", slot_mapping=torch.arange(4).view(2, 2))
    expect_reject("int32/int64", slot_mapping=slots.to(torch.float32))
    expect_reject("uint8", k_data=k_data.to(torch.int32).contiguous())
    expect_reject("float32", k_scale=k_scale.to(torch.float64).contiguous())
    expect_reject("key data cache must be uint8", k_data=k_data[:, :, :, : HEAD - 4].contiguous())
    expect_reject("share a device", k_data=k_data.to("meta"))
    expect_reject("must be contiguous", k_data=k_data[:, :, :, : HEAD - 4])


def test_store_wrapper_launch_contract(monkeypatch):
    k_data, k_scale, v_data, v_scale = _store_views()
    captured = {}

    def fake_launch(key, value, slot_mapping, kd, ks, vd, vs, qmax, qmin, is_int_quant):
        captured.update(kd=kd, ks=ks, vd=vd, vs=vs, qmax=qmax, qmin=qmin, is_int=is_int_quant)

    monkeypatch.setattr(fp8_ops, "_launch_kernel", fake_launch)
    fp8_ops.fp8_per_token_head_store(torch.randn(4, KVH, HEAD), torch.randn(4, KVH, HEAD),
                                     torch.arange(4), k_data, k_scale, v_data, v_scale)
    assert (captured["qmax"], captured["qmin"]) == (448.0, -448.0)
    assert captured["is_int"] is False
    assert captured["kd"].dtype is torch.float8_e4m3fn
    assert captured["vd"].dtype is torch.float8_e4m3fn
    assert captured["kd"].view(torch.uint8).data_ptr() == k_data.data_ptr()
    assert captured["vd"].view(torch.uint8).data_ptr() == v_data.data_ptr()
    assert captured["ks"].data_ptr() == k_scale.data_ptr()


def test_store_wrapper_no_launch_on_empty_and_rejects_first(monkeypatch):
    k_data, k_scale, v_data, v_scale = _store_views()
    launches = []
    monkeypatch.setattr(fp8_ops, "_launch_kernel", lambda *a, **kw: launches.append(a))
    empty = torch.zeros(0, KVH, HEAD)
    fp8_ops.fp8_per_token_head_store(empty, empty.clone(), torch.zeros(0, dtype=torch.long),
                                     k_data, k_scale, v_data, v_scale)
    assert launches == []
    with pytest.raises(RuntimeError, match="token-head grids"):
        fp8_ops.fp8_per_token_head_store(torch.randn(2, KVH, HEAD), torch.randn(2, KVH + 1, HEAD),
                                         torch.arange(2), k_data, k_scale, v_data, v_scale)
    assert launches == []


def test_store_without_gpu_fails_loudly():
    k_data, k_scale, v_data, v_scale = _store_views()
    with pytest.raises(RuntimeError, match="no CPU fallback|not built"):
        fp8_ops.fp8_per_token_head_store(torch.randn(2, KVH, HEAD), torch.randn(2, KVH, HEAD),
                                         torch.arange(2), k_data, k_scale, v_data, v_scale)


def test_gather_metadata_checks():
    k_data, k_scale, v_data, v_scale = _store_views()
    table = torch.tensor([[0, 1], [2, -1]])
    with pytest.raises(RuntimeError, match="invalid block ids"):
        fp8_ops.fp8_per_token_head_dequant_gather(k_data, k_scale, v_data, v_scale, table,
                                                  [10, 200], torch.bfloat16)
    with pytest.raises(RuntimeError, match="outside the cache"):
        fp8_ops.fp8_per_token_head_dequant_gather(k_data, k_scale, v_data, v_scale,
                                                  torch.tensor([[0, NB]]), [200],
                                                  torch.bfloat16)
    with pytest.raises(RuntimeError, match="does not cover"):
        fp8_ops.fp8_per_token_head_dequant_gather(k_data, k_scale, v_data, v_scale,
                                                  torch.tensor([[0, 1]]), [300], torch.bfloat16)
    # an unallocated tail past the live pages is fine (it is never read)
    with pytest.raises(RuntimeError, match="no CPU fallback|not built"):
        fp8_ops.fp8_per_token_head_dequant_gather(k_data, k_scale, v_data, v_scale, table,
                                                  [10, 100], torch.bfloat16)
