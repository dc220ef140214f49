# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head HIP kernels against the oracle (GPU).

* gfx950's E4M3 conversion inside the store kernel, at every rounding
  boundary of the format (rows whose scale is exactly 1, so the kernel's
  quotient is the test value itself), matches the independent encoder;
* rows built so that ``x / scale`` and ``x * (1/scale)`` round to different
  codes follow the division, as the reference semantics does;
* the paged store is bit-exact against the oracle (codes and scales, the
  whole page image, padding slots untouched) for bf16 / fp16 / fp32 inputs,
  int32 / int64 slots and head sizes that exercise every lane width (16, 8
  and 4 codes a lane) and group shape, including partly idle groups;
* the gather is bit-exact against the oracle's dequantize-then-cast, with
  unallocated tail ids;
* attention over the paged codes is within 1e-2 of fp32 attention over the
  oracle's dequantized K/V;
* at a full-size shape (32 requests x 4096 positions, 8 KV heads) a round trip
  of grid values with power-of-two scales is the identity.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kvq_oracle as ref
from tests.test_fp8_per_token_head import E4M3, boundary_points, division_rows, encode_rne
from vllm_ascend_quantized_kv_cache.methods.fp8_per_token_head.byte_cache import (
    Fp8PerTokenHeadLayout,
    fp8_caches_from_byte_tensors,
)
from vllm_ascend_quantized_kv_cache.methods.fp8_per_token_head.semantics import (
    Fp8PerTokenHeadSemantics,
)
from vllm_ascend_quantized_kv_cache.ops import fp8_ops

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-2, rtol=1e-2)


def _views(device, nb, bs, kvh, d, fill=0):
    """(key buffer, value buffer, (k_data, k_scale, v_data, v_scale)) on device."""
    layout = Fp8PerTokenHeadLayout(nb, bs, kvh, d)
    kb = torch.full((nb, bs, kvh, layout.bytes_per_token_head), fill, dtype=torch.uint8,
                    device=device)
    vb = kb.clone()
    return kb, vb, fp8_caches_from_byte_tensors(kb, vb, layout)


def _store_rows(device, rows: np.ndarray) -> np.ndarray:
    """Codes the store kernel gives for fp32 rows ``[T, 1, D]`` (slot t = row t)."""
    t, kvh, d = rows.shape
    _, _, views = _views(device, 1, t, kvh, d)
    x = torch.from_numpy(rows).to(device)
    fp8_ops.fp8_per_token_head_store(x, x, torch.arange(t, device=device), *views)
    torch.cuda.synchronize()
    return views[0][0].cpu().numpy()


def test_hardware_e4m3_conversion_at_every_rounding_boundary(gpu_device):
    pts = boundary_points()
    per_row = 127
    n = -(-pts.size // per_row)
    rows = np.zeros((n, 1, 128), dtype=np.float32)
    rows[:, 0, 0] = 448.0  # amax 448 -> scale exactly 1
    flat = rows[:, 0, 1:].reshape(-1)
    flat[: pts.size] = pts
    rows[:, 0, 1:] = flat.reshape(n, per_row)
    codes = _store_rows(gpu_device, rows)
    np.testing.assert_array_equal(codes[:, 0, :], encode_rne(rows[:, 0, :]))
    # negative zero keeps its sign bit, as the oracle's cast does
    rows = np.zeros((1, 1, 8), dtype=np.float32)
    rows[0, 0, :3] = (448.0, -0.0, 0.0)
    assert list(_store_rows(gpu_device, rows)[0, 0, :3]) == [0x7E, 0x80, 0x00]


def test_quotient_is_a_division_on_the_gpu(gpu_device):
    rows, want = division_rows(256, seed=11)
    codes = _store_rows(gpu_device, rows)
    np.testing.assert_array_equal(codes[:, 0, 1], want)
    oc, _ = ref.fp8_pth_quantize(torch.from_numpy(rows))
    np.testing.assert_array_equal(codes, oc.numpy())


def _inputs(t, kvh, d, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    scales = torch.exp(torch.randn((1, kvh, 1), generator=gen) * 2)
    x = torch.randn((t, kvh, d), generator=gen) * scales
    x[0, 0] = 0.0  # an all-zero row: the floor scale
    if t > 2:
        x[2, -1, d // 3] = 3.0e4  # an outlier in one (token, head)
        x[1, 0, : d // 2] = 0.0
    return x.to(dtype)


@pytest.mark.parametrize(
    "dtype,d,kvh,index",
    [
        (torch.bfloat16, 128, 8, torch.int64),
        (torch.bfloat16, 64, 4, torch.int32),
        (torch.float16, 128, 8, torch.int32),
        (torch.float32, 128, 2, torch.int64),
        (torch.bfloat16, 96, 3, torch.int64),   # 12 lanes of a 16-lane group
        (torch.bfloat16, 100, 2, torch.int64),  # D % 8 == 4: 4 codes a lane
        (torch.float32, 36, 5, torch.int32),
        (torch.bfloat16, 256, 2, torch.int64),
        (torch.bfloat16, 512, 1, torch.int32),  # one wave per row
        (torch.float16, 8, 8, torch.int64),     # one lane per row
        (torch.bfloat16, 40, 3, torch.int64),   # 8 codes a lane, 5 lanes of 8
        (torch.float32, 24, 2, torch.int32),    # 8 codes a lane, 3 lanes of 4
    ],
)
def test_store_matches_oracle_bit_exact(gpu_device, dtype, d, kvh, index):
    nb, bs = 9, 16
    t = 100
    x_k = _inputs(t, kvh, d, dtype, seed=d + kvh)
    x_v = _inputs(t, kvh, d, dtype, seed=d * 7 + kvh)
    gen = torch.Generator().manual_seed(d)
    slots = torch.randperm(nb * bs, generator=gen)[:t]
    slots[5] = -1
    slots[40] = -7
    kb, vb, views = _views(gpu_device, nb, bs, kvh, d, fill=0xA5)
    fp8_ops.fp8_per_token_head_store(x_k.to(gpu_device), x_v.to(gpu_device),
                                     slots.to(index).to(gpu_device), *views)
    torch.cuda.synchronize()
    # the oracle writes into the same page images (padding slots keep 0xA5)
    okb = torch.full(kb.shape, 0xA5, dtype=torch.uint8)
    ovb = okb.clone()
    layout = Fp8PerTokenHeadLayout(nb, bs, kvh, d)
    ref.fp8_pth_store(x_k, x_v, slots, *fp8_caches_from_byte_tensors(okb, ovb, layout))
    assert torch.equal(kb.cpu(), okb), "key page image differs"
    assert torch.equal(vb.cpu(), ovb), "value page image differs"


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d,kvh", [(128, 8), (100, 2), (64, 4), (40, 3)])
def test_gather_matches_oracle_bit_exact(gpu_device, out_dtype, d, kvh):
    nb, bs = 12, 16
    lens = [37, 16, 0, 70]
    table = torch.tensor([[3, 7, 11, -1, -1], [0, -1, -1, -1, -1], [-1] * 5,
                          [1, 2, 4, 5, 6]])
    gen = torch.Generator().manual_seed(d)
    x_k = _inputs(nb * bs, kvh, d, torch.bfloat16, seed=1)
    x_v = _inputs(nb * bs, kvh, d, torch.bfloat16, seed=2)
    slots = torch.randperm(nb * bs, generator=gen)
    kb, vb, views = _views(gpu_device, nb, bs, kvh, d)
    fp8_ops.fp8_per_token_head_store(x_k.to(gpu_device), x_v.to(gpu_device),
                                     slots.to(gpu_device), *views)
    for index in (torch.int32, torch.int64):
        dk, dv = fp8_ops.fp8_per_token_head_dequant_gather(
            *views, table.to(index).to(gpu_device), lens, out_dtype)
        torch.cuda.synchronize()
        cpu_views = [v.cpu() for v in views]
        wk, wv = ref.fp8_pth_gather(*cpu_views, table, lens, out_dtype)
        assert dk.dtype == out_dtype and dk.shape == (sum(lens), kvh, d)
        assert torch.equal(dk.cpu(), wk) and torch.equal(dv.cpu(), wv)


def test_semantics_object_matches_oracle(gpu_device):
    sem = Fp8PerTokenHeadSemantics(type("Cfg", (), {"head_size": 128})())
    x = _inputs(33, 4, 128, torch.bfloat16, seed=9)
    q, s = sem.quantize(x.to(gpu_device))
    oq, os_ = ref.fp8_pth_quantize(x)
    assert q.dtype == torch.float8_e4m3fn
    assert torch.equal(q.view(torch.uint8).cpu(), oq) and torch.equal(s.cpu(), os_)
    assert torch.equal(sem.compute_scale(x.to(gpu_device)).cpu(), os_)
    back = sem.dequantize(q, s)
    assert torch.equal(back.cpu(), ref.fp8_pth_dequantize(oq, os_))
    fq = sem.fake_quant(x.to(gpu_device))
    assert torch.equal(fq.cpu(), ref.fp8_pth_dequantize(oq, os_).to(torch.bfloat16))
    assert sem.quantize(x[:0].to(gpu_device))[0].shape == (0, 4, 128)


@pytest.mark.parametrize("query_lens", [[1, 1, 1, 1], [5, 1, 17, 40]])
def test_attention_over_paged_codes(gpu_device, query_lens):
    nb, bs, kvh, hq, d = 40, 16, 4, 16, 128
    lens = [150, 33, 97, 300]
    gen = torch.Generator().manual_seed(13)
    perm = torch.randperm(nb, generator=gen)
    maxb = -(-max(lens) // bs)
    table = torch.full((len(lens), maxb), -1, dtype=torch.int64)
    used = 0
    for b, n in enumerate(lens):
        k = -(-n // bs)
        table[b, :k] = perm[used:used + k]
        used += k
    slots = torch.cat([table[b, torch.arange(n) // bs] * bs + torch.arange(n) % bs
                       for b, n in enumerate(lens)])
    x_k = torch.randn((sum(lens), kvh, d), generator=gen).to(torch.bfloat16)
    x_v = torch.randn((sum(lens), kvh, d), generator=gen).to(torch.bfloat16)
    _, _, views = _views(gpu_device, nb, bs, kvh, d)
    fp8_ops.fp8_per_token_head_store(x_k.to(gpu_device), x_v.to(gpu_device),
                                     slots.to(gpu_device), *views)
    q = (torch.randn((sum(query_lens), hq, d), generator=gen)).to(torch.bfloat16)
    out = fp8_ops.fp8_per_token_head_attention(
        q.to(gpu_device), *views, table.to(gpu_device), lens, query_lens, d ** -0.5,
        block_table_host=table.numpy())
    torch.cuda.synchronize()
    dk, dv = ref.fp8_pth_gather(*[v.cpu() for v in views], table, lens, torch.float32)
    want = ref.attention(q.float(), dk, dv, query_lens, lens, d ** -0.5, True)
    torch.testing.assert_close(out.float().cpu(), want, **TOL)


def test_full_size_round_trip_of_grid_values(gpu_device):
    """32 requests x 4096 positions x 8 KV heads x 128: values on the E4M3 grid
    times 2^k, with 448 * 2^k in each row, come back exactly."""
    b, n, kvh, d, bs = 32, 4096, 8, 128, 128
    t = b * n
    gen = torch.Generator(device=gpu_device).manual_seed(21)
    codes = torch.randint(0, 0x7E, (t, kvh, d), generator=gen, device=gpu_device,
                          dtype=torch.int32)
    codes |= torch.randint(0, 2, codes.shape, generator=gen, device=gpu_device,
                           dtype=torch.int32) << 7
    codes[:, :, 5] = 0x7E
    grid = torch.from_numpy(E4M3.astype(np.float32)).to(gpu_device)
    k = torch.randint(-8, 8, (t, kvh, 1), generator=gen, device=gpu_device).float()
    x = (grid[codes.long()] * torch.exp2(k)).to(torch.bfloat16)  # exact in bf16
    del codes
    nb = t // bs + 3
    perm = torch.randperm(nb, generator=gen, device=gpu_device)[: t // bs]
    table = perm.view(b, n // bs)
    slots = (table.view(-1, 1) * bs + torch.arange(bs, device=gpu_device)).view(-1)
    _, _, views = _views(gpu_device, nb, bs, kvh, d)
    fp8_ops.fp8_per_token_head_store(x, x, slots, *views)
    dk, dv = fp8_ops.fp8_per_token_head_dequant_gather(
        *views, table, [n] * b, torch.bfloat16, block_table_host=table.cpu().numpy())
    torch.cuda.synchronize()
    assert torch.equal(dk, x) and torch.equal(dv, x)
    assert torch.equal(views[1].view(-1, kvh)[slots], torch.exp2(k).view(t, kvh))
