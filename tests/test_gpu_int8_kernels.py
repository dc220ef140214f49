# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the INT8 dynamic per-channel HIP kernels against the oracle.

Scales and codes are bit-exact (every step rounds to the activation dtype as
torch does); paged dequant is bit-exact; decode attention is within
atol/rtol 1e-2 of the oracle's dequant followed by fp32 SDPA.
"""

from __future__ import annotations

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._util import make_kv, shuffled_table, slots_for

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("t,kvh,d", [(16, 2, 8), (300, 8, 128), (1, 4, 64),
                                     (5000, 16, 256),  # two 2048-channel chunks, 5 token slices
                                     (700, 3, 40)])    # 15 threads per row, 17 phases
def test_int8_scales_and_quant_bit_exact(gpu_device, dtype, t, kvh, d):
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_calc_scales, int8_quant_scatter

    key, value = make_kv(t, kvh, d, dtype=dtype, seed=t + d)
    if t > 1:
        key[:, 0, 0] = 0  # an all-zero channel exercises the 1e-12 clamp
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(key, value)
    g_k_inv, g_v_inv, g_k_aq, g_v_aq = int8_calc_scales(key.to(gpu_device), value.to(gpu_device))
    for want, got in ((k_inv, g_k_inv), (v_inv, g_v_inv), (k_aq, g_k_aq), (v_aq, g_v_aq)):
        got = got.cpu().reshape(want.shape)
        assert torch.equal(want, got) or (want.isinf() == got.isinf()).all() and torch.equal(
            want[~want.isinf()], got[~got.isinf()]
        )
    bs, nb = 16, (t + 15) // 16 + 2
    slots = torch.randperm(nb * bs, generator=torch.Generator().manual_seed(1))[:t]
    if t > 2:
        slots[1] = -1  # padding token
    kc = torch.zeros(nb, bs, kvh, d, dtype=torch.int8)
    vc = torch.zeros_like(kc)
    ref.int8_reshape_and_cache(key, value, k_inv, v_inv, slots, kc, vc)
    gkc = torch.zeros_like(kc, device=gpu_device)
    gvc = torch.zeros_like(gkc)
    int8_quant_scatter(
        key.to(gpu_device), value.to(gpu_device), g_k_inv, g_v_inv, slots.to(gpu_device), gkc, gvc
    )
    if dtype == torch.float16 and t > 1:
        # fp16 cannot hold the 1e-12 clamp: the zero channel's inv is inf and
        # 0*inf is NaN, whose int8 cast is platform-defined; compare the rest
        kc[..., 0, 0] = 0
        gkc[..., 0, 0] = 0
    assert torch.equal(kc, gkc.cpu())
    assert torch.equal(vc, gvc.cpu())


def _int8_state(dev, b, lens, kvh, d, bs, dtype, seed):
    nblk = [-(-n // bs) for n in lens]
    nb = sum(nblk) + 3
    maxb = max(nblk)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    table = torch.zeros(b, maxb, dtype=torch.int32)
    used = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[used : used + n]
        used += n
    kc = torch.zeros(nb, bs, kvh, d, dtype=torch.int8)
    vc = torch.zeros_like(kc)
    first_k, first_v = make_kv(max(lens), kvh, d, dtype=dtype, seed=seed)
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(first_k, first_v)
    for i, n in enumerate(lens):
        key, value = make_kv(n, kvh, d, dtype=dtype, seed=seed + 1 + i)
        ref.int8_reshape_and_cache(
            key, value, k_inv, v_inv, slots_for(table[i], range(n), bs), kc, vc
        )
    return table, kc, vc, k_inv, v_inv, k_aq, v_aq


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_int8_dequant_gather_bit_exact(gpu_device, dtype):
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_dequant_gather

    lens = [37, 128, 1, 200]
    table, kc, vc, k_inv, v_inv, k_aq, v_aq = _int8_state(gpu_device, 4, lens, 4, 64, 32, dtype, 3)
    want_k, want_v = ref.int8_paged_dequant(kc, vc, table, lens, dtype, k_inv, v_inv)
    got_k, got_v = int8_dequant_gather(
        kc.to(gpu_device), vc.to(gpu_device), table.to(gpu_device), lens, dtype,
        k_aq.to(gpu_device), v_aq.to(gpu_device),
    )
    assert torch.equal(want_k, got_k.cpu())
    assert torch.equal(want_v, got_v.cpu())


@pytest.mark.parametrize("rep", [1, 4, 8])
@pytest.mark.parametrize("kvh,d,bs", [(2, 64, 16), (8, 128, 128), (4, 128, 32), (16, 128, 64)])
def test_int8_decode_matches_oracle(gpu_device, rep, kvh, d, bs):
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_decode_attention

    dtype = torch.bfloat16
    lens = [513, 7, 128, 1000]
    table, kc, vc, k_inv, v_inv, k_aq, v_aq = _int8_state(gpu_device, 4, lens, kvh, d, bs, dtype, 8)
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(2)).to(dtype)
    scale = d ** -0.5
    # antiquant semantics: code * aq with aq = dtype(1/inv), evaluated in fp32
    dk, dv = ref.int8_paged_dequant(kc, vc, table, lens, torch.float32, k_inv, v_inv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    for split in (None, 100):
        got = int8_decode_attention(
            q.to(gpu_device), kc.to(gpu_device), vc.to(gpu_device), k_aq.to(gpu_device),
            v_aq.to(gpu_device), table.to(gpu_device), lens, scale, split_tokens=split,
        )
        torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


def test_int8_decode_empty_request_is_zero(gpu_device):
    """A request with no cached tokens gets an empty work item: its output is
    zero and the other requests still match the oracle."""
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_decode_attention

    dtype = torch.bfloat16
    kvh, d, bs, rep = 8, 128, 128, 4
    lens = [300, 0, 129]
    table, kc, vc, k_inv, v_inv, k_aq, v_aq = _int8_state(gpu_device, 3, lens, kvh, d, bs, dtype, 5)
    hq = kvh * rep
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(4)).to(dtype)
    scale = d ** -0.5
    got = int8_decode_attention(
        q.to(gpu_device), kc.to(gpu_device), vc.to(gpu_device), k_aq.to(gpu_device),
        v_aq.to(gpu_device), table.to(gpu_device), lens, scale,
    ).float().cpu()
    assert torch.equal(got[1], torch.zeros_like(got[1]))
    live = [0, 2]
    dk, dv = ref.int8_paged_dequant(kc, vc, table[live], [lens[i] for i in live], torch.float32,
                                    k_inv, v_inv)
    want = ref.attention(q[live], dk, dv, [1, 1], [lens[i] for i in live], scale, causal=True)
    torch.testing.assert_close(got[live], want, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("kvh,d,bs,rep", [(8, 128, 128, 4), (4, 64, 32, 2)])
def test_int8_decode_with_row_maxima_growing_every_block(gpu_device, kvh, d, bs, rep):
    """Keys along one direction per kv head with a magnitude that grows with
    the position (even heads) or shrinks (odd heads), queries along it: the
    even heads' running maximum rises on every block of every item, so the
    online softmax rescales each time; split items too."""
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_decode_attention

    dtype = torch.bfloat16
    lens = [513, 1000, 129]
    u = torch.randn(kvh, d, generator=torch.Generator().manual_seed(23))
    u = u / u.norm(dim=1, keepdim=True)
    sign = torch.tensor([1.0 if h % 2 == 0 else -1.0 for h in range(kvh)])

    def make(n, seed):
        gen = torch.Generator().manual_seed(seed)
        pos = torch.arange(n, dtype=torch.float32)
        key = u[None] * (sign[None, :, None] * 0.05 * pos[:, None, None]) + 0.05 * torch.randn(
            n, kvh, d, generator=gen)
        return key.to(dtype), torch.randn(n, kvh, d, generator=gen).to(dtype)

    nblk = [-(-n // bs) for n in lens]
    nb = sum(nblk) + 3
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(7))
    table = torch.zeros(len(lens), max(nblk), dtype=torch.int32)
    used = 0
    for i, n in enumerate(nblk):
        table[i, :n] = perm[used : used + n]
        used += n
    kc = torch.zeros(nb, bs, kvh, d, dtype=torch.int8)
    vc = torch.zeros_like(kc)
    # scales from the longest ramp, so no request's keys clip
    first_k, first_v = make(max(lens), 99)
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(first_k, first_v)
    for i, n in enumerate(lens):
        key, value = make(n, 100 + i)
        ref.int8_reshape_and_cache(key, value, k_inv, v_inv, slots_for(table[i], range(n), bs),
                                   kc, vc)
    hq = kvh * rep
    q = (8.0 * u.repeat_interleave(rep, dim=0)[None].expand(len(lens), hq, d)
         + 0.05 * torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(3)))
    q = q.to(dtype)
    scale = d ** -0.5
    dk, dv = ref.int8_paged_dequant(kc, vc, table, lens, torch.float32, k_inv, v_inv)
    want = ref.attention(q, dk, dv, [1] * len(lens), lens, scale, causal=True)
    for split in (None, 256):
        got = int8_decode_attention(
            q.to(gpu_device), kc.to(gpu_device), vc.to(gpu_device), k_aq.to(gpu_device),
            v_aq.to(gpu_device), table.to(gpu_device), lens, scale, split_tokens=split,
        )
        torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)
