# SPDX-License-Identifier: Apache-2.0
"""End-to-end GPU parity of the attention mixins (every HIP kernel in the loop).

One multi-step serving flow (bulk prefill, a run of decode steps that crosses
key flushes and value evictions, a fall-through cache-hit chunk, a chunked
prefill with decode rows) is driven twice with identical inputs:

* through the mixin on the GPU, with its real launch hooks (ring write,
  gather-pack, gather-dequant with overlay, fused decode, MFMA prefill);
* through the same mixin on the CPU with oracle-backed hooks.

The packed int4 codes, the fp32 scales/mins and the residual rings must be
bit-identical after every step; attention outputs agree within atol/rtol
1e-2 of the oracle's fp32 attention.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._cpu_kernels import install_cpu_kernels
from vllm_ascend_quantized_kv_cache.methods.int8_dynamic.attention_backend import (
    AscendInt8AttentionBackendMixin,
)
from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import attention_backend as ab
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.byte_cache import KiviByteCacheLayout

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-2, rtol=1e-2)


def _make_kivi(device, *, head, kvh, hq, group, residual, block, num_blocks, rows):
    class Impl(ab.AscendKiviInt4AttentionBackendMixin):
        pass

    impl = Impl()
    impl.num_heads, impl.num_kv_heads, impl.head_size = hq, kvh, head
    impl.scale = head ** -0.5
    impl._init_kivi_state(None)
    impl.enable_kivi = True
    impl.kivi_group_size, impl.kivi_residual_length = group, residual
    impl.kivi_max_num_seqs = rows
    # the host's form: two uint8 page buffers the mixin slices into six views
    layout = KiviByteCacheLayout(num_blocks, block, kvh, head, group)
    kbuf = torch.zeros((num_blocks, block, kvh, layout.bytes_per_token_head),
                       dtype=torch.uint8, device=device)
    impl._bind_kivi_cache((kbuf, torch.zeros_like(kbuf)))
    assert impl.k_quant_cache.data_ptr() == kbuf.data_ptr()
    return impl


def _md(state, **kw):
    base = dict(attn_state=SimpleNamespace(name=state), causal=True, finished_req_ids=None)
    base.update(kw)
    return SimpleNamespace(**base)


def _assert_same_state(gpu, cpu):
    for a, b in zip(gpu._kivi_caches(), cpu._kivi_caches()):
        assert torch.equal(a.cpu(), b), "packed history differs"
    rg, rc = gpu._kivi_ring, cpu._kivi_ring
    assert rg.state() == rc.state()
    assert torch.equal(rg.key.cpu(), rc.key) and torch.equal(rg.value.cpu(), rc.value)


GEOMS = {
    # production: MFMA decode path (D=128, G>=32, GQA 5)
    "d128_g128": dict(head=128, kvh=8, hq=40, group=128, residual=128, block=128),
    # config-5 style group of 64
    "d128_g64": dict(head=128, kvh=4, hq=16, group=64, residual=128, block=128),
    # small geometry: the generic decode kernel
    "d64_g32": dict(head=64, kvh=2, hq=4, group=32, residual=64, block=64),
}


@pytest.mark.parametrize("geom", list(GEOMS))
def test_kivi_mixin_serving_flow_matches_oracle(gpu_device, geom):
    g = GEOMS[geom]
    head, kvh, hq, group, residual, block = (g[k] for k in
                                             ("head", "kvh", "hq", "group", "residual", "block"))
    nb, rows = 24, 4
    gen = torch.Generator().manual_seed(list(GEOMS).index(geom))
    dt = torch.bfloat16
    gpu = _make_kivi(gpu_device, num_blocks=nb, rows=rows, **g)
    cpu = _make_kivi("cpu", num_blocks=nb, rows=rows, **g)
    install_cpu_kernels(cpu)
    perm = torch.randperm(nb, generator=gen)
    table = perm[:18].view(3, 6).to(torch.int64)
    reqs = ["a", "b", "c"]

    def slot(r, p):
        return int(table[r, p // block]) * block + p % block

    def step(md, q, k, v, out_shape):
        outs = []
        for impl, dev in ((gpu, gpu_device), (cpu, "cpu")):
            m = SimpleNamespace(**vars(md))
            for name in ("slot_mapping", "block_tables"):
                if hasattr(m, name):
                    setattr(m, name, getattr(m, name).to(dev))
            # the oracle side keeps its fp32 result (no second bf16 rounding)
            out = torch.zeros(out_shape, dtype=dt if impl is gpu else torch.float32,
                              device=dev)
            impl.forward(None, q.to(dev), None if k is None else k.to(dev),
                         None if v is None else v.to(dev), None, m, out)
            outs.append(out.float().cpu())
        torch.testing.assert_close(outs[0], outs[1], **TOL)
        _assert_same_state(gpu, cpu)

    def rnd(n, h):
        return torch.randn(n, h, head, generator=gen).to(dt)

    # 1. bulk prefill: lengths straddle the residual window
    lens = [residual + 3, 2 * residual + group // 2, 7]
    t = sum(lens)
    cu = [sum(lens[:i + 1]) for i in range(3)]
    slots = torch.tensor([slot(r, p) for r in range(3) for p in range(lens[r])])
    k = rnd(t, kvh) * torch.exp(torch.randn(kvh, head, generator=gen)).to(dt)
    step(_md("PrefillNoCache", actual_seq_lengths_q=cu, seq_lens_list=list(lens),
             slot_mapping=slots, block_tables=table, req_ids=reqs, num_actual_tokens=t),
         rnd(t, hq), k, rnd(t, kvh), (t, hq, head))

    # 2. decode steps crossing a key flush for every request
    for _ in range(residual + 5):
        new = torch.tensor([slot(r, lens[r]) for r in range(3)])
        lens = [n + 1 for n in lens]
        step(_md("DecodeOnly", seq_lens_list=list(lens), slot_mapping=new, block_tables=table,
                 req_ids=reqs, num_actual_tokens=3),
             rnd(3, hq), rnd(3, kvh), rnd(3, kvh), (3, hq, head))

    # 3. fall-through chunk on request c (incremental writes + gather + dense attention)
    n_new = 9
    sl = torch.tensor([slot(2, lens[2] + i) for i in range(n_new)])
    lens[2] += n_new
    step(_md("PrefillCacheHit", actual_seq_lengths_q=[n_new], seq_lens_list=[lens[2]],
             slot_mapping=sl, block_tables=table[2:3], req_ids=["c"],
             num_actual_tokens=n_new),
         rnd(n_new, hq), rnd(n_new, kvh), rnd(n_new, kvh), (n_new, hq, head))

    # 4. chunked prefill: two decode rows + an all-new prompt in a fresh row
    prompt = 37
    new = [slot(0, lens[0]), slot(1, lens[1])]
    lens[0] += 1
    lens[1] += 1
    ptable = torch.cat([table[:2], perm[18:24].view(1, 6).to(torch.int64)])
    psl = [int(ptable[2, p // block]) * block + p % block for p in range(prompt)]
    step(_md("ChunkedPrefill", actual_seq_lengths_q=[1, 2, 2 + prompt],
             seq_lens_list=[lens[0], lens[1], prompt], num_decodes=2, num_decode_tokens=2,
             num_prefills=1, slot_mapping=torch.tensor(new + psl), block_tables=ptable,
             req_ids=["a", "b", "p"], num_actual_tokens=2 + prompt),
         rnd(2 + prompt, hq), rnd(2 + prompt, kvh), rnd(2 + prompt, kvh),
         (2 + prompt, hq, head))

    # 5. the dense K/V the GPU gather produces equal the oracle's, bit for bit
    gk, gv = gpu._gather_dequant_kivi_paged_cache(table.to(gpu_device), lens, dt, reqs)
    ck, cv = cpu._gather_dequant_kivi_paged_cache(table, lens, dt, reqs)
    assert torch.equal(gk.cpu(), ck) and torch.equal(gv.cpu(), cv)


def test_kivi_mixin_rollback_and_release_on_gpu(gpu_device):
    """Pruning a rolled-back window and releasing rows keep GPU and CPU rings equal."""
    g = GEOMS["d64_g32"]
    gpu = _make_kivi(gpu_device, num_blocks=8, rows=2, **g)
    cpu = _make_kivi("cpu", num_blocks=8, rows=2, **g)
    install_cpu_kernels(cpu)
    gen = torch.Generator().manual_seed(5)
    n = 50
    k = torch.randn(n, g["kvh"], g["head"], generator=gen).to(torch.bfloat16)
    v = torch.randn(n, g["kvh"], g["head"], generator=gen).to(torch.bfloat16)
    table = torch.tensor([[3, 1]])
    slots = torch.tensor([int(table[0, p // 64]) * 64 + p % 64 for p in range(n)])
    for impl, dev in ((gpu, gpu_device), (cpu, "cpu")):
        impl._write_kivi_cache(k.to(dev), v.to(dev), slots.to(dev), ["r"], [n])
        impl._sync_kivi_residual_windows(table.to(dev), [n - 13], ["r"])
    _assert_same_state(gpu, cpu)
    # the request regrows over the pruned positions with new content, then finishes
    k2 = torch.randn(13, g["kvh"], g["head"], generator=gen).to(torch.bfloat16)
    v2 = torch.randn(13, g["kvh"], g["head"], generator=gen).to(torch.bfloat16)
    for impl, dev in ((gpu, gpu_device), (cpu, "cpu")):
        impl._write_kivi_cache(k2.to(dev), v2.to(dev), slots[n - 13:].to(dev), ["r"], [13])
        impl._sync_kivi_residual_windows(table.to(dev), [n], ["r"])
    _assert_same_state(gpu, cpu)
    for impl, dev in ((gpu, gpu_device), (cpu, "cpu")):
        impl._sync_kivi_residual_windows(table.to(dev), [n], ["r"], finished_req_ids={"r"})
        assert impl._get_kivi_residual_row("r", create=False) is None
    _assert_same_state(gpu, cpu)


# ---------------------------------------------------------------------------
# INT8 mixin
# ---------------------------------------------------------------------------


def test_int8_mixin_prefill_then_decode_matches_oracle(gpu_device):
    hq, kvh, d, bs, nb = 32, 8, 128, 128, 40
    dt = torch.bfloat16

    class Impl(AscendInt8AttentionBackendMixin):
        num_heads, num_kv_heads, head_size, scale = hq, kvh, d, d ** -0.5

    impl = Impl()
    layer = SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)
    cache = torch.zeros(2, nb, bs, kvh, d, dtype=torch.int8, device=gpu_device)
    gen = torch.Generator().manual_seed(8)
    lens = [300, 129, 1]
    table = torch.randperm(nb, generator=gen)[:12].view(3, 4).to(torch.int64)
    slots = [int(table[b, p // bs]) * bs + p % bs for b, n in enumerate(lens) for p in range(n)]
    t = sum(lens)
    k = (torch.randn(t, kvh, d, generator=gen) * torch.exp(torch.randn(kvh, d, generator=gen)))
    k, v = k.to(dt), torch.randn(t, kvh, d, generator=gen).to(dt)
    q = torch.randn(t, hq, d, generator=gen).to(dt)
    md = SimpleNamespace(attn_state=SimpleNamespace(name="PrefillNoCache"),
                         model_runner_type="generate", causal=True,
                         slot_mapping=torch.tensor(slots, device=gpu_device),
                         num_actual_tokens=t, actual_seq_lengths_q=[300, 429, 430],
                         seq_lens_list=lens, block_tables=table.to(gpu_device))
    out = torch.zeros(t, hq, d, dtype=dt, device=gpu_device)
    impl.forward(layer, q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), cache, md, out)
    k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(k, v)
    assert torch.equal(layer._int8_k_inv_scale.cpu(), k_inv)
    assert torch.equal(layer._int8_v_aq_scale.cpu().flatten(), v_aq.flatten())
    want_cache = torch.zeros(2, nb, bs, kvh, d, dtype=torch.int8)
    ref.int8_reshape_and_cache(k, v, k_inv, v_inv, torch.tensor(slots), want_cache[0],
                               want_cache[1])
    assert torch.equal(cache.cpu(), want_cache)
    torch.testing.assert_close(out.float().cpu(), ref.attention(q, k, v, lens, lens, d ** -0.5,
                                                                True), **TOL)
    # one decode step per request
    kd = torch.randn(3, kvh, d, generator=gen).to(dt)
    vd = torch.randn(3, kvh, d, generator=gen).to(dt)
    qd = torch.randn(3, hq, d, generator=gen).to(dt)
    new = [int(table[b, n // bs]) * bs + n % bs for b, n in enumerate(lens)]
    lens = [n + 1 for n in lens]
    md = SimpleNamespace(attn_state=SimpleNamespace(name="DecodeOnly"),
                         model_runner_type="generate", causal=True,
                         slot_mapping=torch.tensor(new, device=gpu_device), num_actual_tokens=3,
                         seq_lens_list=lens, block_tables=table.to(gpu_device))
    out = torch.zeros(3, hq, d, dtype=dt, device=gpu_device)
    impl.forward(layer, qd.to(gpu_device), kd.to(gpu_device), vd.to(gpu_device), cache, md, out)
    ref.int8_reshape_and_cache(kd, vd, k_inv, v_inv, torch.tensor(new), want_cache[0],
                               want_cache[1])
    assert torch.equal(cache.cpu(), want_cache)
    # decode is FIA's per-channel antiquant: code * aq (aq = bf16(1/inv)) in fp32
    dk, dv = ref.int8_paged_dequant(want_cache[0], want_cache[1], table, lens, torch.float32,
                                    k_inv, v_inv)
    want = ref.attention(qd, dk, dv, [1, 1, 1], lens, d ** -0.5, True)
    torch.testing.assert_close(out.float().cpu(), want, **TOL)
