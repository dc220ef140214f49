# SPDX-License-Identifier: Apache-2.0
"""INT8 dynamic mixin on the CPU: calibration, cache writes and the branch
table of ``forward`` (``pkg/methods/int8_dynamic/attention_backend.py:34-404``).

The mixin's kernel entry points (``ops.int8_ops`` / ``ops.attention``) are
replaced by oracle-backed CPU versions; the HIP kernels behind them are
checked on the GPU in ``test_gpu_int8_kernels.py`` and ``test_gpu_mixins.py``.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._util import make_kv
from vllm_ascend_quantized_kv_cache.methods.int8_dynamic.attention_backend import (
    AscendInt8AttentionBackendMixin,
)

HQ, KVH, D, BS, NB = 4, 2, 16, 8, 12


def _gather_codes(cache, table, seq_lens):
    rows = []
    for b, n in enumerate(seq_lens):
        for p in range(n):
            rows.append(cache[int(table[b, p // BS]), p % BS])
    return torch.stack(rows) if rows else cache.new_zeros((0, KVH, D))


@pytest.fixture
def cpu_ops(monkeypatch):
    from vllm_ascend_quantized_kv_cache.ops import attention, int8_ops

    calls = {"decode": [], "dense": [], "dequant": []}

    def calc_scales(key, value):
        k_inv, v_inv, k_aq, v_aq = ref.int8_calc_scales(key, value)
        return k_inv, v_inv, k_aq.view(1, KVH, 1, D), v_aq.view(1, KVH, 1, D)

    def quant_scatter(key, value, k_inv, v_inv, slots, kc, vc):
        ref.int8_reshape_and_cache(key, value, k_inv, v_inv, slots, kc, vc)

    def dequant_gather(kc, vc, table, seq_lens, dtype, aq_k, aq_v):
        calls["dequant"].append(list(seq_lens))
        dk = _gather_codes(kc, table, seq_lens).to(dtype) * aq_k.reshape(KVH, D).to(dtype)
        dv = _gather_codes(vc, table, seq_lens).to(dtype) * aq_v.reshape(KVH, D).to(dtype)
        return dk, dv

    def decode(q, kc, vc, k_aq, v_aq, table, seq_lens, scale, out=None, **_):
        calls["decode"].append(list(seq_lens))
        dk, dv = dequant_gather(kc, vc, table, seq_lens, q.dtype, k_aq, v_aq)
        res = ref.attention(q, dk, dv, [1] * len(seq_lens), seq_lens, scale, True)
        out.copy_(res.to(out.dtype))
        return out

    def dense(q, k, v, q_lens, kv_lens, scale, causal, out=None):
        calls["dense"].append((list(q_lens), list(kv_lens)))
        out.copy_(ref.attention(q, k, v, q_lens, kv_lens, scale, causal).to(out.dtype))
        return out

    monkeypatch.setattr(int8_ops, "int8_calc_scales", calc_scales)
    monkeypatch.setattr(int8_ops, "int8_quant_scatter", quant_scatter)
    monkeypatch.setattr(int8_ops, "int8_dequant_gather", dequant_gather)
    monkeypatch.setattr(int8_ops, "int8_decode_attention", decode)
    monkeypatch.setattr(attention, "prefill_attention", dense)
    return calls


class _Host:
    num_heads, num_kv_heads, head_size, scale = HQ, KVH, D, D ** -0.5


class _Impl(AscendInt8AttentionBackendMixin, _Host):
    pass


def _layer():
    return SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)


def _cache():
    return torch.zeros(2, NB, BS, KVH, D, dtype=torch.int8)


def _md(state, **kw):
    base = dict(attn_state=SimpleNamespace(name=state), model_runner_type="generate",
                causal=True)
    base.update(kw)
    return SimpleNamespace(**base)


def test_forward_guards():
    impl = _Impl()
    out = torch.ones(2, HQ, D)
    assert impl.forward(_layer(), out, None, None, _cache(), None, out) is out
    assert not out.any()
    with pytest.raises(NotImplementedError, match="fused output quantization"):
        impl.forward(_layer(), out, None, None, _cache(), _md("DecodeOnly"), out,
                     output_scale=out)


def test_decode_without_calibration_fails_closed(cpu_ops):
    impl = _Impl()
    q = torch.randn(1, HQ, D)
    md = _md("DecodeOnly", seq_lens_list=[1], block_tables=torch.tensor([[0]]))
    with pytest.raises(RuntimeError, match="no scales yet"):
        impl.forward(_layer(), q, None, None, _cache(), md, torch.zeros_like(q))


def test_pooling_encoder_stays_with_host(cpu_ops):
    impl = _Impl()
    k, v = make_kv(4, KVH, D, dtype=torch.bfloat16)
    md = _md("PrefillNoCache", model_runner_type="pooling", causal=False,
             slot_mapping=torch.arange(4), num_actual_tokens=4, actual_seq_lengths_q=[4])
    q = torch.randn(4, HQ, D).to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="pooling"):
        impl.forward(_layer(), q, k, v, _cache(), md, torch.zeros_like(q))


def test_prefill_calibrates_once_writes_pages_and_attends_raw_kv(cpu_ops):
    impl = _Impl()
    layer = _layer()
    cache = _cache()
    lens = [5, 11]
    t = sum(lens)
    k, v = make_kv(t + 3, KVH, D, dtype=torch.bfloat16, seed=1)  # 3 padding rows
    q = torch.randn(t + 3, HQ, D).to(torch.bfloat16)
    table = torch.tensor([[3, 0], [7, 5]])
    slots = [int(table[b, p // BS]) * BS + p % BS for b, n in enumerate(lens) for p in range(n)]
    md = _md("PrefillNoCache", slot_mapping=torch.tensor(slots + [-1] * 3),
             num_actual_tokens=t, actual_seq_lengths_q=[5, t], seq_lens_list=lens,
             block_tables=table)
    out = torch.zeros(t + 3, HQ, D, dtype=torch.bfloat16)
    impl.forward(layer, q, k, v, cache, md, out)
    # scales come from the whole first K/V, padding rows included
    k_inv, v_inv, _, _ = ref.int8_calc_scales(k, v)
    assert torch.equal(layer._int8_k_inv_scale, k_inv) and layer._int8_scales_ready
    want_k = torch.zeros(NB, BS, KVH, D, dtype=torch.int8)
    ref.int8_reshape_and_cache(k[:t], v[:t], k_inv, v_inv, torch.tensor(slots), want_k,
                               torch.zeros_like(want_k))
    assert torch.equal(cache[0], want_k)
    assert cpu_ops["dense"] == [(lens, lens)]
    want = ref.attention(q[:t], k[:t], v[:t], lens, lens, D ** -0.5, True)
    torch.testing.assert_close(out[:t].float(), want, atol=1e-2, rtol=1e-2)
    # a second forward does not recalibrate
    impl.forward(layer, q, k * 4, v, cache, md, out)
    assert torch.equal(layer._int8_k_inv_scale, k_inv)


def test_decode_and_cache_hit_prefill_read_the_int8_pages(cpu_ops):
    impl = _Impl()
    layer = _layer()
    cache = _cache()
    n = 20
    k, v = make_kv(n, KVH, D, dtype=torch.bfloat16, seed=2)
    table = torch.tensor([[4, 9, 1]])
    slots = torch.tensor([int(table[0, p // BS]) * BS + p % BS for p in range(n)])
    md = _md("PrefillNoCache", slot_mapping=slots[:n - 1], num_actual_tokens=n - 1,
             actual_seq_lengths_q=[n - 1], seq_lens_list=[n - 1], block_tables=table)
    q = torch.randn(n, HQ, D).to(torch.bfloat16)
    impl.forward(layer, q, k[:n - 1], v[:n - 1], cache, md, torch.zeros_like(q))
    # decode one token: written first, then attended through the pages
    md = _md("DecodeOnly", slot_mapping=slots[n - 1:], num_actual_tokens=1,
             seq_lens_list=[n], block_tables=table)
    out = torch.zeros(1, HQ, D, dtype=torch.bfloat16)
    impl.forward(layer, q[:1], k[n - 1:], v[n - 1:], cache, md, out)
    assert cpu_ops["decode"] == [[n]]
    dk, dv = ref.int8_paged_dequant(cache[0], cache[1], table, [n], torch.bfloat16,
                                    layer._int8_k_inv_scale, layer._int8_v_inv_scale)
    want = ref.attention(q[:1], dk, dv, [1], [n], D ** -0.5, True)
    torch.testing.assert_close(out.float(), want, atol=1e-2, rtol=1e-2)
    # the quantization is visible: attention over the raw K/V differs
    exact = ref.attention(q[:1], k, v, [1], [n], D ** -0.5, True)
    assert (want - exact).abs().max() > 1e-4
    # a cache-hit prefill dequantizes the pages to dense TND first
    md = _md("PrefillCacheHit", actual_seq_lengths_q=[4], seq_lens_list=[n],
             block_tables=table)
    out4 = torch.zeros(4, HQ, D, dtype=torch.bfloat16)
    impl.forward(layer, q[:4], None, None, cache, md, out4)
    assert cpu_ops["dequant"][-1] == [n] and cpu_ops["dense"][-1] == ([4], [n])


def test_chunked_prefill_splits_decode_rows_and_history_aware_prompts(cpu_ops):
    impl = _Impl()
    layer = _layer()
    cache = _cache()
    k, v = make_kv(40, KVH, D, dtype=torch.bfloat16, seed=3)
    q = torch.randn(40, HQ, D).to(torch.bfloat16)
    impl._prepare_int8_scales(layer, k, v)
    table = torch.tensor([[0, 1, 2], [3, 4, 5]])
    # decode row (seq 9) + prompt row with 6 tokens of history plus a 4-token chunk
    md = _md("ChunkedPrefill", num_decode_tokens=1, num_decodes=1, num_prefills=1,
             actual_seq_lengths_q=[1, 5], seq_lens_list=[9, 10], block_tables=table,
             slot_mapping=torch.tensor([8, 3 * BS + 6, 3 * BS + 7, 4 * BS, 4 * BS + 1]),
             num_actual_tokens=5)
    out = torch.zeros(5, HQ, D, dtype=torch.bfloat16)
    impl.forward(layer, q[:5], k[:5], v[:5], cache, md, out)
    assert cpu_ops["decode"] == [[9]]
    assert cpu_ops["dequant"][-1] == [10]  # history-aware prompt reads the pages
    assert cpu_ops["dense"][-1] == ([4], [10])
    # all-new prompt rows attend their own float K/V
    md.seq_lens_list = [9, 4]
    impl.forward(layer, q[:5], k[:5], v[:5], cache, md, out)
    assert cpu_ops["dense"][-1] == ([4], [4])
    want = ref.attention(q[1:5], k[1:5], v[1:5], [4], [4], D ** -0.5, True)
    torch.testing.assert_close(out[1:5].float(), want, atol=1e-2, rtol=1e-2)


def test_int8_split_fills_one_round_of_workgroups():
    """The INT8 decode split: one item per CU for up to 8 KV heads (config 2:
    64 x 4096 tokens -> 1024-position items, 256 of them), more waves per CU
    with more heads, and per-request cuts that never overflow one round."""
    from vllm_ascend_quantized_kv_cache.ops.int8_ops import int8_split_tokens

    assert int8_split_tokens(64 * 4096, 8, seq_lens=[4096] * 64) == 1024
    assert int8_split_tokens(64 * 4096, 8) == 1024
    assert int8_split_tokens(64 * 4096, 16) == 4096  # one wave per head: 4 per CU
    gen = torch.Generator().manual_seed(3)
    for trial in range(200):
        b = int(torch.randint(1, 300, (1,), generator=gen))
        lens = torch.randint(1, 20000, (b,), generator=gen).tolist()
        kvh = [1, 2, 4, 8][trial % 4]
        target = 256 * 8 // kvh
        split = int8_split_tokens(sum(lens), kvh, seq_lens=lens)
        assert split % 128 == 0 and 256 <= split <= 4096
        items = sum(-(-n // split) for n in lens)
        # within one round unless even 4096-position items cannot make it
        assert items <= target or split == 4096
        # and no longer than needed: one step down would overflow (or is the floor)
        if split > max(256, -(-(-(-sum(lens) // target)) // 128) * 128):
            assert sum(-(-n // (split - 128)) for n in lens) > target


def _capturing(monkeypatch):
    from vllm_ascend_quantized_kv_cache.methods.int8_dynamic import attention_backend as i8ab

    monkeypatch.setattr(i8ab, "stream_capturing", lambda: True)


def test_forward_under_capture_without_graph_is_refused(cpu_ops, monkeypatch):
    """A captured forward() would record one step's staged plan and replay it
    forever; with no capturable step created for the batch it raises before
    anything is written or launched (``i8ab.py:97-104`` routes capture to the
    host's graph path instead)."""
    impl = _Impl()
    layer = _layer()
    cache = _cache()
    k, v = make_kv(2, KVH, D, dtype=torch.bfloat16, seed=3)
    md = _md("DecodeOnly", seq_lens_list=[3, 5], block_tables=torch.tensor([[0], [1]]),
             slot_mapping=torch.tensor([2, 12]), num_actual_tokens=2)
    q = torch.randn(2, HQ, D).to(torch.bfloat16)
    _capturing(monkeypatch)
    for state in ("DecodeOnly", "ChunkedPrefill", "PrefillNoCache"):
        md.attn_state = SimpleNamespace(name=state)
        with pytest.raises(RuntimeError, match="graph capture"):
            impl.forward(layer, q, k, v, cache, md, torch.zeros_like(q))
    assert not cache.any() and not getattr(layer, "_int8_scales_ready", False)
    assert cpu_ops == {"decode": [], "dense": [], "dequant": []}


def test_forward_under_capture_routes_decode_to_the_batch_graph(cpu_ops, monkeypatch):
    impl = _Impl()
    launched = []

    class _Graph:
        def launch(self, query, key, value, output):
            launched.append(query.shape[0])
            return output

    impl._int8_capture_graphs = {2: _Graph()}
    md = _md("DecodeOnly", seq_lens_list=[3, 5], block_tables=torch.tensor([[0], [1]]))
    q = torch.randn(2, HQ, D)
    out = torch.zeros_like(q)
    _capturing(monkeypatch)
    assert impl.forward(_layer(), q, None, None, _cache(), md, out) is out
    assert launched == [2]
    md.seq_lens_list = [3, 5, 7]  # no capturable step for batch 3
    with pytest.raises(RuntimeError, match="batch-3"):
        impl.forward(_layer(), torch.randn(3, HQ, D), None, None, _cache(), md,
                     torch.zeros(3, HQ, D))
    with pytest.raises(RuntimeError, match="no capturable step for batch 3"):
        impl.prepare_int8_graph_replay(md)
