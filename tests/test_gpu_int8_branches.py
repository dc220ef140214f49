# SPDX-License-Identifier: Apache-2.0
"""INT8 mixin branches on the GPU against the oracle.

* ``ChunkedPrefill`` with decode rows plus an all-new prompt (the prompt
  attends to its own bf16 K/V), and with decode rows plus a prompt that
  continues a cached prefix (the prompt attends to the dequantized pages);
* the fall-through prefill over a cached prefix (``PrefillCacheHit``);
* the planned decode step (one pinned plan, quantize + scatter and decode
  reading it) equal, bit for bit, to the op path; and the same step captured
  once in a HIP graph and replayed for many steps, equal to an eager twin
  and to the oracle (``pkg/methods/int8_dynamic/attention_backend.py:97-104,
  173-404``).

Oracle: int8 pages from ``int8_reshape_and_cache`` with the first K/V's
scales; the decode rows and steps are FIA's per-channel antiquant (fp32
product with the bf16 ``aq``), the prefill branches dequantize to the
activation dtype first, then fp32 attention.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import kvq_oracle as ref
from vllm_ascend_quantized_kv_cache.methods.int8_dynamic.attention_backend import (
    AscendInt8AttentionBackendMixin,
)

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-2, rtol=1e-2)
HQ, KVH, D, BS = 32, 8, 128, 128


def _impl():
    class Impl(AscendInt8AttentionBackendMixin):
        num_heads, num_kv_heads, head_size, scale = HQ, KVH, D, D ** -0.5

    return Impl(), SimpleNamespace(_k_scale_float=1.0, _v_scale_float=1.0)


class _Pool:
    """Requests' block tables, seeded K/V, and the oracle's int8 pages."""

    def __init__(self, nb, seed):
        self.gen = torch.Generator().manual_seed(seed)
        self.nb = nb
        self.perm = torch.randperm(nb, generator=self.gen).tolist()
        self.tables = {}
        self.scales = torch.exp(torch.randn(KVH, D, generator=self.gen))
        self.want = torch.zeros(2, nb, BS, KVH, D, dtype=torch.int8)

    def table(self, req, n_blocks):
        t = self.tables.setdefault(req, [])
        while len(t) < n_blocks:
            t.append(self.perm.pop())
        return t

    def slots(self, req, p0, p1):
        t = self.table(req, -(-p1 // BS))
        return [t[p // BS] * BS + p % BS for p in range(p0, p1)]

    def kv(self, n):
        k = (torch.randn(n, KVH, D, generator=self.gen) * self.scales).to(torch.bfloat16)
        return k, torch.randn(n, KVH, D, generator=self.gen).to(torch.bfloat16)

    def q(self, n):
        return torch.randn(n, HQ, D, generator=self.gen).to(torch.bfloat16)

    def block_tables(self, reqs, width):
        rows = [self.tables[r] + [0] * (width - len(self.tables[r])) for r in reqs]
        return torch.tensor(rows, dtype=torch.int64)


def _md(state, dev, **kw):
    md = SimpleNamespace(attn_state=SimpleNamespace(name=state), model_runner_type="generate",
                         causal=True, **kw)
    for name in ("slot_mapping", "block_tables"):
        if hasattr(md, name):
            setattr(md, name + "_cpu", getattr(md, name))
            setattr(md, name, getattr(md, name).to(dev))
    return md


def _dequant(pool, reqs, lens, dtype, inv):
    table = pool.block_tables(reqs, max(-(-n // BS) for n in lens))
    return ref.int8_paged_dequant(pool.want[0], pool.want[1], table, lens, dtype, inv[0], inv[1])


def test_int8_chunked_prefill_and_cache_hit_branches_match_oracle(gpu_device):
    dev = gpu_device
    pool = _Pool(96, seed=31)
    impl, layer = _impl()
    cache = torch.zeros(2, pool.nb, BS, KVH, D, dtype=torch.int8, device=dev)

    def write(k, v, slots, inv):
        ref.int8_reshape_and_cache(k, v, inv[0], inv[1], torch.tensor(slots), pool.want[0],
                                   pool.want[1])

    # 1. PrefillNoCache: a, b (decode rows later) and c (a prefix continued later)
    lens = {"a": 300, "b": 129, "c": 700}
    reqs = list(lens)
    kvs = {r: pool.kv(n) for r, n in lens.items()}
    k = torch.cat([kvs[r][0] for r in reqs])
    v = torch.cat([kvs[r][1] for r in reqs])
    slots = sum((pool.slots(r, 0, lens[r]) for r in reqs), [])
    q = pool.q(k.shape[0])
    cu = [300, 429, 1129]
    out = torch.zeros(k.shape[0], HQ, D, dtype=torch.bfloat16, device=dev)
    impl.forward(layer, q.to(dev), k.to(dev), v.to(dev), cache,
                 _md("PrefillNoCache", dev, slot_mapping=torch.tensor(slots),
                     num_actual_tokens=k.shape[0], actual_seq_lengths_q=cu,
                     seq_lens_list=list(lens.values()),
                     block_tables=pool.block_tables(reqs, 6)), out)
    inv = ref.int8_calc_scales(k, v)[:2]
    write(k, v, slots, inv)
    assert torch.equal(cache.cpu(), pool.want)

    def check_rows(out, rows, q, kk, vv, q_lens, kv_lens):
        want = ref.attention(q, kk, vv, q_lens, kv_lens, D ** -0.5, True)
        torch.testing.assert_close(out[rows].float().cpu(), want, **TOL)

    # 2. ChunkedPrefill: decode rows a, b + an all-new prompt d (37 tokens)
    for state_prompt, prompt, p0, n_new in (("all-new", "d", 0, 37), ("history", "c", 700, 200)):
        dec = ["a", "b"]
        kd, vd = pool.kv(2)
        kp, vp = pool.kv(n_new)
        dslots = [pool.slots(r, lens[r], lens[r] + 1)[0] for r in dec]
        pslots = pool.slots(prompt, p0, p0 + n_new)
        for r in dec:
            lens[r] += 1
        lens[prompt] = p0 + n_new
        order = dec + [prompt]
        qq = pool.q(2 + n_new)
        md = _md("ChunkedPrefill", dev, slot_mapping=torch.tensor(dslots + pslots),
                 num_actual_tokens=2 + n_new, actual_seq_lengths_q=[1, 2, 2 + n_new],
                 seq_lens_list=[lens[r] for r in order], num_decodes=2, num_decode_tokens=2,
                 num_prefills=1, block_tables=pool.block_tables(order, 8))
        out = torch.zeros(2 + n_new, HQ, D, dtype=torch.bfloat16, device=dev)
        impl.forward(layer, qq.to(dev), torch.cat([kd, kp]).to(dev),
                     torch.cat([vd, vp]).to(dev), cache, md, out)
        write(torch.cat([kd, kp]), torch.cat([vd, vp]), dslots + pslots, inv)
        torch.cuda.synchronize()
        assert torch.equal(cache.cpu(), pool.want), state_prompt
        dk, dv = _dequant(pool, dec, [lens[r] for r in dec], torch.float32, inv)
        check_rows(out, slice(0, 2), qq[:2], dk, dv, [1, 1], [lens[r] for r in dec])
        if state_prompt == "all-new":  # its own bf16 K/V
            check_rows(out, slice(2, None), qq[2:], kp, vp, [n_new], [n_new])
        else:  # the dequantized pages (activation dtype) of prefix + chunk
            pk, pv = _dequant(pool, [prompt], [lens[prompt]], torch.bfloat16, inv)
            check_rows(out, slice(2, None), qq[2:], pk, pv, [n_new], [lens[prompt]])

    # 3. PrefillCacheHit (fall-through prefill): d continues with 50 tokens
    kh, vh = pool.kv(50)
    hslots = pool.slots("d", 37, 87)
    lens["d"] = 87
    qh = pool.q(50)
    out = torch.zeros(50, HQ, D, dtype=torch.bfloat16, device=dev)
    impl.forward(layer, qh.to(dev), kh.to(dev), vh.to(dev), cache,
                 _md("PrefillCacheHit", dev, slot_mapping=torch.tensor(hslots),
                     num_actual_tokens=50, actual_seq_lengths_q=[50], seq_lens_list=[87],
                     block_tables=pool.block_tables(["d"], 1)), out)
    write(kh, vh, hslots, inv)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), pool.want)
    pk, pv = _dequant(pool, ["d"], [87], torch.bfloat16, inv)
    check_rows(out, slice(0, None), qh, pk, pv, [50], [87])


class _DecodeCase:
    """A calibrated INT8 layer with prefilled requests, on one pool."""

    def __init__(self, dev, b=16, seed=41, steps=0):
        self.dev = dev
        self.pool = _Pool(b * (20 + 1), seed)
        gen = torch.Generator().manual_seed(seed)
        self.lens = torch.randint(300, 2400, (b,), generator=gen).tolist()
        self.reqs = [f"r{i}" for i in range(b)]
        self.kvs = {r: self.pool.kv(n + steps) for r, n in zip(self.reqs, self.lens)}
        self.qs = self.pool.q(b * max(1, steps)).view(max(1, steps), b, HQ, D)
        for r, n in zip(self.reqs, self.lens):
            self.pool.slots(r, 0, n + steps)
        self.width = max(len(t) for t in self.pool.tables.values())
        self.table = self.pool.block_tables(self.reqs, self.width)

    def build(self):
        impl, layer = _impl()
        cache = torch.zeros(2, self.pool.nb, BS, KVH, D, dtype=torch.int8, device=self.dev)
        k = torch.cat([self.kvs[r][0][:n] for r, n in zip(self.reqs, self.lens)])
        v = torch.cat([self.kvs[r][1][:n] for r, n in zip(self.reqs, self.lens)])
        slots = sum((self.pool.slots(r, 0, n) for r, n in zip(self.reqs, self.lens)), [])
        cu = torch.tensor(self.lens).cumsum(0).tolist()
        out = torch.zeros(k.shape[0], HQ, D, dtype=torch.bfloat16, device=self.dev)
        impl.forward(layer, torch.zeros_like(out), k.to(self.dev), v.to(self.dev), cache,
                     _md("PrefillNoCache", self.dev, slot_mapping=torch.tensor(slots),
                         num_actual_tokens=k.shape[0], actual_seq_lengths_q=cu,
                         seq_lens_list=list(self.lens), block_tables=self.table), out)
        return impl, layer, cache

    def step(self, j):
        pos = [n + j for n in self.lens]
        slots = [self.pool.slots(r, p, p + 1)[0] for r, p in zip(self.reqs, pos)]
        k = torch.stack([self.kvs[r][0][p] for r, p in zip(self.reqs, pos)])
        v = torch.stack([self.kvs[r][1][p] for r, p in zip(self.reqs, pos)])
        md = _md("DecodeOnly", self.dev, slot_mapping=torch.tensor(slots),
                 num_actual_tokens=len(pos), seq_lens_list=[p + 1 for p in pos],
                 block_tables=self.table)
        return md, self.qs[j].to(self.dev), k.to(self.dev), v.to(self.dev)

    def oracle(self, layer, cache, j, out):
        lens = [n + j + 1 for n in self.lens]
        inv = (layer._int8_k_inv_scale.cpu(), layer._int8_v_inv_scale.cpu())
        dk, dv = ref.int8_paged_dequant(cache[0].cpu(), cache[1].cpu(), self.table, lens,
                                        torch.float32, inv[0], inv[1])
        want = ref.attention(self.qs[j], dk, dv, [1] * len(lens), lens, D ** -0.5, True)
        torch.testing.assert_close(out.float().cpu(), want, **TOL)


def test_int8_planned_decode_step_equals_op_path(gpu_device):
    case = _DecodeCase(gpu_device, steps=6)
    (a, la, ca), (b, lb, cb) = case.build(), case.build()
    b._int8_step_enabled = lambda query: False  # the op path
    for j in range(6):
        md, q, k, v = case.step(j)
        outs = []
        for impl, layer, cache in ((a, la, ca), (b, lb, cb)):
            out = torch.zeros_like(q)
            impl.forward(layer, q, k, v, cache, md, out)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(ca, cb) and torch.equal(outs[0], outs[1]), f"step {j}"
    case.oracle(la, ca, 5, outs[0])
    assert getattr(a, "int8_host_reads", 0) == 0 and a._int8_step_bufs is not None


def test_int8_decode_graph_replays_match_eager_twin_and_oracle(gpu_device):
    steps = 24
    case = _DecodeCase(gpu_device, steps=steps, seed=43)
    (g, lg, cg), (e, le, ce) = case.build(), case.build()
    gstep = g.int8_decode_graph(lg, len(case.reqs), max_blocks=case.width)
    q_s = torch.zeros(len(case.reqs), HQ, D, dtype=torch.bfloat16, device=gpu_device)
    k_s = torch.zeros(len(case.reqs), KVH, D, dtype=torch.bfloat16, device=gpu_device)
    v_s = torch.zeros_like(k_s)
    out_s = torch.zeros_like(q_s)
    graph = None
    for j in range(steps):
        md, q, k, v = case.step(j)
        q_s.copy_(q)
        k_s.copy_(k)
        v_s.copy_(v)
        g.prepare_int8_graph_replay(md)  # the host's per-replay hook (gstep.prepare)
        if graph is None:
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                # the host records forward() itself: under capture it routes
                # the decode to the batch's capturable step
                g.forward(lg, q_s, k_s, v_s, cg, md, out_s)
        graph.replay()
        out = torch.zeros_like(q_s)
        e.forward(le, q, k, v, ce, md, out)
        torch.cuda.synchronize()
        assert torch.equal(cg, ce), f"replay {j}: int8 pages differ from the eager step"
        torch.testing.assert_close(out_s, out, atol=0, rtol=0)
        if j in (0, steps - 1):
            case.oracle(lg, cg, j, out_s)
    assert getattr(g, "int8_host_reads", 0) == 0
    assert g._int8_capture_graphs == {len(case.reqs): gstep}
