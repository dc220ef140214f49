# SPDX-License-Identifier: Apache-2.0
"""The planned KIVI decode step on the GPU: sync-free, and capturable.

* ``forward(DecodeOnly)`` through the planned step (one pinned plan, the
  planned store, the fused decode) leaves the same int4 pages and rings as
  the general path (per-request planning, the one-launch store) and gives
  the same output, over steps that flush key windows and evict values;
* with the host's copies of ``slot_mapping`` and ``block_tables`` in the
  metadata, a step reads nothing back from the device;
* the step's two launches captured once in a HIP graph, replayed over many
  steps (each after the host stages that step's plan), match an eager twin
  bit for bit and the oracle's fp32 attention over the reference dequant.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from oracle import kvq_oracle as ref
from tests._cpu_kernels import windows_from_meta
from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import attention_backend as ab
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.byte_cache import KiviByteCacheLayout

pytestmark = pytest.mark.gpu

TOL = dict(atol=1e-2, rtol=1e-2)


def _impl(device, *, hq, kvh, d, g, r, nb, bs, rows, general=False):
    class Impl(ab.AscendKiviInt4AttentionBackendMixin):
        pass

    impl = Impl()
    impl.num_heads, impl.num_kv_heads, impl.head_size, impl.scale = hq, kvh, d, d ** -0.5
    impl._init_kivi_state(None)
    impl.enable_kivi = True
    impl.kivi_group_size, impl.kivi_residual_length, impl.kivi_max_num_seqs = g, r, rows
    layout = KiviByteCacheLayout(nb, bs, kvh, d, g)
    kbuf = torch.zeros((nb, bs, kvh, layout.bytes_per_token_head), dtype=torch.uint8,
                       device=device)
    impl._bind_kivi_cache((kbuf, torch.zeros_like(kbuf)))
    if general:
        # the same GPU launch, installed as an instance hook: the planned step
        # stands aside and forward takes the general path
        impl._launch_kivi_decode = impl._launch_kivi_decode
    return impl


class _Case:
    """Requests with int4 history and windows, identical on every impl built."""

    def __init__(self, device, *, b=6, hq=40, kvh=8, d=128, g=128, r=128, bs=128, steps=140,
                 seed=0, data_seed=None):
        gen = torch.Generator().manual_seed(seed)
        self.device, self.b, self.hq, self.kvh, self.d, self.g, self.r, self.bs = (
            device, b, hq, kvh, d, g, r, bs)
        self.lens = torch.randint(200, 1500, (b,), generator=gen).tolist()
        nblk = [-(-(n + steps + 1) // bs) for n in self.lens]
        self.nb = sum(nblk) + 4
        perm = torch.randperm(self.nb, generator=gen)
        self.table = torch.zeros((b, max(nblk)), dtype=torch.int64)
        used = 0
        for i, n in enumerate(nblk):
            self.table[i, :n] = perm[used:used + n]
            used += n
        self.table_dev = self.table.to(device)
        if data_seed is not None:  # same geometry and slots, other keys, values, queries
            gen = torch.Generator().manual_seed(data_seed)
        scales = torch.exp(torch.randn((kvh, d), generator=gen))
        self.keys = [(torch.randn(n + steps, kvh, d, generator=gen) * scales).to(torch.bfloat16)
                     for n in self.lens]
        self.values = [torch.randn(n + steps, kvh, d, generator=gen).to(torch.bfloat16)
                       for n in self.lens]
        self.queries = torch.randn(steps, b, hq, d, generator=gen).to(torch.bfloat16)
        self.reqs = [f"r{i}" for i in range(b)]

    def slot(self, i, p):
        return int(self.table[i, p // self.bs]) * self.bs + p % self.bs

    def build(self, *, reverse=False, **kw):
        """An impl holding the requests' history (``reverse``: registered last
        to first, so each request gets another residual row)."""
        impl = _impl(self.device, hq=self.hq, kvh=self.kvh, d=self.d, g=self.g, r=self.r,
                     nb=self.nb, bs=self.bs, rows=self.b, **kw)
        order = list(enumerate(self.lens))
        for i, n in (order[::-1] if reverse else order):
            sl = torch.tensor([self.slot(i, p) for p in range(n)], device=self.device)
            impl._write_kivi_cache(self.keys[i][:n].to(self.device),
                                   self.values[i][:n].to(self.device), sl, [self.reqs[i]], [n],
                                   [n])
        return impl

    def step(self, j, *, host_copies=True):
        """(metadata, q, k, v) of decode step j (each request gains token n + j)."""
        pos = [n + j for n in self.lens]
        sm = torch.tensor([self.slot(i, p) for i, p in enumerate(pos)])
        md = SimpleNamespace(attn_state=SimpleNamespace(name="DecodeOnly"), causal=True,
                             finished_req_ids=None, seq_lens_list=[p + 1 for p in pos],
                             slot_mapping=sm.to(self.device), block_tables=self.table_dev,
                             req_ids=self.reqs, num_actual_tokens=self.b)
        if host_copies:
            md.slot_mapping_cpu = sm
            md.block_tables_cpu = self.table
        k = torch.stack([self.keys[i][p] for i, p in enumerate(pos)]).to(self.device)
        v = torch.stack([self.values[i][p] for i, p in enumerate(pos)]).to(self.device)
        return md, self.queries[j].to(self.device), k, v

    def oracle(self, impl, j, out):
        """The oracle's attention for step j from the GPU state after it."""
        caches = tuple(t.cpu() for t in impl._kivi_caches())
        lens = [n + j + 1 for n in self.lens]
        meta = impl._ring_meta_rows(lens, self.reqs)
        ring = impl._kivi_ring
        cpu_ring = SimpleNamespace(_kivi_ring=SimpleNamespace(
            key=ring.key.cpu(), value=ring.value.cpu(), ring_len=ring.ring_len))
        wk, wv = windows_from_meta(cpu_ring, meta, lens)
        dk, dv = ref.dequant_gather(*caches, self.table, torch.tensor(lens), torch.float32,
                                    self.g)
        dk = ref.overlay_residual(dk, lens, wk)
        dv = ref.overlay_residual(dv, lens, wv)
        want = ref.attention(self.queries[j], dk, dv, [1] * self.b, lens, self.d ** -0.5, True)
        torch.testing.assert_close(out.float().cpu(), want, **TOL)


def _same_state(a, b):
    for x, y in zip(a._kivi_caches(), b._kivi_caches()):
        assert torch.equal(x, y), "int4 pages differ"
    ra, rb = a._kivi_ring, b._kivi_ring
    assert ra.state() == rb.state()
    assert torch.equal(ra.key, rb.key) and torch.equal(ra.value, rb.value)


@pytest.mark.parametrize("g", [128, 64])
def test_planned_decode_step_equals_general_path(gpu_device, g):
    case = _Case(gpu_device, g=g, r=128, steps=135, seed=1 if g == 128 else 2)
    fast, general = case.build(), case.build(general=True)
    for j in range(135):  # a key window flushes for every request
        outs = []
        for impl in (fast, general):
            md, q, k, v = case.step(j)
            out = torch.zeros((case.b, case.hq, case.d), dtype=torch.bfloat16, device=gpu_device)
            impl.forward(None, q, k, v, None, md, out)
            outs.append(out)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), f"step {j}"
        if j % 45 == 0 or j == 134:
            _same_state(fast, general)
            case.oracle(fast, j, outs[0])
    assert fast._kivi_step_bufs is not None and general._kivi_step_bufs is None
    assert fast.kivi_host_reads == 0


def test_layers_share_one_planned_step(gpu_device, monkeypatch):
    """Layers called with one metadata object per engine step: the first
    plans and stages the step, the others whose window mirror matches take
    its plan and launch against their own caches.  Each layer has its own
    keys, values and queries; its output equals, bit for bit, a lone twin's
    that plans every step itself, over steps that flush key windows, and the
    oracle's.  A layer whose requests sit in other residual rows (a mirror
    that differs) plans on its own within the same steps."""
    steps = 135
    cases = [_Case(gpu_device, steps=steps, seed=5, data_seed=100 + i) for i in range(3)]
    layers = [c.build() for c in cases[:2]] + [cases[2].build(reverse=True)]
    twins = [c.build() for c in cases[:2]] + [cases[2].build(reverse=True)]
    replayed = []
    orig = ab.AscendKiviInt4AttentionBackendMixin._replay_shared_kivi_step

    def counting(self, *a, **k):
        replayed.append(self)
        return orig(self, *a, **k)

    monkeypatch.setattr(ab.AscendKiviInt4AttentionBackendMixin, "_replay_shared_kivi_step",
                        counting)
    for j in range(steps):
        steps_j = [c.step(j) for c in cases]
        md = steps_j[0][0]  # one metadata object for the engine step
        outs, want = [], []
        for impl, (_, q, k, v) in zip(layers, steps_j):
            out = torch.zeros((cases[0].b, cases[0].hq, cases[0].d), dtype=torch.bfloat16,
                              device=gpu_device)
            impl.forward(None, q, k, v, None, md, out)
            outs.append(out)
        for twin, c in zip(twins, cases):
            own_md, q, k, v = c.step(j)  # a metadata object of its own: plans alone
            out = torch.zeros_like(outs[0])
            twin.forward(None, q, k, v, None, own_md, out)
            want.append(out)
        torch.cuda.synchronize()
        for li in range(3):
            assert torch.equal(outs[li], want[li]), f"step {j} layer {li}"
        if j % 45 == 0 or j == steps - 1:
            for li in range(3):
                _same_state(layers[li], twins[li])
                cases[li].oracle(layers[li], j, outs[li])
    # layer 1 reused layer 0's plan every step; layer 2 (other rows) never did
    assert replayed == [layers[1]] * steps
    assert layers[1]._kivi_step_bufs is None and layers[2]._kivi_step_bufs is not None


def test_layer_graphs_share_one_planned_step(gpu_device, monkeypatch):
    """Each layer's step captured once; per engine step every layer's
    ``prepare`` sees the same metadata object.  The first layer plans and
    stages, the next takes that plan with one copy (its mirror matches), a
    layer whose requests sit in other rows plans on its own.  Every replay
    equals an eager twin bit for bit, over steps that flush key windows."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import decode_step as dstep

    steps = 131
    cases = [_Case(gpu_device, steps=steps, seed=8, data_seed=200 + i) for i in range(3)]
    layers = [c.build() for c in cases[:2]] + [cases[2].build(reverse=True)]
    twins = [c.build() for c in cases[:2]] + [cases[2].build(reverse=True)]
    copied = []
    orig = dstep.DecodeStepBuffers.copy_staged_from

    def counting(self, *a, **k):
        copied.append(self)
        return orig(self, *a, **k)

    monkeypatch.setattr(dstep.DecodeStepBuffers, "copy_staged_from", counting)
    c0 = cases[0]
    gsteps = [impl.kivi_decode_graph(c0.b, max_blocks=c0.table.shape[1]) for impl in layers]
    statics = [tuple(torch.zeros(shape, dtype=torch.bfloat16, device=gpu_device)
                     for shape in ((c0.b, c0.hq, c0.d), (c0.b, c0.kvh, c0.d),
                                   (c0.b, c0.kvh, c0.d), (c0.b, c0.hq, c0.d)))
               for _ in layers]
    graphs = [None] * 3
    for j in range(steps):
        steps_j = [c.step(j) for c in cases]
        md = steps_j[0][0]
        for li, impl in enumerate(layers):
            q_s, k_s, v_s, out_s = statics[li]
            _, q, k, v = steps_j[li]
            q_s.copy_(q)
            k_s.copy_(k)
            v_s.copy_(v)
            impl.prepare_kivi_graph_replay(md, k_s, v_s)
            if graphs[li] is None:
                torch.cuda.synchronize()
                graphs[li] = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graphs[li]):
                    impl.forward(None, q_s, k_s, v_s, None, md, out_s)
            graphs[li].replay()
        want = []
        for twin, c in zip(twins, cases):
            own_md, q, k, v = c.step(j)
            out = torch.zeros_like(statics[0][0])
            twin.forward(None, q, k, v, None, own_md, out)
            want.append(out)
        torch.cuda.synchronize()
        for li in range(3):
            assert torch.equal(statics[li][3], want[li]), f"replay {j} layer {li}"
        if j in (0, 64, steps - 1):
            for li in range(3):
                _same_state(layers[li], twins[li])
    assert copied == [gsteps[1].bufs] * steps


def test_planned_decode_step_reads_nothing_back(gpu_device):
    case = _Case(gpu_device, steps=4, seed=3)
    impl = case.build()
    md, q, k, v = case.step(0)
    out = torch.zeros((case.b, case.hq, case.d), dtype=torch.bfloat16, device=gpu_device)
    impl.forward(None, q, k, v, None, md, out)  # first call sizes the buffers
    # the steps' metadata and inputs, built (and copied to the device) by the
    # host runner before the steps run
    steps = [case.step(j) for j in (1, 2)]
    torch.cuda.synchronize()
    probe = torch.ones(4, device=gpu_device)
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        try:
            probe.cpu()
            detects = False
        except RuntimeError:
            detects = True
        for md, q, k, v in steps:
            impl.forward(None, q, k, v, None, md, out)
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    torch.cuda.synchronize()
    assert impl.kivi_host_reads == 0
    case.oracle(impl, 2, out)
    if not detects:
        pytest.skip("this torch build does not flag synchronising calls; host reads counted only")
    # without host copies the mixin reads the two tensors back, once each
    md, q, k, v = case.step(3, host_copies=False)
    impl.forward(None, q, k, v, None, md, out)
    assert impl.kivi_host_reads == 2


def test_decode_step_graph_replays_match_eager_twin_and_oracle(gpu_device):
    """Capture store + decode + combine once; replay it for 131 steps (key
    windows flush inside replays), each step's plan staged by the host
    between replays, with the program's own eager work in between."""
    steps = 131
    case = _Case(gpu_device, steps=steps, seed=4)
    graphed, eager = case.build(), case.build()
    gstep = graphed.kivi_decode_graph(case.b, max_blocks=case.table.shape[1])
    q_s = torch.zeros((case.b, case.hq, case.d), dtype=torch.bfloat16, device=gpu_device)
    k_s = torch.zeros((case.b, case.kvh, case.d), dtype=torch.bfloat16, device=gpu_device)
    v_s = torch.zeros_like(k_s)
    out_s = torch.zeros_like(q_s)
    graph = None
    for j in range(steps):
        md, q, k, v = case.step(j)
        q_s.copy_(q)
        k_s.copy_(k)
        v_s.copy_(v)
        graphed.prepare_kivi_graph_replay(md, k_s, v_s)  # the host's per-replay hook
        if graph is None:
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                # the host records forward() itself: under capture it routes
                # the decode to the batch's capturable step
                graphed.forward(None, q_s, k_s, v_s, None, md, out_s)
        graph.replay()
        out = torch.zeros_like(q_s)
        eager.forward(None, q, k, v, None, md, out)
        torch.cuda.synchronize()
        assert torch.equal(out_s, out), f"replay {j} differs from the eager step"
        if j in (0, 1, 64, steps - 1):
            _same_state(graphed, eager)
            case.oracle(graphed, j, out_s)
    assert graphed.kivi_host_reads == 0
    assert graphed._kivi_capture_graphs == {case.b: gstep}


def test_decode_graph_prepare_refuses_before_the_mirror_moves(gpu_device):
    """Every check of ``KiviDecodeGraph.prepare`` that can refuse a step runs
    before the window mirror moves: a batch other than the captured one, a
    wider block table, or an activation dtype the planned store does not
    cover.  The mirror (and so the device pages) stay as they were."""
    case = _Case(gpu_device, b=4, steps=3, seed=6)
    impl = case.build()
    gstep = impl.kivi_decode_graph(case.b + 1, max_blocks=case.table.shape[1])
    ring = impl._kivi_ring
    before = ring.state()
    md, q, k, v = case.step(0)
    with pytest.raises(RuntimeError, match="captured for batch"):
        gstep.prepare(md, k, v)
    assert ring.state() == before
    narrow = impl.kivi_decode_graph(case.b, max_blocks=case.table.shape[1] - 1)
    with pytest.raises(RuntimeError, match="wider than captured"):
        narrow.prepare(md, k, v)
    assert ring.state() == before
    with pytest.raises(RuntimeError, match="geometry or activation dtype"):
        impl.kivi_decode_graph(case.b, max_blocks=case.table.shape[1]).prepare(
            md, k.float(), v.float())
    assert ring.state() == before and ring.dtype == torch.bfloat16
    with pytest.raises(RuntimeError, match="prepare\\(\\) once before"):
        gstep.launch(q, k, v, torch.zeros_like(q))


def test_forward_under_real_capture_without_a_graph_is_refused(gpu_device):
    """The capture check reads the stream's real capture status: forward()
    inside ``torch.cuda.graph`` with no capturable step for the batch raises
    before anything is recorded."""
    case = _Case(gpu_device, b=3, steps=2, seed=7)
    impl = case.build()
    md, q, k, v = case.step(0)
    before = impl._kivi_ring.state()
    out = torch.zeros((case.b, case.hq, case.d), dtype=torch.bfloat16, device=gpu_device)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="graph capture"):
        with torch.cuda.graph(graph):
            impl.forward(None, q, k, v, None, md, out)
    torch.cuda.synchronize()
    assert impl._kivi_ring.state() == before
    impl.forward(None, q, k, v, None, md, out)  # eager, outside the capture: runs
    torch.cuda.synchronize()
    case.oracle(impl, 0, out)


@pytest.mark.parametrize("g", [128, 64])
def test_host_kv_tensor_shape_runs_decode_against_oracle(gpu_device, g):
    """The host allocates one ``(2, NB, Bs, KVH, S)`` uint8 tensor through
    ``host_integration.kivi_int4_kv_cache_shape`` and hands ``(kv[0], kv[1])``
    to every forward (as the patched runner slices it); prefill writes and
    decode steps through ``forward`` leave pages and outputs that match the
    oracle, and the K and V halves hold exactly the two byte regions."""
    from vllm_ascend_quantized_kv_cache import host_integration as hi

    case = _Case(gpu_device, b=4, steps=131, seed=8 + g)
    shape = hi.kivi_int4_kv_cache_shape(case.nb, case.bs, case.kvh, case.d, g)
    assert shape == (2, case.nb, case.bs, case.kvh, case.d // 2 + 8 * case.d // g)
    kv = torch.zeros(shape, dtype=torch.uint8, device=gpu_device)
    case.g = g

    class Impl(ab.AscendKiviInt4AttentionBackendMixin):
        pass

    impl = Impl()
    impl.num_heads, impl.num_kv_heads, impl.head_size = case.hq, case.kvh, case.d
    impl.scale = case.d ** -0.5
    impl._init_kivi_state("kivi_int4")
    impl.kivi_group_size, impl.kivi_max_num_seqs = g, case.b
    for i, n in enumerate(case.lens):  # prefill: all-new prompts
        sl = torch.tensor([case.slot(i, p) for p in range(n)], device=gpu_device)
        md = SimpleNamespace(attn_state=SimpleNamespace(name="PrefillNoCache"), causal=True,
                             finished_req_ids=None, seq_lens_list=[n],
                             actual_seq_lengths_q=[n], slot_mapping=sl,
                             block_tables=case.table_dev[i:i + 1], req_ids=[case.reqs[i]],
                             num_actual_tokens=n)
        q = torch.randn(n, case.hq, case.d, device=gpu_device).to(torch.bfloat16)
        impl.forward(None, q, case.keys[i][:n].to(gpu_device),
                     case.values[i][:n].to(gpu_device), (kv[0], kv[1]), md,
                     torch.zeros_like(q))
    assert impl.k_quant_cache.untyped_storage().data_ptr() == kv.untyped_storage().data_ptr()
    for j in range(131):  # a key window flushes for every request
        md, q, k, v = case.step(j)
        out = torch.zeros((case.b, case.hq, case.d), dtype=torch.bfloat16, device=gpu_device)
        impl.forward(None, q, k, v, (kv[0], kv[1]), md, out)
        if j in (0, 130):
            torch.cuda.synchronize()
            case.oracle(impl, j, out)
    # the six views cover the two halves exactly: K views inside kv[0], V inside kv[1]
    k0, k1 = kv[0].data_ptr(), kv[0].data_ptr() + kv[0].numel()
    v0 = kv[1].data_ptr()
    caches = impl._kivi_caches()
    for t in caches[:3]:
        assert k0 <= t.data_ptr() and t.data_ptr() + t.numel() * t.element_size() <= k1
    for t in caches[3:]:
        assert v0 <= t.data_ptr() < v0 + kv[1].numel()
