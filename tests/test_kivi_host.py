# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 host logic on the CPU: geometry, byte views, the residual-window
state machine and every ``forward`` branch of the mixin.

Mirrors the reference's ``tests/test_kivi_int4.py``: the mixin runs for real
with only its kernel launch hooks replaced (pack, ring write, gather, decode
and dense attention), here by CPU versions built on the oracle.  The HIP
kernels behind the same hooks are checked on the GPU elsewhere.
"""

from __future__ import annotations

import random
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import kvq_oracle as ref
from tests._cpu_kernels import install_cpu_kernels
from vllm_ascend_quantized_kv_cache.methods.base import MethodConfig
from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import attention_backend as ab
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.byte_cache import (
    KiviByteCacheLayout,
    kivi_byte_cache_layout,
    kivi_caches_from_byte_tensors,
)
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.geometry import validate_kivi_config
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.semantics import KiviInt4Semantics

HEAD, KVH, GROUP, BLOCK = 32, 2, 8, 16


# ---------------------------------------------------------------------------
# geometry and semantics helpers
# ---------------------------------------------------------------------------


def test_validate_config_accepts_aligned_geometry():
    validate_kivi_config(MethodConfig(head_size=128, group_size=64, residual_length=128,
                                      block_size=128))


@pytest.mark.parametrize("overrides,match", [
    ({"group_size": 12}, "group_size divisible by 8"),
    ({"group_size": 16, "residual_length": 24}, "residual_length"),
    ({"head_size": 36, "group_size": 8}, "head_size divisible by 8"),
    ({"head_size": 48, "group_size": 32}, "divisible by group_size"),
    ({"group_size": 64, "block_size": 96}, "block_size"),
])
def test_validate_config_rejects_bad_geometry(overrides, match):
    base = dict(head_size=128, group_size=32, residual_length=64, block_size=128)
    base.update(overrides)
    with pytest.raises(ValueError, match=match):
        validate_kivi_config(MethodConfig(**base))


def _sem(residual=2 * GROUP, head=HEAD, group=GROUP):
    return KiviInt4Semantics(MethodConfig(head_size=head, num_kv_heads=KVH, group_size=group,
                                          residual_length=residual, block_size=BLOCK))


def test_is_aligned_key_window():
    sem = _sem()
    assert sem.is_aligned_key_window(list(range(8)), BLOCK)
    assert sem.is_aligned_key_window(list(range(8, 24)), BLOCK)
    assert not sem.is_aligned_key_window(list(range(1, 9)), BLOCK)
    assert not sem.is_aligned_key_window(list(range(12, 20)), BLOCK)  # straddles a block
    assert not sem.is_aligned_key_window([], BLOCK)
    assert not sem.is_aligned_key_window(list(range(7)), BLOCK)


def test_ordered_slots_matches_per_position_walk():
    rng = random.Random(0)
    table = torch.tensor([[3, -1, 0, 2], [1, 4, -1, -1]])
    lens = [50, 20]
    got = KiviInt4Semantics.ordered_slots(table, lens, BLOCK)
    for req, n in enumerate(lens):
        want = []
        for pos in range(n):
            blk = int(table[req, pos // BLOCK])
            if blk >= 0:
                want.append(blk * BLOCK + pos % BLOCK)
        assert got[req] == want
    assert rng is not None


def test_build_causal_mask_shape_and_values():
    mask = _sem().build_causal_mask(2, 4, torch.float32, "cpu")
    neg = torch.finfo(torch.float32).min
    assert mask.shape == (1, 2, 4)
    assert mask[0, 0, :3].equal(torch.zeros(3)) and mask[0, 0, 3].item() == neg
    assert mask[0, 1].equal(torch.zeros(4))


# ---------------------------------------------------------------------------
# the mixin over a stub host
# ---------------------------------------------------------------------------


class _StubBase:
    num_kv_heads = KVH
    head_size = HEAD
    num_heads = KVH
    num_queries_per_kv = 1
    scale = 0.125
    vllm_config = None


def _make_impl(residual=2 * GROUP, max_seqs=2, *, head=HEAD, kvh=KVH, group=GROUP,
               block=BLOCK, num_blocks=4, num_heads=None):
    class Impl(ab.AscendKiviInt4AttentionBackendMixin, _StubBase):
        pass

    impl = Impl()
    impl._init_kivi_state(None)
    impl.enable_kivi = True
    impl.head_size, impl.num_kv_heads = head, kvh
    impl.num_heads = num_heads or kvh
    impl.kivi_group_size, impl.kivi_residual_length = group, residual
    impl.kivi_max_num_seqs = max_seqs
    impl.k_quant_cache = torch.zeros(num_blocks, kvh, head, block // 8, dtype=torch.int32)
    impl.k_scale_cache = torch.ones(num_blocks, kvh, head, block // group)
    impl.k_mn_cache = torch.zeros(num_blocks, kvh, head, block // group)
    impl.v_quant_cache = torch.zeros(num_blocks, block, kvh, head // 8, dtype=torch.int32)
    impl.v_scale_cache = torch.ones(num_blocks, block, kvh, head // group)
    impl.v_mn_cache = torch.zeros(num_blocks, block, kvh, head // group)
    impl.calls = install_cpu_kernels(impl)
    return impl


def _six(impl):
    return impl._kivi_caches()


def _metadata(tokens, **overrides):
    md = SimpleNamespace(
        attn_state=SimpleNamespace(name="PrefillCacheHit"),
        actual_seq_lengths_q=[tokens], seq_lens_list=[tokens],
        slot_mapping=torch.arange(tokens, dtype=torch.long),
        block_tables=torch.tensor([[0, 1]], dtype=torch.long), req_ids=["r"],
        num_actual_tokens=tokens, causal=True, finished_req_ids=None,
    )
    for k, v in overrides.items():
        setattr(md, k, v)
    return md


def test_residual_row_lifecycle():
    impl = _make_impl()
    assert impl._get_kivi_residual_row("a", create=False) is None
    row = impl._get_kivi_residual_row("a", create=True)
    assert row == 0 and impl._get_kivi_residual_row("a", create=False) == row
    impl._release_kivi_residual_row("a")
    assert impl._get_kivi_residual_row("a", create=False) is None
    assert impl.kivi_residual_free_rows == [1, 0]


def test_residual_rows_exhaustion_fails_closed():
    impl = _make_impl(max_seqs=1)
    impl._get_kivi_residual_row("r0", create=True)
    with pytest.raises(RuntimeError, match="exhausted"):
        impl._get_kivi_residual_row("r1", create=True)


def test_store_entries_and_key_flush_whole_window():
    impl = _make_impl()
    key = torch.randn(2 * GROUP, KVH, HEAD)
    slots = torch.arange(2 * GROUP)
    impl._store_kivi_residual_entries(key, slots, req_key="r", is_key=True)
    assert impl.calls["key_pack"] == []
    assert impl._collect_kivi_residual_window("r", is_key=True)[0] == slots.tolist()
    key2 = torch.randn(1, KVH, HEAD)
    impl._store_kivi_residual_entries(key2, torch.tensor([32]), req_key="r", is_key=True)
    assert len(impl.calls["key_pack"]) == 1
    flushed, flush_slots = impl.calls["key_pack"][0]
    assert torch.equal(flushed, key) and torch.equal(flush_slots, slots)
    got_slots, rows = impl._collect_kivi_residual_window("r", is_key=True)
    assert got_slots == [32] and torch.equal(rows[0], key2[0])


def test_store_mixed_overwrite_and_value_eviction_keeps_order():
    impl = _make_impl()
    value = torch.randn(2 * GROUP, KVH, HEAD)
    impl._store_kivi_residual_entries(value, torch.arange(2 * GROUP), req_key="r", is_key=False)
    batch = torch.randn(2, KVH, HEAD)
    impl._store_kivi_residual_entries(batch, torch.tensor([5, 2 * GROUP]), req_key="r",
                                      is_key=False)
    assert len(impl.calls["value_pack"]) == 1
    flushed, flush_slots = impl.calls["value_pack"][0]
    assert flush_slots.tolist() == [0] and torch.equal(flushed[0], value[0])
    slots, rows = impl._collect_kivi_residual_window("r", is_key=False)
    assert slots == list(range(1, 2 * GROUP + 1))
    assert torch.equal(rows[4], batch[0]) and torch.equal(rows[-1], batch[1])
    assert torch.equal(rows[0], value[1])


def test_overwrite_then_evict_packs_the_overwritten_row():
    """A lane overwritten in this batch and evicted later in the same batch
    must be packed with its new content (the plan reads the step's input)."""
    impl = _make_impl()
    value = torch.randn(2 * GROUP, KVH, HEAD)
    impl._store_kivi_residual_entries(value, torch.arange(2 * GROUP), req_key="r", is_key=False)
    batch = torch.randn(3, KVH, HEAD)
    impl._store_kivi_residual_entries(batch, torch.tensor([0, 16, 17]), req_key="r",
                                      is_key=False)
    packed = torch.cat([c[0] for c in impl.calls["value_pack"]])
    slots = torch.cat([c[1] for c in impl.calls["value_pack"]])
    assert slots.tolist() == [0, 1]
    assert torch.equal(packed[0], batch[0]) and torch.equal(packed[1], value[1])


def test_value_flush_is_slot_at_a_time():
    impl = _make_impl()
    value = torch.randn(2 * GROUP + 1, KVH, HEAD)
    slots = torch.arange(2 * GROUP + 1)
    impl._store_kivi_residual_entries(value, slots, req_key="r", is_key=False)
    assert len(impl.calls["value_pack"]) == 1
    assert impl.calls["value_pack"][0][1].tolist() == [0]
    assert impl._collect_kivi_residual_window("r", is_key=False)[0] == slots[1:].tolist()


def test_bulk_prefill_flushes_a_full_window_that_incremental_writes_keep_exact():
    tokens = 2 * GROUP
    key, value = torch.randn(tokens, KVH, HEAD), torch.randn(tokens, KVH, HEAD)
    slots = torch.arange(tokens)
    bulk = _make_impl()
    bulk._write_kivi_prefill_cache(key, value, slots, ["bulk"], [tokens])
    assert len(bulk.calls["key_pack"]) == len(bulk.calls["value_pack"]) == 1
    assert torch.equal(bulk.calls["key_pack"][0][1], slots)
    assert bulk._get_kivi_residual_row("bulk", create=False) is None
    inc = _make_impl()
    for s in range(tokens):
        inc._write_kivi_cache(key[s:s + 1], value[s:s + 1], slots[s:s + 1], ["i"], [s + 1])
    assert inc.calls["key_pack"] == [] and inc.calls["value_pack"] == []
    row = inc._get_kivi_residual_row("i", create=False)
    assert inc.kivi_residual_key_len[row] == tokens == inc.kivi_residual_value_len[row]


def test_single_token_steps_plan_one_launch():
    """With R + 1 lanes per row, a step that appends one token per request
    never writes a ring lane the same step packs (keys flush whole windows,
    values evict one lane), so every such plan is one launch; the window still
    holds the newest R tokens in order."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.residual import (
        KiviResidualRing,
        StorePlan,
    )

    window, rows = 8, 3
    ring = KiviResidualRing(rows, window, 1, 8, device="cpu")
    assert ring.ring_len == window + 1 and ring.key.shape[1] == window + 1
    seen = {"kp": 0, "vp": 0}
    for step in range(5 * window + 3):
        plan = StorePlan()
        for row in range(rows):
            slot = [row * 1000 + step]
            for is_key in (True, False):
                ring.plan_store(plan, row, slot, [row], is_key=is_key, block_size=8,
                                group_size=8)
        one = plan.one_launch_jobs()
        assert one is not None, f"step {step} writes a lane it packs"
        jobs, (nkp, nvp, nkr, nvr) = one
        assert len(jobs) == 2 * (nkp + nvp + nkr + nvr)
        assert (nkr, nvr) == (rows, rows)
        seen["kp"] += nkp
        seen["vp"] += nvp
        for row in range(rows):
            newest = [row * 1000 + x for x in range(step + 1)]
            assert ring.window_slots(row, is_key=False) == newest[-window:]
            n_keys = len(ring.window_slots(row, is_key=True))
            assert ring.window_slots(row, is_key=True) == newest[len(newest) - n_keys:]
            assert 1 <= n_keys <= window
    assert seen["kp"] > 0 and seen["vp"] > 0


@pytest.mark.parametrize("seed", range(6))
def test_closed_form_run_plan_equals_token_replay(seed):
    """``_plan_run`` (a run of new slots in closed form) leaves the same mirror
    and emits the same plan as the per-token replay, over random run lengths
    (shorter and longer than the window, several windows at once), starting
    from windows of every fill level, several runs into one plan, and an
    unaligned key window that both reject."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.residual import (
        KiviResidualRing,
        StorePlan,
    )

    rng = random.Random(seed)
    group = rng.choice([8, 16])
    window = group * rng.choice([1, 2])
    block = max(window, group) * rng.choice([1, 2])
    rows = 3
    rings = [KiviResidualRing(rows, window, 1, 8, device="cpu") for _ in range(2)]
    pos = [0] * rows
    base = [(rng.randrange(0, 4) + 64 * r) * block for r in range(rows)]

    def state(ring):
        return ring.state()

    for _step in range(12):
        plans = [StorePlan(), StorePlan()]
        for _ in range(rng.randrange(1, 4)):
            row = rng.randrange(rows)
            n = rng.choice([2, 3, window - 1, window, window + 1, 3 * window + 5])
            n = max(2, n)
            slots = list(range(base[row] + pos[row], base[row] + pos[row] + n))
            inputs = [rng.randrange(0, 500) for _ in range(n)]
            for is_key in (True, False):
                rings[0]._plan_run(plans[0], row, slots, inputs, is_key=is_key,
                                   block_size=block, group_size=group)
                rings[1]._plan_tokens(plans[1], row, slots, inputs, is_key=is_key,
                                      block_size=block, group_size=group)
            pos[row] += n
        assert state(rings[0]) == state(rings[1])
        for a, b in ((plans[0].key, plans[1].key), (plans[0].value, plans[1].value)):
            assert a.pack_src == b.pack_src and a.pack_slots == b.pack_slots
            assert a.ring == b.ring and a.lane_src == b.lane_src
    # a key window that starts off a group boundary is rejected by both
    row = 0
    ring_a, ring_b = (KiviResidualRing(1, window, 1, 8, device="cpu") for _ in range(2))
    slots = list(range(3, 3 + window + 1))
    for ring, fn in ((ring_a, ring_a._plan_run), (ring_b, ring_b._plan_tokens)):
        with pytest.raises(RuntimeError, match="aligned token groups"):
            fn(StorePlan(), row, slots, list(range(len(slots))), is_key=True,
               block_size=block, group_size=group)


@pytest.mark.parametrize("seed", range(4))
def test_decode_step_plan_equals_token_replay(seed):
    """``plan_decode_step`` (one token per request, the whole batch at once)
    leaves the same mirror and emits the same jobs as ``plan_store`` token by
    token, over steps that fill windows, flush key windows and evict values,
    with requests joining at different lengths; an unaligned key window is
    rejected with no row changed."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.residual import (
        KiviResidualRing,
        StorePlan,
    )

    rng = random.Random(seed)
    group = rng.choice([8, 16])
    window = group * rng.choice([1, 2, 3])
    block = 2 * window
    rows = 6
    fast, slow = (KiviResidualRing(rows, window, 1, 8, device="cpu") for _ in range(2))
    pos = [rng.randrange(0, 3 * window) if r % 2 else 0 for r in range(rows)]
    base = [(64 * r + 1) * block for r in range(rows)]
    for r in range(rows):  # earlier tokens, written as one run
        if pos[r]:
            slots = list(range(base[r], base[r] + pos[r]))
            for ring in (fast, slow):
                for k in (True, False):
                    ring.plan_store(StorePlan(), r, slots, list(range(pos[r])), is_key=k,
                                    block_size=block, group_size=group,
                                    positions=list(range(pos[r])))
    for _ in range(3 * window + 5):
        batch = sorted(rng.sample(range(rows), rng.randrange(1, rows + 1)))
        rws = np.asarray(batch, dtype=np.int64)
        slots = np.asarray([base[r] + pos[r] for r in batch], dtype=np.int64)
        p = np.asarray([pos[r] for r in batch], dtype=np.int64)
        jobs = fast.plan_decode_step(rws, slots, p, np.arange(len(batch)), block_size=block,
                                     group_size=group)
        assert jobs is not None
        plan = StorePlan()
        for i, r in enumerate(batch):
            for k in (True, False):
                slow.plan_store(plan, r, [int(slots[i])], [i], is_key=k, block_size=block,
                                group_size=group, positions=[pos[r]])
        assert fast.state() == slow.state()
        for k in (True, False):
            assert np.array_equal(fast.lane_pos[k], slow.lane_pos[k])
        assert jobs.key_pack_src.tolist() == plan.key.pack_src
        assert jobs.key_pack_slot.tolist() == plan.key.pack_slots
        assert jobs.value_pack_src.tolist() == plan.value.pack_src
        assert jobs.value_pack_slot.tolist() == plan.value.pack_slots
        assert dict(zip(jobs.key_ring_dst.tolist(), jobs.key_ring_src.tolist())) == plan.key.ring
        assert dict(zip(jobs.value_ring_dst.tolist(),
                        jobs.value_ring_src.tolist())) == plan.value.ring
        for r in batch:
            pos[r] += 1
    # a held slot, or a repeated row, is left to the per-token path
    r0 = np.asarray([0], dtype=np.int64)
    held = np.asarray([base[0] + pos[0] - 1], dtype=np.int64)
    assert fast.plan_decode_step(r0, held, held - base[0], r0, block_size=block,
                                 group_size=group) is None
    assert fast.plan_decode_step(np.asarray([1, 1]), np.asarray([7, 8]), np.asarray([0, 1]),
                                 np.asarray([0, 1]), block_size=block, group_size=group) is None
    # a full key window that starts off a group boundary: rejected, nothing changed
    bad = KiviResidualRing(2, window, 1, 8, device="cpu")
    for r in range(2):
        sl = list(range(3 + 64 * block * r, 3 + 64 * block * r + window))
        for k in (True, False):
            bad.plan_store(StorePlan(), r, sl, list(range(window)), is_key=k, block_size=block,
                           group_size=group)
    before = bad.state()
    with pytest.raises(RuntimeError, match="aligned token groups"):
        bad.plan_decode_step(np.asarray([0, 1]), np.asarray([3 + window, 64 * block + 3 + window]),
                             np.asarray([window, window]), np.asarray([0, 1]), block_size=block,
                             group_size=group)
    assert bad.state() == before


def test_multi_token_batch_that_reuses_a_packed_lane_is_not_one_launch():
    """Two tokens into a full value window: the second lands on the lane the
    first evicted and packed, so the plan must keep packs before ring writes."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.residual import (
        KiviResidualRing,
        StorePlan,
    )

    window = 4
    ring = KiviResidualRing(1, window, 1, 8, device="cpu")
    plan = StorePlan()
    ring.plan_store(plan, 0, list(range(window)), list(range(window)), is_key=False,
                    block_size=8, group_size=8)
    assert plan.one_launch_jobs() is not None  # no pack yet
    plan = StorePlan()
    ring.plan_store(plan, 0, [window, window + 1], [0, 1], is_key=False, block_size=8,
                    group_size=8)
    assert plan.value.pack_slots == [0, 1]
    assert plan.one_launch_jobs() is None


def test_one_launch_store_geometry_gate():
    from vllm_ascend_quantized_kv_cache.ops.kivi_pack import store_one_launch_supported

    assert store_one_launch_supported(128, 128, torch.bfloat16)
    assert store_one_launch_supported(128, 64, torch.float16)
    assert not store_one_launch_supported(64, 64, torch.bfloat16)
    assert not store_one_launch_supported(128, 32, torch.bfloat16)
    assert not store_one_launch_supported(128, 128, torch.float32)


@pytest.mark.parametrize("cu_count,kvh,tile",
                         [(256, 8, 64), (3, 4, 64), (1, 1, 64), (256, 2, 64), (256, 8, 128),
                          (3, 8, 128)])
def test_plan_decode_pieces_invariants(cu_count, kvh, tile):
    """Equal-cost pieces: at most one wave slot per piece, items of a request
    contiguous and covering it exactly (int4 items on `tile`-position starts,
    both sides int4 over them), pieces covering the list in order, and piece
    costs within one step of each other.  Tile 128 (the page-streaming
    decode's pages): no page is split between two pieces."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        PIECE_MAX_COST,
        TAIL_POSITION_COST,
        DecodeSeq,
        plan_decode_pieces,
    )

    rng = random.Random(cu_count * 10 + kvh)
    seqs = []
    for i in range(40):
        n = rng.choice([0, 1, 63, 64, 65, 300, 4097, rng.randrange(1, 20000)])
        r = 128
        hk = ((n - 1) // r) * r if n else 0
        hv = max(0, n - r)
        seqs.append(DecodeSeq(n, hk, hv, i, 0, 0))
    meta, work, pieces = plan_decode_pieces(seqs, kvh, cu_count, tile=tile)
    slots = max(1, cu_count * 8 // kvh)
    total = 0.0
    for s in seqs:
        a = max(0, min(s.k_hist, s.v_hist, s.seq_len))
        total += -(-a // tile) * tile + (s.seq_len - a) * TAIL_POSITION_COST
    per_round = slots
    rounds = max(1, -(-int(total) // int(slots * PIECE_MAX_COST)))  # whole rounds
    slots *= rounds
    if tile == 128 and rounds >= 2 and total / slots >= 8 * tile:
        slots += per_round  # the last round in pieces of half the cost
    assert 1 <= len(pieces) - 1 <= slots
    assert pieces[0] == 0 and pieces[-1] == len(work)
    assert all(a < b for a, b in zip(pieces[:-1], pieces[1:]))
    for b, s in enumerate(seqs):
        first, count = int(meta[b, 6]), int(meta[b, 7])
        assert count >= 1
        its = work[first : first + count]
        assert (its[:, 0] == b).all()
        pos = 0
        for _, p, e, kind in its.tolist():
            assert p == pos and e >= p
            pos = e
            if kind == 0:
                assert p % tile == 0 and e <= min(s.k_hist, s.v_hist) and e > p
        assert pos == s.seq_len
    if len(pieces) - 1 == slots and slots > 1 and rounds == 1 and not (tile == 128 and slots == cu_count):
        cost = [
            sum(-(-(e - p) // tile) * tile if k == 0 else (e - p) * TAIL_POSITION_COST
                for _, p, e, k in work[pieces[i] : pieces[i + 1]].tolist())
            for i in range(len(pieces) - 1)
        ]
        step = sum(cost) / slots
        assert max(cost) <= step + 2 * 32 * TAIL_POSITION_COST + tile


def test_page_streaming_one_round_plan_weights_the_first_dispatched_pieces():
    """Config 3's shape (32 requests of 2048-16384 positions, 8 KV heads, 256
    CUs, page tiles): one round of 256 pieces whose first half (the first
    workgroup on each CU) carries 1.4 times the cost of the second half, each
    piece within a step of its share, the requests covered exactly."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        PAGE_TILE,
        TAIL_POSITION_COST,
        DecodeSeq,
        plan_decode_pieces,
    )

    rng = random.Random(3)
    seqs = []
    for i in range(32):
        n = rng.randrange(2048, 16385)
        seqs.append(DecodeSeq(n, ((n - 1) // 128) * 128, n - 128, i, 0, 0))
    meta, work, pieces = plan_decode_pieces(seqs, 8, 256, tile=PAGE_TILE)
    assert len(pieces) - 1 == 256
    cost = [
        sum(-(-(e - p) // PAGE_TILE) * PAGE_TILE if k == 0 else (e - p) * TAIL_POSITION_COST
            for _, p, e, k in work[pieces[i] : pieces[i + 1]].tolist())
        for i in range(256)
    ]
    unit = sum(cost) / (1.4 * 128 + 128)
    margin = PAGE_TILE + 2 * 32 * TAIL_POSITION_COST
    for i, c in enumerate(cost):
        share = 1.4 * unit if i < 128 else unit
        assert abs(c - share) <= margin, (i, c, share)
    ratio = (sum(cost[:128]) / 128) / (sum(cost[128:]) / 128)
    assert 1.3 < ratio < 1.5
    for b, s in enumerate(seqs):
        first, count = int(meta[b, 6]), int(meta[b, 7])
        pos = 0
        for _, p, e, _ in work[first : first + count].tolist():
            assert p == pos
            pos = e
        assert pos == s.seq_len


def test_plan_pieces_rejects_other_tiles():
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, plan_decode_pieces

    with pytest.raises(RuntimeError):
        plan_decode_pieces([DecodeSeq(300, 256, 172, 0, 0, 0)], 8, 256, tile=96)


def test_page_streaming_plan_covers_any_amount_of_work_in_pieces():
    """With page streaming the default plan is pieces on page bounds, also for
    work that takes many rounds (config 5's shape)."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        DecodeSeq,
        page_streaming_applies,
        plan_decode,
    )

    big = [DecodeSeq(32768, 32640, 32640, i, 0, 0) for i in range(256)]
    _, work, pieces = plan_decode(big, 8, 256, page_streaming=True)
    assert pieces is not None and pieces[0] == 0 and pieces[-1] == len(work)
    # 32640 int4 positions + 128 tail positions at 6 each: 9 rounds of 256,
    # the last of them cut into 512 pieces of half the cost
    assert len(pieces) - 1 == 256 * 8 + 512
    cost = [
        sum(-(-(e - p) // 128) * 128 if k == 0 else (e - p) * 6.0
            for _, p, e, k in work[pieces[i] : pieces[i + 1]].tolist())
        for i in range(len(pieces) - 1)
    ]
    step = sum(cost) / (256 * 9)
    assert all(abs(c - step) <= 128 + 2 * 32 * 6.0 for c in cost[:2048])
    assert all(abs(c - step / 2) <= 128 + 2 * 32 * 6.0 for c in cost[2048:])
    int4 = work[work[:, 3] == 0]
    assert (int4[:, 1] % 128 == 0).all()
    assert page_streaming_applies(64, 8, 128, 128, 64, torch.bfloat16, torch.bfloat16)
    assert page_streaming_applies(40, 8, 128, 128, 128, torch.float16, torch.float16)
    assert not page_streaming_applies(40, 8, 128, 128, 128, torch.float16, torch.bfloat16)
    assert not page_streaming_applies(32, 4, 128, 128, 128, torch.bfloat16, torch.bfloat16)
    assert not page_streaming_applies(64, 8, 128, 64, 64, torch.bfloat16, torch.bfloat16)
    assert not page_streaming_applies(136, 8, 128, 128, 64, torch.bfloat16, torch.bfloat16)


def test_plan_decode_picks_pieces_for_one_round_and_splits_beyond():
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, plan_decode

    small = [DecodeSeq(9000, 8960, 8872, i, 0, 0) for i in range(32)]
    _, work, pieces = plan_decode(small, 8, 256)
    assert pieces is not None and pieces[-1] == len(work)
    big = [DecodeSeq(32768, 32640, 32640, i, 0, 0) for i in range(256)]
    _, work, pieces = plan_decode(big, 8, 256)
    assert pieces is None
    assert (work[work[:, 3] == 0][:, 1] % 128 == 0).all()


@pytest.mark.parametrize("split", [128, 256, 4096])
def test_plan_decode_work_pairs(split):
    """Paired int4 items: kind 2 at an even index, its kind-3 twin right after
    over the same range; a request's items stay contiguous and cover it."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import DecodeSeq, plan_decode_work

    rng = random.Random(split)
    seqs = []
    for i in range(30):
        n = rng.choice([0, 1, 130, 300, 4097, rng.randrange(1, 30000)])
        hk = ((n - 1) // 128) * 128 if n else 0
        seqs.append(DecodeSeq(n, hk, max(0, n - 128), i, 0, 0))
    meta, work = plan_decode_work(seqs, split, paired=True)
    kinds = work[:, 3].tolist()
    for i, k in enumerate(kinds):
        if k == 2:
            assert i % 2 == 0 and kinds[i + 1] == 3
            assert (work[i, :3] == work[i + 1, :3]).all()
            assert work[i, 1] % 128 == 0 and work[i, 2] - work[i, 1] <= 2 * split
        if k == 3:
            assert i % 2 == 1 and kinds[i - 1] == 2
        assert k != 0
    for b, s in enumerate(seqs):
        first, count = int(meta[b, 6]), int(meta[b, 7])
        its = work[first : first + count]
        assert (its[:, 0] == b).all()
        covered = 0
        for _, p, e, k in its.tolist():
            if k == 3:
                continue
            assert p == covered or (p == 0 and e == 0)
            covered = max(covered, e)
        assert covered == s.seq_len


def test_misaligned_key_flush_fails_closed_before_kernel():
    impl = _make_impl()
    key = torch.randn(GROUP, KVH, HEAD)
    with pytest.raises(RuntimeError, match="aligned token groups"):
        impl._write_kivi_key_quant_cache(key, torch.arange(1, 1 + GROUP))
    with pytest.raises(RuntimeError, match="whole token groups"):
        impl._write_kivi_key_quant_cache(key[:-1], torch.arange(GROUP - 1))
    assert impl.calls["key_pack"] == []


def test_misaligned_window_flush_fails_closed_before_any_launch():
    impl = _make_impl()
    key = torch.randn(2 * GROUP, KVH, HEAD)
    impl._store_kivi_residual_entries(key, torch.arange(3, 3 + 2 * GROUP), req_key="r",
                                      is_key=True)
    with pytest.raises(RuntimeError, match="aligned token groups"):
        impl._store_kivi_residual_entries(key[:1], torch.tensor([40]), req_key="r",
                                          is_key=True)
    assert impl.calls["key_pack"] == []


def test_rejected_batch_leaves_every_mirror_unchanged():
    """A batch whose second request fails its key flush launches nothing, and
    the first request's window (and the row a new request took) roll back."""
    impl = _make_impl(max_seqs=3)
    kv = torch.randn(2 * GROUP, KVH, HEAD)
    impl._write_kivi_cache(kv[:1], kv[:1], torch.tensor([40]), ["a"], [1])
    # an unaligned full window for "b": its next token must flush slots 3..18
    impl._write_kivi_cache(kv, kv, torch.arange(3, 3 + 2 * GROUP), ["b"], [2 * GROUP])
    ring = impl._kivi_ring

    def snapshot():
        return (dict(impl.kivi_residual_req_to_row), list(impl.kivi_residual_free_rows),
                ring.state())

    before = snapshot()
    launches = {k: len(v) for k, v in impl.calls.items()}
    batch = torch.randn(3, KVH, HEAD)
    with pytest.raises(RuntimeError, match="aligned token groups"):
        impl._write_kivi_cache(batch, batch, torch.tensor([41, 60, 3 + 2 * GROUP]),
                               ["a", "c", "b"], [1, 2, 3])
    assert snapshot() == before
    assert {k: len(v) for k, v in impl.calls.items()} == launches
    # the rolled-back mirror still plans the next good step from the old state
    impl._write_kivi_cache(batch[:1], batch[:1], torch.tensor([41]), ["a"], [1])
    row = impl._get_kivi_residual_row("a", create=False)
    assert ring.window_slots(row, is_key=True) == [40, 41]


def test_aligned_key_flush_reaches_kernel_hook():
    impl = _make_impl()
    key = torch.randn(GROUP, KVH, HEAD)
    impl._write_kivi_key_quant_cache(key, torch.arange(GROUP))
    assert len(impl.calls["key_pack"]) == 1
    assert impl.calls["key_pack"][0][0].dtype == torch.float32  # reference hands fp32 rows


def test_release_finished_rows_clears_windows():
    impl = _make_impl()
    impl._store_kivi_residual_entries(torch.randn(2, KVH, HEAD), torch.tensor([0, 1]),
                                      req_key="r", is_key=False)
    assert impl._has_kivi_residual_entry(0, req_key="r", is_key=False)
    impl._release_finished_kivi_residual_rows({"r"})
    assert not impl._has_kivi_residual_entry(0, req_key="r", is_key=False)
    assert impl._get_kivi_residual_row("r", create=False) is None


def test_sync_windows_releases_finished_and_keeps_live():
    impl = _make_impl()
    impl._get_kivi_residual_row("live", create=True)
    impl._get_kivi_residual_row("dead", create=True)
    impl._sync_kivi_residual_windows(torch.tensor([[0], [1]]), [1, 1], ["live"],
                                     finished_req_ids={"dead"})
    assert impl._get_kivi_residual_row("dead", create=False) is None
    assert impl._get_kivi_residual_row("live", create=False) is not None


def test_sync_prunes_residual_slots_the_request_no_longer_owns():
    impl = _make_impl()
    value = torch.randn(4, KVH, HEAD)
    impl._store_kivi_residual_entries(value, torch.tensor([0, 1, 2, 3]), req_key="r",
                                      is_key=False)
    impl._sync_kivi_residual_windows(torch.tensor([[0]]), [2], ["r"])
    slots, rows = impl._collect_kivi_residual_window("r", is_key=False)
    assert slots == [0, 1] and torch.equal(rows, value[:2])
    assert impl._get_kivi_residual_row("r", create=False) is not None


def test_prune_compacts_a_wrapped_window():
    """Pruning after the ring wrapped keeps FIFO order and the right rows."""
    impl = _make_impl(residual=GROUP)
    value = torch.randn(GROUP + 3, KVH, HEAD)
    impl._store_kivi_residual_entries(value, torch.arange(GROUP + 3), req_key="r",
                                      is_key=False)
    # window now holds slots 3..10 in lanes 3..7,0..2 (wrapped)
    impl._sync_kivi_residual_windows(torch.tensor([[0]]), [9], ["r"])
    slots, rows = impl._collect_kivi_residual_window("r", is_key=False)
    assert slots == list(range(3, 9)) and torch.equal(rows, value[3:9])


def test_bind_kivi_cache_rejects_bad_layouts():
    impl = _make_impl()
    with pytest.raises(RuntimeError, match="6-tuple"):
        impl._bind_kivi_cache((impl.k_quant_cache,))
    impl._bind_kivi_cache(list(_six(impl)))
    assert impl.kivi_residual_key_cache is not None


def test_chunked_prefill_with_history_predicate():
    impl = _make_impl()
    md = SimpleNamespace(actual_seq_lengths_q=[8, 16], seq_lens_list=[32, 16], num_decodes=1,
                         num_decode_tokens=8, num_prefills=1)
    assert impl._is_kivi_chunked_prefill_all_new(md) is False
    md.seq_lens_list = [32, 8]
    assert impl._is_kivi_chunked_prefill_all_new(md) is True


# ---------------------------------------------------------------------------
# forward branches
# ---------------------------------------------------------------------------


def test_forward_guards_fail_closed():
    impl = _make_impl()
    q = torch.randn(1, KVH, HEAD)
    out = torch.ones(1, KVH, HEAD)
    assert impl.forward(None, q, q, q, _six(impl), None, out) is out
    assert torch.equal(out, torch.zeros_like(out))
    with pytest.raises(NotImplementedError, match="fused output quantization"):
        impl.forward(None, q, q, q, _six(impl), _metadata(1), out, output_scale=out.clone())
    with pytest.raises(RuntimeError, match="6-tuple"):
        impl.forward(None, q, q, q, (impl.k_quant_cache,), _metadata(1), out)
    impl.enable_kivi = False
    with pytest.raises(RuntimeError, match="kivi_int4 cache dtype"):
        impl.forward(None, q, q, q, _six(impl), _metadata(1), out)


def _expected_dense(key, value, residual):
    """Closed form of the incremental rule for one request written in one step."""
    t = key.shape[0]
    hk, hv = ref.incremental_split(t, residual)
    g = GROUP
    ek = torch.cat([ref.fake_quant_key(key[:hk], g), key[hk:]])
    ev = torch.cat([ref.fake_quant_value(value[:hv], g), value[hv:]])
    return ek, ev


def test_forward_history_plus_residual_matches_quantized_reference():
    residual = 2 * GROUP
    tokens = residual + 1
    torch.manual_seed(7)
    impl = _make_impl(residual)
    q, k, v = (torch.randn(tokens, KVH, HEAD) for _ in range(3))
    out = torch.zeros(tokens, KVH, HEAD)
    got = impl.forward(None, q, k, v, _six(impl), _metadata(tokens), out)
    ek, ev = _expected_dense(k, v, residual)
    gk, gv = impl._gather_dequant_kivi_paged_cache(torch.tensor([[0, 1]]), [tokens],
                                                   torch.float32, ["r"])
    assert torch.equal(gk, ek) and torch.equal(gv, ev)
    want = ref.attention(q, ek, ev, [tokens], [tokens], impl.scale, True)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)
    exact = ref.attention(q, k, v, [tokens], [tokens], impl.scale, True)
    assert (got - exact).abs().max() > 1e-3  # the int4 history is in the loop
    assert impl.k_quant_cache.any() and impl.v_quant_cache.any()


def test_prefill_nocache_attends_raw_kv_and_writes_history():
    tokens = 2 * GROUP + 1
    impl = _make_impl()
    q, k, v = (torch.randn(tokens, KVH, HEAD) for _ in range(3))
    out = torch.zeros(tokens, KVH, HEAD)
    md = _metadata(tokens, attn_state=SimpleNamespace(name="PrefillNoCache"))
    impl.forward(None, q, k, v, _six(impl), md, out)
    assert impl.calls["dense"] == [([tokens], [tokens], True)]
    torch.testing.assert_close(out, ref.attention(q, k, v, [tokens], [tokens], impl.scale,
                                                  True), atol=1e-5, rtol=1e-5)
    # bulk writer: one full window of R tokens to history, the last token resident
    assert impl.calls["key_pack"][0][1].tolist() == list(range(2 * GROUP))
    row = impl._get_kivi_residual_row("r", create=False)
    assert row is not None and impl.kivi_residual_key_len[row] == 1


def test_decode_only_uses_fused_decode_over_history_and_window():
    impl = _make_impl()
    hist = 2 * GROUP
    pk, pv = torch.randn(2 * hist, KVH, HEAD), torch.randn(2 * hist, KVH, HEAD)
    impl._write_kivi_cache(pk, pv, torch.arange(2 * hist), ["a", "b"], [hist, 2 * hist])
    q, k, v = (torch.randn(2, KVH, HEAD) for _ in range(3))
    out = torch.zeros(2, KVH, HEAD)
    seq = hist + 1
    md = _metadata(2, attn_state=SimpleNamespace(name="DecodeOnly"), seq_lens_list=[seq, seq],
                   slot_mapping=torch.tensor([2 * BLOCK, 3 * BLOCK]),
                   block_tables=torch.tensor([[0, 2], [1, 3]]), req_ids=["a", "b"])
    impl.forward(None, q, k, v, _six(impl), md, out)
    assert len(impl.calls["decode"]) == 1
    seqs = impl.calls["decode"][0]
    assert [(s.seq_len, s.k_hist, s.v_hist) for s in seqs] == [(seq, hist, 1)] * 2
    for i, req in enumerate("ab"):
        kk = torch.cat([pk[i * hist:(i + 1) * hist], k[i:i + 1]])
        vv = torch.cat([pv[i * hist:(i + 1) * hist], v[i:i + 1]])
        ek, ev = _expected_dense(kk, vv, 2 * GROUP)
        want = ref.attention(q[i:i + 1], ek, ev, [1], [seq], impl.scale, True)
        torch.testing.assert_close(out[i:i + 1], want, atol=1e-5, rtol=1e-5)
    assert impl._has_kivi_residual_entry(2 * hist, req_key="a", is_key=True)
    assert not impl._has_kivi_residual_entry(0, req_key="a", is_key=True)


def test_chunked_prefill_dispatches_decode_rows_then_prompt_rows():
    impl = _make_impl()
    nd, prompt = 1, 4
    tokens = nd + prompt
    q, k, v = (torch.randn(tokens, KVH, HEAD) for _ in range(3))
    out = torch.zeros(tokens, KVH, HEAD)
    md = _metadata(tokens, attn_state=SimpleNamespace(name="ChunkedPrefill"),
                   actual_seq_lengths_q=[nd, tokens], seq_lens_list=[nd, prompt],
                   num_decodes=nd, num_decode_tokens=nd, num_prefills=1, req_ids=["d", "p"],
                   block_tables=torch.tensor([[0, 0], [1, 1]]))
    impl.forward(None, q, k, v, _six(impl), md, out)
    assert len(impl.calls["decode"]) == 1 and impl.calls["dense"] == [([prompt], [prompt], True)]
    torch.testing.assert_close(out[:nd], ref.attention(q[:nd], k[:nd], v[:nd], [1], [1],
                                                       impl.scale, True), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(out[nd:], ref.attention(q[nd:], k[nd:], v[nd:], [prompt],
                                                       [prompt], impl.scale, True),
                               atol=1e-5, rtol=1e-5)


def test_chunked_prefill_with_prompt_history_fails_closed():
    impl = _make_impl()
    tokens = 5
    md = _metadata(tokens, attn_state=SimpleNamespace(name="ChunkedPrefill"),
                   actual_seq_lengths_q=[1, tokens], seq_lens_list=[1, tokens + 2],
                   num_decodes=1, num_decode_tokens=1, num_prefills=1)
    x = torch.randn(tokens, KVH, HEAD)
    with pytest.raises(RuntimeError, match="historical KV cache"):
        impl.forward(None, x, x, x, _six(impl), md, torch.zeros_like(x))
    assert impl.calls["key_pack"] == [] and impl.calls["ring"] == []


def test_multi_step_decode_matches_window_model():
    """Prefill then many decode steps for two requests with shuffled pages:
    after every step the gathered K/V equal the reference-free window model
    (history packed in flush order by the oracle, window overlaid)."""
    residual, steps = 2 * GROUP, 2 * 2 * GROUP + 5  # two key flushes for request b
    nb = 8
    impl = _make_impl(residual, max_seqs=3, num_blocks=nb)
    table = torch.tensor([[5, 0, 3, 6], [2, 7, 1, 4]])
    rng = torch.Generator().manual_seed(3)
    lens = [11, 2 * GROUP]
    models = [ref.KiviWindowModel(residual) for _ in lens]
    caches = tuple(torch.zeros_like(t) if t.dtype == torch.int32 else torch.ones_like(t)
                   for t in _six(impl))
    oracle_caches = (caches[0], caches[1], torch.zeros_like(caches[2]), caches[3], caches[4],
                     torch.zeros_like(caches[5]))

    def slot(req, pos):
        return int(table[req, pos // BLOCK]) * BLOCK + pos % BLOCK

    # prefill (bulk writer) in one PrefillNoCache step
    kp = torch.randn(sum(lens), KVH, HEAD, generator=rng)
    vp = torch.randn(sum(lens), KVH, HEAD, generator=rng)
    slots = [slot(r, p) for r, n in enumerate(lens) for p in range(n)]
    md = _metadata(sum(lens), attn_state=SimpleNamespace(name="PrefillNoCache"),
                   actual_seq_lengths_q=[lens[0], sum(lens)], seq_lens_list=list(lens),
                   slot_mapping=torch.tensor(slots), block_tables=table, req_ids=["a", "b"])
    impl.forward(None, kp, kp, vp, _six(impl), md, torch.zeros_like(kp))
    start = 0
    for r, n in enumerate(lens):
        models[r].write_prefill(kp[start:start + n], vp[start:start + n], slots[start:start + n])
        start += n

    for _ in range(steps):
        q = torch.randn(2, KVH, HEAD, generator=rng)
        k = torch.randn(2, KVH, HEAD, generator=rng)
        v = torch.randn(2, KVH, HEAD, generator=rng)
        new = [slot(r, lens[r]) for r in range(2)]
        lens = [n + 1 for n in lens]
        md = _metadata(2, attn_state=SimpleNamespace(name="DecodeOnly"),
                       seq_lens_list=list(lens), slot_mapping=torch.tensor(new),
                       block_tables=table, req_ids=["a", "b"])
        impl.forward(None, q, k, v, _six(impl), md, torch.zeros(2, KVH, HEAD))
        for r in range(2):
            models[r].write(k[r:r + 1], v[r:r + 1], [new[r]])

    # oracle side: pack every model's history into fresh caches, gather, overlay
    for m in models:
        hk = m.history[True]
        hv = m.history[False]
        if hk:
            ref.pack_key_cache(torch.stack([row for _, row in hk]),
                               torch.tensor([s for s, _ in hk]), *oracle_caches[:3], GROUP)
        if hv:
            ref.pack_value_cache(torch.stack([row for _, row in hv]),
                                 torch.tensor([s for s, _ in hv]), *oracle_caches[3:], GROUP)
    dk, dv = ref.dequant_gather(*oracle_caches, table, torch.tensor(lens), torch.float32, GROUP)
    wk = [torch.stack([row for _, row in m.win[True]]) for m in models]
    wv = [torch.stack([row for _, row in m.win[False]]) for m in models]
    want_k = ref.overlay_residual(dk, lens, wk)
    want_v = ref.overlay_residual(dv, lens, wv)
    gk, gv = impl._gather_dequant_kivi_paged_cache(table, lens, torch.float32, ["a", "b"])
    assert torch.equal(gk, want_k) and torch.equal(gv, want_v)
    for r in range(2):
        row = impl._get_kivi_residual_row("ab"[r], create=False)
        hk_n, hv_n = len(models[r].history[True]), len(models[r].history[False])
        assert impl.kivi_residual_key_len[row] == lens[r] - hk_n
        assert impl.kivi_residual_value_len[row] == lens[r] - hv_n


# ---------------------------------------------------------------------------
# byte-region caches (the host's two buffers)
# ---------------------------------------------------------------------------


def _byte_caches(num_blocks=4, block=BLOCK):
    layout = KiviByteCacheLayout(num_blocks=num_blocks, block_size=block, num_kv_heads=KVH,
                                 head_size=HEAD, group_size=GROUP)
    key = torch.zeros(num_blocks, block, KVH, layout.bytes_per_token_head, dtype=torch.uint8)
    return key, torch.zeros_like(key), layout


def test_byte_cache_budget_matches_view_sizes():
    key, _, layout = _byte_caches()
    assert layout.bytes_per_token_head == HEAD // 2 + 8 * HEAD // GROUP
    assert key.numel() == layout.region_bytes == layout.key_bytes == layout.value_bytes
    assert layout.bytes_per_token == 2 * KVH * layout.bytes_per_token_head
    default = KiviByteCacheLayout(num_blocks=1, block_size=128, num_kv_heads=8, head_size=128,
                                  group_size=128)
    assert default.bytes_per_token_head == 72
    assert default.compression_vs_fp16() == pytest.approx(256 / 72, rel=1e-6)
    assert layout.compression_vs_fp16() < 2.0
    wide = KiviByteCacheLayout(num_blocks=1, block_size=128, num_kv_heads=1, head_size=256,
                               group_size=128)
    assert wide.bytes_per_token_head == 144
    g64 = KiviByteCacheLayout(num_blocks=1, block_size=128, num_kv_heads=8, head_size=128,
                              group_size=64)
    assert g64.bytes_per_token_head == 80


def test_byte_cache_views_alias_the_host_buffers():
    key, value, layout = _byte_caches()
    kq, ks, km, vq, vs, vm = kivi_caches_from_byte_tensors(key, value, layout)
    assert kq.shape == (4, KVH, HEAD, BLOCK // 8) and kq.dtype == torch.int32
    assert ks.shape == km.shape == (4, KVH, HEAD, BLOCK // GROUP) and ks.dtype == torch.float32
    assert vq.shape == (4, BLOCK, KVH, HEAD // 8)
    assert vs.shape == vm.shape == (4, BLOCK, KVH, HEAD // GROUP)
    kq[0, 0, 0, 0] = 0x04030201
    assert key.reshape(-1)[:4].tolist() == [1, 2, 3, 4]
    vs[0, 0, 0, 0] = 2.5
    off = vq.numel() * 4
    flat = value.reshape(-1)
    assert not flat[:off].any() and flat[off:off + 4].tolist() == [0, 0, 0x20, 0x40]
    assert key.reshape(-1)[:4].tolist() == [1, 2, 3, 4]


@pytest.mark.parametrize("break_it,match", [
    (lambda kv: (kv[0], kv[1][:1]), "equal regions"),
    (lambda kv: (kv[0].transpose(0, 1), kv[1]), "must be contiguous"),
    (lambda kv: (kv[0].reshape(-1)[:-7], kv[1].reshape(-1)[:-7]), "whole number of pages"),
])
def test_byte_cache_layout_rejects_bad_buffers(break_it, match):
    key, value, _ = _byte_caches()
    key, value = break_it((key, value))
    with pytest.raises(RuntimeError, match=match):
        kivi_byte_cache_layout(key, value, num_kv_heads=KVH, head_size=HEAD, group_size=GROUP)


@pytest.mark.parametrize("head,group,block,kvh,nb",
                         [(128, 128, 128, 8, 7), (32, 8, 16, 2, 3), (64, 32, 256, 4, 2)])
def test_host_published_numbers_rebuild_the_plugin_layout(head, group, block, kvh, nb):
    layout = KiviByteCacheLayout(num_blocks=nb, block_size=block, num_kv_heads=kvh,
                                 head_size=head, group_size=group)
    page = 2 * block * kvh * layout.bytes_per_token_head
    assert page * nb == 2 * layout.region_bytes == layout.page_size_bytes * nb
    raw = torch.zeros((2, nb, block, kvh, layout.bytes_per_token_head), dtype=torch.uint8)
    assert kivi_byte_cache_layout(raw[0], raw[1], num_kv_heads=kvh, head_size=head,
                                  group_size=group) == layout
    kq, ks, km, vq, vs, vm = kivi_caches_from_byte_tensors(raw[0], raw[1], layout)
    assert [t.dtype for t in (kq, ks, km)] == [torch.int32, torch.float32, torch.float32]
    assert kq.shape == (nb, kvh, head, block // 8) and vq.shape == (nb, block, kvh, head // 8)
    ks[0, 0, 0, 0] = 3.5
    assert float(raw[0].reshape(-1).view(torch.float32)[kq.numel()]) == 3.5


def test_forward_on_two_byte_buffers_matches_six_tuple_run():
    residual = 2 * GROUP
    tokens = residual + 1
    torch.manual_seed(21)
    q, k, v = (torch.randn(tokens, KVH, HEAD) for _ in range(3))
    six = _make_impl(residual)
    six_out = torch.zeros(tokens, KVH, HEAD)
    six.forward(None, q, k, v, _six(six), _metadata(tokens), six_out)
    kb, vb, layout = _byte_caches(num_blocks=six.k_quant_cache.shape[0])
    two = _make_impl(residual)
    two_out = torch.zeros(tokens, KVH, HEAD)
    two.forward(None, q, k, v, (kb, vb), _metadata(tokens), two_out)
    assert torch.equal(two_out, six_out)
    derived = kivi_caches_from_byte_tensors(kb, vb, layout)
    assert all(torch.equal(a, b) for a, b in zip(derived, _six(two)))
    assert kb.any()


@pytest.mark.parametrize("head,kvh,num_heads", [(128, 8, 8), (256, 1, 8)])
def test_forward_at_production_geometries_on_byte_buffers(head, kvh, num_heads):
    block = group = residual = 128
    nb = 3
    tokens = residual + 1
    layout = KiviByteCacheLayout(num_blocks=nb, block_size=block, num_kv_heads=kvh,
                                 head_size=head, group_size=group)
    kb = torch.zeros(nb, block, kvh, layout.bytes_per_token_head, dtype=torch.uint8)
    vb = torch.zeros_like(kb)
    impl = _make_impl(residual, head=head, kvh=kvh, group=group, block=block, num_blocks=nb,
                      num_heads=num_heads)
    torch.manual_seed(31)
    q = torch.randn(tokens, num_heads, head)
    k, v = torch.randn(tokens, kvh, head), torch.randn(tokens, kvh, head)
    out = torch.zeros(tokens, num_heads, head)
    impl.forward(None, q, k, v, (kb, vb), _metadata(tokens), out)
    assert torch.isfinite(out).all()
    hk, hv = ref.incremental_split(tokens, residual)
    ek = torch.cat([ref.fake_quant_key(k[:hk], group), k[hk:]])
    ev = torch.cat([ref.fake_quant_value(v[:hv], group), v[hv:]])
    gk, gv = impl._gather_dequant_kivi_paged_cache(torch.tensor([[0, 1]]), [tokens],
                                                   torch.float32, ["r"])
    assert torch.equal(gk, ek) and torch.equal(gv, ev)
    assert 3.5 < layout.compression_vs_fp16() < 3.7


# ---------------------------------------------------------------------------
# kernel-boundary validators and their agreement with the state machine
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("slots,num_tokens,match", [
    (torch.arange(8).view(2, 4), 8, "must be 1D"),
    (torch.arange(7), 8, "must match num_tokens"),
    (torch.arange(8, dtype=torch.float32), 8, "int32/int64"),
])
def test_slot_mapping_validator_rejects(slots, num_tokens, match):
    from vllm_ascend_quantized_kv_cache.ops.kivi_layout import _check_slot_mapping

    with pytest.raises(RuntimeError, match=match):
        _check_slot_mapping(slots, num_tokens)


def test_kivi_slot_group_guards_agree():
    from vllm_ascend_quantized_kv_cache.ops.kivi_layout import _check_key_slot_groups

    def kernel_accepts(slots):
        try:
            _check_key_slot_groups(torch.tensor(slots, dtype=torch.long), block_size=BLOCK,
                                   group_size=GROUP)
        except RuntimeError:
            return False
        return True

    sem = _sem()
    windows = {
        "one aligned group": list(range(GROUP)),
        "two aligned groups": list(range(2 * GROUP)),
        "second group of a block": list(range(GROUP, 2 * GROUP)),
        "misaligned start": list(range(1, 1 + GROUP)),
        "offset inside block": list(range(4, 4 + GROUP)),
        "hole in the window": [0, 1, 2, 3, 4, 5, 6, 9],
        "partial group": list(range(GROUP - 1)),
        "padding slot present": [-1] + list(range(1, GROUP)),
    }
    for label, slots in windows.items():
        assert sem.is_aligned_key_window(slots, BLOCK) == kernel_accepts(slots), label


@pytest.mark.parametrize("break_it,match", [
    (lambda c: c.__setitem__("kq", c["kq"].transpose(1, 2)), "must be contiguous"),
    (lambda c: c.__setitem__("ks", torch.zeros(2, 2, 32, 3)), "k_scale_cache layout"),
    (lambda c: c.__setitem__("vq", torch.zeros(2, 8, 2, 4, dtype=torch.int32)),
     "layout mismatch"),
    (lambda c: c.__setitem__("block_table", c["block_table"].float()),
     "block_table must be int32/int64"),
    (lambda c: c.__setitem__("seq_lens", torch.tensor([16, 16])), "must match"),
])
def test_gather_op_rejects_broken_cache_layout(break_it, match):
    from vllm_ascend_quantized_kv_cache.ops.kivi_gather import kivi_dequant_gather_cache

    nb, kvh, head = 2, 2, 32
    kq = torch.zeros(nb, kvh, head, BLOCK // 8, dtype=torch.int32)
    c = {"kq": kq, "ks": torch.ones(nb, kvh, head, BLOCK // GROUP),
         "km": torch.zeros(nb, kvh, head, BLOCK // GROUP),
         "vq": torch.zeros(nb, BLOCK, kvh, head // 8, dtype=torch.int32),
         "vs": torch.ones(nb, BLOCK, kvh, head // GROUP),
         "vm": torch.zeros(nb, BLOCK, kvh, head // GROUP),
         "block_table": torch.arange(nb).view(1, nb), "seq_lens": torch.tensor([nb * BLOCK])}
    break_it(c)
    with pytest.raises(RuntimeError, match=match):
        kivi_dequant_gather_cache(c["kq"], c["ks"], c["km"], c["vq"], c["vs"], c["vm"],
                                  c["block_table"], c["seq_lens"], torch.float32, GROUP)


def test_gather_op_requires_eight_lane_groups():
    from vllm_ascend_quantized_kv_cache.ops.kivi_gather import kivi_dequant_gather_cache

    caches = [torch.zeros(2, KVH, HEAD, 2, dtype=torch.int32), torch.ones(2, KVH, HEAD, 2),
              torch.zeros(2, KVH, HEAD, 2), torch.zeros(2, 16, KVH, 4, dtype=torch.int32),
              torch.ones(2, 16, KVH, 4), torch.zeros(2, 16, KVH, 4)]
    with pytest.raises(RuntimeError, match="divisible by 8"):
        kivi_dequant_gather_cache(*caches, torch.arange(2).view(1, 2), torch.tensor([32]),
                                  torch.float32, 4)


GEOMETRIES = [(32, 2, 8, 16, 16), (64, 4, 16, 32, 32), (128, 8, 128, 128, 128),
              (128, 4, 32, 64, 64), (256, 2, 64, 64, 128)]


@pytest.mark.parametrize("head,kvh,group,block,residual", GEOMETRIES,
                         ids=[f"h{h}_g{g}_b{b}" for h, _, g, b, _ in GEOMETRIES])
def test_int4_pipeline_across_geometries(head, kvh, group, block, residual):
    tokens = residual + group + 8
    pages = -(-tokens // block) + 1
    layout = KiviByteCacheLayout(num_blocks=pages, block_size=block, num_kv_heads=kvh,
                                 head_size=head, group_size=group)
    kb = torch.zeros(pages, block, kvh, layout.bytes_per_token_head, dtype=torch.uint8)
    vb = torch.zeros_like(kb)
    impl = _make_impl(residual, head=head, kvh=kvh, group=group, block=block, num_blocks=pages)
    torch.manual_seed(41)
    q, k, v = (torch.randn(tokens, kvh, head) for _ in range(3))
    out = torch.zeros(tokens, kvh, head)
    md = _metadata(tokens, block_tables=torch.arange(pages).view(1, pages))
    impl.forward(None, q, k, v, (kb, vb), md, out)
    hk = ((tokens - 1) // residual) * residual
    hv = max(0, tokens - residual)
    ek = torch.cat([ref.fake_quant_key(k[:hk], group), k[hk:]])
    ev = torch.cat([ref.fake_quant_value(v[:hv], group), v[hv:]])
    gk, gv = impl._gather_dequant_kivi_paged_cache(md.block_tables, [tokens], torch.float32,
                                                   ["r"])
    assert torch.equal(gk, ek) and torch.equal(gv, ev)
    assert torch.isfinite(out).all() and out.abs().sum() > 0
    assert kivi_byte_cache_layout(kb, vb, num_kv_heads=kvh, head_size=head,
                                  group_size=group) == layout


def test_native_step_check_matches_the_python_checks():
    """kvq_kivi_step_check (the decode step's one-pass host check) raises as
    check_gather_metadata_host does and flags the rows suspect_rows flags."""
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.residual import KiviResidualRing
    from vllm_ascend_quantized_kv_cache.ops.kivi_layout import check_gather_metadata_host

    rng = np.random.default_rng(0)
    bs, nb, rows_n, window = 16, 24, 6, 8
    seen = {"ok": 0, "err": 0, "suspect": 0}
    for _ in range(400):
        ring = KiviResidualRing(rows_n, window, 2, 8, device="cpu")
        b = int(rng.integers(1, 6))
        maxb = int(rng.integers(1, 5))
        table = rng.integers(0, nb, size=(b, maxb))
        if rng.random() < 0.15:
            table[rng.integers(b), rng.integers(maxb)] = -1
        if rng.random() < 0.15:
            table[rng.integers(b), rng.integers(maxb)] = nb + int(rng.integers(0, 3))
        lens = rng.integers(0, maxb * bs + (3 if rng.random() < 0.1 else 1), size=b)
        rows = np.full(b, -1, dtype=np.int64)
        for i, r in enumerate(rng.permutation(rows_n)[:b]):
            if rng.random() < 0.8:
                rows[i] = r
        for side in (True, False):
            for i in range(b):
                if rows[i] < 0:
                    continue
                for lane in range(window + 1):
                    if rng.random() < 0.5:
                        continue
                    p = int(rng.integers(-1, int(lens[i]) + 2))
                    col = min(max(p, 0) // bs, maxb - 1)
                    good = table[i, col] * bs + max(p, 0) % bs
                    s = good if rng.random() < 0.9 else int(rng.integers(0, nb * bs))
                    ring.lane_slot[side][rows[i], lane] = s
                    ring.lane_pos[side][rows[i], lane] = p
        want_err = got_err = None
        want = got = None
        try:
            check_gather_metadata_host(table, lens.tolist(), max_blocks=maxb, num_blocks=nb,
                                       block_size=bs)
            have = rows >= 0
            idx = ring.suspect_rows(rows[have], lens[have], table[have], bs)
            want = np.flatnonzero(have)[idx]
        except RuntimeError as e:
            want_err = str(e)
        try:
            got = ring.step_check(rows, lens, table, num_blocks=nb, block_size=bs)
        except RuntimeError as e:
            got_err = str(e)
        assert want_err == got_err
        if want_err is None:
            assert np.array_equal(want, got)
            seen["suspect" if got.size else "ok"] += 1
        else:
            seen["err"] += 1
    assert min(seen.values()) > 10, seen


def test_forward_under_capture_is_refused_or_routed(monkeypatch):
    """KIVI has no graph path in the reference (``--enforce-eager``,
    ``docs/int4-host-integration.md:137-138``).  Under capture, forward()
    records only a capturable decode step created for the batch, and refuses
    anything else before the mirror or the caches change."""
    impl = _make_impl()
    monkeypatch.setattr(ab, "stream_capturing", lambda: True)
    k = torch.randn(1, KVH, HEAD)
    md = _metadata(1, attn_state=SimpleNamespace(name="DecodeOnly"), seq_lens_list=[5],
                   slot_mapping=torch.tensor([4]))
    q = torch.randn(1, KVH, HEAD)
    state = impl._ensure_kivi_residual_buffers().state()
    for name in ("DecodeOnly", "PrefillNoCache", "ChunkedPrefill"):
        md.attn_state = SimpleNamespace(name=name)
        with pytest.raises(RuntimeError, match="graph capture"):
            impl.forward(None, q, k, k, None, md, torch.zeros_like(q))
    assert impl._kivi_ring.state() == state and not impl.kivi_residual_req_to_row
    assert all(not impl.calls[c] for c in impl.calls)

    launched = []

    class _Graph:
        def launch(self, query, key, value, output):
            launched.append(query.shape[0])
            return output

    impl._kivi_capture_graphs = {1: _Graph()}
    md.attn_state = SimpleNamespace(name="DecodeOnly")
    out = torch.zeros_like(q)
    assert impl.forward(None, q, k, k, None, md, out) is out and launched == [1]


def test_plan_decode_step_rolls_back_when_a_later_stage_raises():
    """The decode step plans the whole batch on the mirror, then stages and
    launches; an error after the planning (here: staging) must leave the
    mirror exactly as it was, flushed key windows included."""
    impl = _make_impl(residual=GROUP, max_seqs=3)
    ring = impl._ensure_kivi_residual_buffers()
    rows = np.asarray([impl._get_kivi_residual_row(k, create=True) for k in ("a", "b")])
    bs = BLOCK
    # row a: a full key window (one aligned group) in block 0; row b: two tokens
    ring.load_row(int(rows[0]), is_key=True, slots=list(range(GROUP)))
    ring.load_row(int(rows[0]), is_key=False, slots=list(range(GROUP)))
    ring.load_row(int(rows[1]), is_key=True, slots=[bs, bs + 1])
    ring.load_row(int(rows[1]), is_key=False, slots=[bs, bs + 1])
    before = ring.state()
    slots = np.asarray([GROUP, bs + 2])
    with pytest.raises(RuntimeError, match="staging failed"):
        with impl._kivi_planning():
            jobs = ring.plan_decode_step(rows, slots, slots % bs, np.arange(2),
                                         block_size=bs, group_size=GROUP)
            assert jobs is not None and jobs.key_pack_src.size == GROUP
            assert ring.state() != before
            raise RuntimeError("staging failed")
    assert ring.state() == before


def test_page_tile_plan_of_two_rounds_at_16_kv_heads():
    """16 KV heads on 256 CUs (128 pieces a round): a plan of about 1.5
    rounds of cost has 128 pieces of the full step, then the last round as 256
    pieces of half of it; no first-half weighting (that is for one-round
    plans), so each group is within a step of its share."""
    from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
        PAGE_TILE,
        PIECE_MAX_COST,
        TAIL_POSITION_COST,
        DecodeSeq,
        plan_decode_pieces,
    )

    per_round = 256 * 8 // 16
    n = int(per_round * PIECE_MAX_COST * 1.5) // 64  # 1.5 rounds of cost over 64 requests
    seqs = [DecodeSeq(n, ((n - 1) // 128) * 128, n - 128, i, 0, 0) for i in range(64)]
    meta, work, pieces = plan_decode_pieces(seqs, 16, 256, tile=PAGE_TILE)
    assert len(pieces) - 1 == per_round + 2 * per_round
    cost = [
        sum(-(-(e - p) // PAGE_TILE) * PAGE_TILE if k == 0 else (e - p) * TAIL_POSITION_COST
            for _, p, e, k in work[pieces[i] : pieces[i + 1]].tolist())
        for i in range(len(pieces) - 1)
    ]
    step = sum(cost) / (2 * per_round)
    margin = PAGE_TILE + 2 * 32 * TAIL_POSITION_COST
    assert all(abs(c - step) <= margin for c in cost[:per_round])
    assert all(abs(c - step / 2) <= margin for c in cost[per_round:])
