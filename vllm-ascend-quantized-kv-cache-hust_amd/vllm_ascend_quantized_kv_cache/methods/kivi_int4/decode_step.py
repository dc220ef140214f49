# SPDX-License-Identifier: Apache-2.0
"""One KIVI INT4 decode step -- store, fused decode, combine -- from a host plan.

The reference's decode step (``pkg/methods/kivi_int4/attention_backend.py:
411-462, 813-836, 1193-1230``) walks every request's residual window in
Python, reads slots and block ids back from the device, and needs
``--enforce-eager`` (``docs/int4-host-integration.md:137-138``).  Here the
host plans the whole step from host integers -- the window mirror, the
request lengths, and the step's slots and block table as host arrays -- and
writes the plan into one pinned buffer:

* the store jobs (key-window flushes, value evictions, ring writes) with
  their counts, for ``kvq_kivi_store_planned``;
* the decode plan (per-request geometry, work items, pieces) from the native
  planner ``kvq_plan_kivi_decode``.

One asynchronous copy moves it to a persistent device buffer; two launches
read it.  Nothing in a step reads the device back, and with ``fixed``
capacities (the grid covers the capacity, the kernels read the counts and
the pieces from the buffer) the two launches can be captured once in a HIP
graph and replayed every step after the host has staged that step's plan
(``KiviDecodeGraph``).
"""

from __future__ import annotations

import numpy as np
import torch

from ...ops import _native
from ...ops.kivi_decode import (
    PAGE_TILE,
    WAVES_PER_CU,
    page_streaming_applies,
    plan_into,
    work_capacity,
)
from .residual import StepJobs

#: int64 words before the store job sections (the four counts)
_HEADER = 4


class StagedPlan:
    """Where a staged plan's parts sit in the device buffer, and its counts."""

    def __init__(self, counts, jobs_off: int, meta_off: int, work_off: int, pieces_off: int,
                 num_work: int, num_pieces: int, fixed: bool) -> None:
        self.counts = counts
        self.jobs_off = jobs_off
        self.meta_off = meta_off
        self.work_off = work_off
        self.pieces_off = pieces_off
        self.num_work = num_work
        self.num_pieces = num_pieces
        self.fixed = fixed


class DecodeStepBuffers:
    """Persistent device buffers of a decode step and the layouts of its plan.

    Fixed layout (a captured launch reads it, so every part sits at a
    capacity offset): int64 ``[n_key_pack, n_value_pack, n_key_ring,
    n_value_ring]``, the eight int64 job sections of
    ``kvq_kivi_store_planned``, then int32 ``seq_meta [batch, 8]``,
    ``work [work_cap, 4]`` and ``pieces [pieces_cap + 1]``.  Compact layout
    (an eager step, whose launches take the counts as arguments): the eight
    job sections at their exact sizes, then ``seq_meta``, ``work`` and
    ``pieces`` at theirs, so the copy moves only the bytes the step uses.

    Plans are written into a ring of pinned host buffers allocated once; a
    buffer is reused after the copy that last read it has completed (an
    event query; the ring is deep enough that the host does not wait).
    """

    STAGING = 4

    def __init__(self, device, *, batch: int, window: int, num_heads: int, head_size: int,
                 work_cap: int, pieces_cap: int) -> None:
        self.device = device
        self.batch = batch
        self.cap_key_pack = batch * window
        self.cap_value = batch
        self.work_cap = work_cap
        self.pieces_cap = pieces_cap
        words = _HEADER + 2 * self.cap_key_pack + 2 * batch + 4 * batch
        self.meta_off = -(-words * 8 // 16) * 16
        self.work_off = self.meta_off + batch * 8 * 4
        self.pieces_off = self.work_off + work_cap * 4 * 4
        self.nbytes = self.pieces_off + (pieces_cap + 1) * 4
        self.plan = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        ws = _native.lib().kvq_kivi_decode_workspace_bytes(max(1, work_cap), num_heads, head_size)
        self.workspace = torch.empty((ws + 3) // 4, dtype=torch.float32, device=device)
        self._host = [torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=True)
                      for _ in range(self.STAGING)]
        self._events = [torch.cuda.Event() for _ in range(self.STAGING)]
        self._used = [False] * self.STAGING
        self._next = 0
        self._pieces = np.zeros(pieces_cap + 1, dtype=np.int32)
        self.last_host: tuple[int, int] | None = None  # (host buffer, bytes) of the last stage

    def same_layout(self, other: "DecodeStepBuffers") -> bool:
        """Fixed-layout plans of ``other`` read the same here (same capacities)."""
        return (self.batch, self.cap_key_pack, self.cap_value, self.work_cap, self.pieces_cap,
                self.nbytes) == (other.batch, other.cap_key_pack, other.cap_value,
                                 other.work_cap, other.pieces_cap, other.nbytes)

    def copy_staged_from(self, src: "DecodeStepBuffers", index: int, nbytes: int) -> None:
        """Queue a copy of the plan ``src`` staged in its host buffer ``index``
        into this device buffer; the copy is recorded on ``src``'s event for
        that buffer, so ``src`` rewrites it only after the copy has read it."""
        self.plan[:nbytes].copy_(src._host[index][:nbytes], non_blocking=True)
        src._events[index].record()
        src._used[index] = True

    def fits(self, batch: int, work_cap: int, pieces_cap: int) -> bool:
        return batch <= self.batch and work_cap <= self.work_cap and pieces_cap <= self.pieces_cap

    def ptr(self, offset: int) -> int:
        return self.plan.data_ptr() + offset

    def _staging(self) -> tuple[int, np.ndarray]:
        i = self._next
        self._next = (i + 1) % self.STAGING
        if self._used[i] and not self._events[i].query():
            self._events[i].synchronize()  # the copy from four steps back
        return i, self._host[i].numpy()

    def _upload(self, i: int, nbytes: int) -> None:
        self.plan[:nbytes].copy_(self._host[i][:nbytes], non_blocking=True)
        self._events[i].record()
        self._used[i] = True

    def stage(self, jobs: StepJobs | None, seqs: np.ndarray, *, num_kv_heads: int,
              cu_count: int, mode: int, fixed: bool, tile: int = 0) -> StagedPlan:
        """Write a step's plan to pinned memory and queue its copy to ``plan``.

        ``mode`` / ``tile``: the planner's mode and, for pieces, its int4 tile
        (``step_plan_mode``).

        ``fixed``: the capacity layout, with the unused pieces filled with
        empty ranges, so a launch over all ``pieces_cap`` pieces (a captured
        one) runs exactly this plan.
        """
        i, h = self._staging()
        b = seqs.shape[0]
        arrays = () if jobs is None else (
            jobs.key_pack_src, jobs.key_pack_slot, jobs.value_pack_src, jobs.value_pack_slot,
            jobs.key_ring_src, jobs.key_ring_dst, jobs.value_ring_src, jobs.value_ring_dst)
        counts = (0, 0, 0, 0) if jobs is None else (
            jobs.key_pack_src.size, jobs.value_pack_src.size, jobs.key_ring_src.size,
            jobs.value_ring_src.size)
        if fixed:
            caps = (self.cap_key_pack,) * 2 + (self.cap_value,) * 2 + (self.batch,) * 4
            words = h[: self.meta_off].view(np.int64)
            words[:_HEADER] = counts
            off = _HEADER
            jobs_off = 0
            meta_off, work_off = self.meta_off, self.work_off
            work_cap = self.work_cap
        else:
            caps = tuple(a.size for a in arrays)
            off = 0
            jobs_off = 0
            meta_off = -(-sum(caps) * 8 // 16) * 16
            work_off = meta_off + b * 8 * 4
            # the workspace holds partials for work_cap items, whatever the layout
            work_cap = min(self.work_cap,
                           (self.nbytes - work_off) // 16 - (self.pieces_cap + 1 + 3) // 4)
            words = h[:meta_off].view(np.int64)
        for arr, cap in zip(arrays, caps):
            if arr.size > cap:
                raise RuntimeError("KIVI decode step: store jobs exceed the plan capacity.")
            words[off:off + arr.size] = arr
            off += cap
        meta = h[meta_off:work_off].view(np.int32).reshape(b, 8)
        work = h[work_off:work_off + work_cap * 16].view(np.int32).reshape(work_cap, 4)
        n, npc = plan_into(seqs, num_kv_heads, cu_count, mode, split_tokens=tile, meta=meta,
                           work=work, pieces=self._pieces)
        if fixed:
            if npc == 0:
                raise RuntimeError("KIVI decode step: a fixed launch needs a plan in pieces.")
            # a launch over the whole capacity finds empty items past the plan
            # (request 0, no positions: m = -inf into the item's own partial)
            work[n:] = 0
            pieces_off = self.pieces_off
            pieces = h[pieces_off:].view(np.int32)
            pieces[: npc + 1] = self._pieces[: npc + 1]
            pieces[npc + 1:] = n
            nbytes = self.nbytes
        else:
            pieces_off = work_off + n * 16
            h[pieces_off:pieces_off + 4 * (npc + 1)].view(np.int32)[:] = self._pieces[: npc + 1]
            nbytes = pieces_off + 4 * (npc + 1)
        self._upload(i, nbytes)
        self.last_host = (i, nbytes)  # where this plan sits in host memory
        return StagedPlan(counts, jobs_off, meta_off, work_off, pieces_off, n, npc, fixed)


class KiviDecodeLauncher:
    """The two launches of a decode step over a ``DecodeStepBuffers`` plan."""

    def __init__(self, impl) -> None:
        self.impl = impl

    def store(self, bufs: DecodeStepBuffers, staged: StagedPlan, key: torch.Tensor,
              value: torch.Tensor) -> None:
        impl = self.impl
        ring = impl._kivi_ring
        kq, ks, km, vq, vs, vm = impl._kivi_caches()
        lib = _native.lib()
        common = (_native.ptr(key), _native.ptr(value), _native.ptr(ring.key),
                  _native.ptr(ring.value), ring.rows * ring.ring_len,
                  _native.dtype_code(ring.dtype), ring.num_kv_heads, ring.head_size,
                  impl.kivi_group_size, impl._get_kivi_block_size())
        caches = (_native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq),
                  _native.ptr(vs), _native.ptr(vm), _native.stream_of(key))
        if staged.fixed:
            rc = lib.kvq_kivi_store_planned(*common, bufs.ptr(staged.jobs_off), bufs.cap_key_pack,
                                            bufs.cap_value, bufs.batch, *caches)
            _native.check(rc, "kvq_kivi_store_planned")
        else:
            if not any(staged.counts):
                return
            rc = lib.kvq_kivi_store(*common, bufs.ptr(staged.jobs_off), *staged.counts, *caches)
            _native.check(rc, "kvq_kivi_store")
        ring.written = True

    def decode(self, bufs: DecodeStepBuffers, staged: StagedPlan, query: torch.Tensor,
               block_table: torch.Tensor, out: torch.Tensor) -> None:
        impl = self.impl
        ring = impl._kivi_ring
        kq, ks, km, vq, vs, vm = impl._kivi_caches()
        batch, hq, d = query.shape
        num_work = bufs.work_cap if staged.fixed else staged.num_work
        num_pieces = bufs.pieces_cap if staged.fixed else staged.num_pieces
        rc = _native.lib().kvq_kivi_decode_attn(
            _native.ptr(query), _native.dtype_code(query.dtype), batch, hq, ring.num_kv_heads, d,
            float(impl.scale), _native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq),
            _native.ptr(vs), _native.ptr(vm), kq.shape[0], impl._get_kivi_block_size(),
            impl.kivi_group_size, _native.ptr(block_table), block_table.shape[1],
            bufs.ptr(staged.meta_off), bufs.ptr(staged.work_off), num_work,
            bufs.ptr(staged.pieces_off) if num_pieces else None, num_pieces,
            _native.ptr(ring.key), _native.ptr(ring.value), _native.dtype_code(ring.dtype),
            ring.ring_len, _native.ptr(bufs.workspace), _native.ptr(out), _native.stream_of(query),
        )
        _native.check(rc, "kvq_kivi_decode_attn")


def step_geometry_ok(impl, query: torch.Tensor) -> bool:
    """The planned store and the pieces decode cover this layer: head size 128,
    group 64 or 128, a 16-bit activation dtype shared with the ring, at most
    16 query heads per kv head, a power-of-two block size."""
    ring = impl._kivi_ring
    bs = impl._get_kivi_block_size()
    return (impl.head_size == 128 and impl.kivi_group_size in (64, 128)
            and query.dtype in (torch.bfloat16, torch.float16) and ring.dtype == query.dtype
            and impl.num_heads // impl.num_kv_heads <= 16 and bs & (bs - 1) == 0)


def step_plan_mode(impl, query: torch.Tensor, *, fixed: bool) -> tuple[int, int]:
    """``(mode, tile)`` of a decode step's plan: pieces on page bounds where the
    page-streaming decode covers the layer; else pieces on 64-position tiles
    for a fixed (captured) launch, the default plan for an eager one."""
    if page_streaming_applies(impl.num_heads, impl.num_kv_heads, impl.head_size,
                              impl._get_kivi_block_size(), impl.kivi_group_size, query.dtype,
                              impl._kivi_ring.dtype):
        return _native.KVQ_PLAN_PIECES, PAGE_TILE
    return (_native.KVQ_PLAN_PIECES if fixed else _native.KVQ_PLAN_DEFAULT), 0


def pieces_capacity(num_kv_heads: int, cu_count: int, rounds: int) -> int:
    # plans of two or more rounds cut the last round into twice as many pieces
    rounds = max(1, rounds)
    return max(1, cu_count * WAVES_PER_CU // max(1, num_kv_heads)) * (rounds + (rounds > 1))


def eager_capacities(batch: int, num_kv_heads: int, cu_count: int, seqs: np.ndarray
                     ) -> tuple[int, int]:
    """``(work_cap, pieces_cap)`` that any default plan of ``seqs`` fits."""
    total = int(seqs[:, 0].sum()) if seqs.size else 0
    work = work_capacity(batch, num_kv_heads, cu_count, total)
    return work, work


class _SharedGraphStep:
    """The last step a layer's ``KiviDecodeGraph.prepare`` planned, for the
    other layers' graphs of the same engine step (the graph-path twin of the
    eager path's shared step): the metadata object, the layer signature, the
    window mirror before and after, and where the staged plan sits in the
    planning graph's host memory."""

    __slots__ = ("md", "sig", "before", "after", "bufs", "host", "staged")

    last: "_SharedGraphStep | None" = None


class KiviDecodeGraph:
    """A decode step of one layer captured in a HIP graph and replayed per step.

    ``prepare(attn_metadata, key, value)`` runs the host half of a step: it
    replays the window rules on the mirror and stages the plan (the step's
    slots and block table must be host arrays, or come with host copies).
    ``launch(query, key, value, output)`` issues the store and the decode over
    the staged plan with fixed capacities, so the two launches captured once
    serve every later step::

        g = KiviDecodeGraph(impl, batch=32)
        g.prepare(md0, k0, v0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            g.launch(q_static, k_static, v_static, out_static)
        graph.replay()                         # step 0
        g.prepare(md1, k1, v1); (fill statics); graph.replay()   # step 1, ...

    The block table the kernels read is a persistent int32 copy that
    ``prepare`` refreshes (on the stream, before the replay).  A step whose
    windows need compaction (entries no longer live) cannot be replayed and
    raises; a host runs it eagerly through ``forward``.
    """

    def __init__(self, impl, batch: int, *, max_blocks: int, rounds: int = 1) -> None:
        from ...ops.kivi_decode import _cu_count

        impl._ensure_kivi_residual_buffers()
        dev = impl.k_quant_cache.device
        self.impl = impl
        self.cu_count = _cu_count(dev)
        pieces = pieces_capacity(impl.num_kv_heads, self.cu_count, rounds)
        self.bufs = DecodeStepBuffers(dev, batch=batch, window=impl.kivi_residual_length,
                                      num_heads=impl.num_heads, head_size=impl.head_size,
                                      work_cap=pieces + 4 * batch + 8, pieces_cap=pieces)
        self.table = torch.zeros((batch, max_blocks), dtype=torch.int32, device=dev)
        self.launcher = KiviDecodeLauncher(impl)
        self.staged: StagedPlan | None = None

    def prepare(self, attn_metadata, key: torch.Tensor, value: torch.Tensor) -> None:
        """Stage one step's plan for the next replay (outside any capture).

        Every check that can refuse the step runs before the window mirror
        moves, and the planning, staging and table refresh form one
        transaction: a step that raises leaves the mirror as it was.
        """
        from ...core.runtime import stream_capturing

        impl = self.impl
        if stream_capturing():
            raise RuntimeError(
                "KIVI decode graph: prepare() stages the step's plan from host memory and "
                "must run before a replay, not inside the capture."
            )
        b = len(attn_metadata.seq_lens_list)
        if b != self.bufs.batch:
            raise RuntimeError(
                f"KIVI decode graph was captured for batch {self.bufs.batch}, got {b}."
            )
        if attn_metadata.block_tables.shape[1] > self.table.shape[1]:
            raise RuntimeError("KIVI decode graph: block table wider than captured.")
        ring = impl._ensure_kivi_residual_buffers()
        ok = key.dtype in (torch.bfloat16, torch.float16) and value.dtype == key.dtype
        if ok and not ring.written:
            ring.adopt_dtype(key.dtype)  # a ring with no data takes the activation dtype
        if not ok or ring.dtype != key.dtype or not step_geometry_ok(impl, key):
            raise RuntimeError(
                "KIVI decode graph: the layer's geometry or activation dtype is not one the "
                "planned store and the pieces decode cover (head size 128, group 64 or 128, "
                "16-bit activations shared with the ring, at most 16 query heads per kv head, "
                "a power-of-two block size); run it eagerly through forward."
            )
        # another layer's graph planned this engine step from the same mirror:
        # take its plan (one host-to-device copy) instead of planning again
        sig = (impl.num_heads, impl.num_kv_heads, impl.head_size, impl.kivi_group_size,
               impl._get_kivi_block_size(), impl.kivi_residual_length, ring.rows, ring.dtype,
               key.dtype, key.device, int(impl.k_quant_cache.shape[0]), self.cu_count,
               torch.cuda.current_stream(key.device).cuda_stream)
        shared = _SharedGraphStep.last
        if (shared is not None and shared.md is attn_metadata and shared.sig == sig
                and shared.bufs is not self.bufs and shared.bufs.same_layout(self.bufs)
                and impl._kivi_mirror_matches(shared.before)):
            impl._kivi_mirror_load(shared.after)
            try:
                self.bufs.copy_staged_from(shared.bufs, *shared.host)
                table_dev = attn_metadata.block_tables[:b]
                rows, cols = table_dev.shape
                self.table[:rows, :cols].copy_(table_dev, non_blocking=True)
            except BaseException:
                impl._kivi_mirror_load(shared.before)
                raise
            self.staged = shared.staged
            return
        before = impl._kivi_mirror_snapshot()
        with impl._kivi_planning():
            plan = impl._plan_kivi_decode_step(attn_metadata, key, value, allow_compaction=False)
            if plan is None:
                raise RuntimeError(
                    "KIVI decode graph: this step is not one token per request with slots that "
                    "follow the block table; run it eagerly through forward."
                )
            jobs, seqs, table_dev = plan
            mode, tile = step_plan_mode(impl, key, fixed=True)
            staged = self.bufs.stage(jobs, seqs, num_kv_heads=impl.num_kv_heads,
                                     cu_count=self.cu_count, mode=mode, fixed=True, tile=tile)
            rows, cols = table_dev.shape
            self.table[:rows, :cols].copy_(table_dev, non_blocking=True)
        self.staged = staged
        rec = _SharedGraphStep()
        rec.md, rec.sig, rec.before, rec.after = attn_metadata, sig, before, impl._kivi_mirror_snapshot()
        rec.bufs, rec.host, rec.staged = self.bufs, self.bufs.last_host, staged
        _SharedGraphStep.last = rec

    def launch(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
               output: torch.Tensor) -> torch.Tensor:
        impl = self.impl
        if self.staged is None:
            raise RuntimeError("KIVI decode graph: call prepare() once before the capture.")
        b = self.bufs.batch
        q = query[:b].view(b, impl.num_heads, impl.head_size)
        out = output[:b].view(b, impl.num_heads, impl.head_size)
        self.launcher.store(self.bufs, self.staged, key[:b], value[:b])
        self.launcher.decode(self.bufs, self.staged, q, self.table, out)
        return output


__all__ = [
    "DecodeStepBuffers",
    "StagedPlan",
    "KiviDecodeGraph",
    "KiviDecodeLauncher",
    "eager_capacities",
    "pieces_capacity",
    "step_geometry_ok",
]
