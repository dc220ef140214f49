# SPDX-License-Identifier: Apache-2.0
"""The INT8 decode step -- quantize + scatter, fused decode, combine -- from a host plan.

The reference runs its INT8 decode eagerly, or, while the host captures a
graph, through the host's ``full_graph_fia`` (``pkg/methods/int8_dynamic/
attention_backend.py:97-104``).  Here a step's plan -- the new tokens' slots,
each request's geometry and the split-K work list -- is written into a
pinned host buffer and moved by one asynchronous copy into a persistent
device buffer that both launches read.  With fixed capacities (the work list
padded with empty items to its capacity, so the grid never changes) the two
launches are captured once in a HIP graph and replayed every step after the
host stages that step's plan (``Int8DecodeGraph``).
"""

from __future__ import annotations

import numpy as np
import torch

from ...ops import _native
from ...ops.int8_ops import int8_split_tokens, plan_int8_work


class Int8StepBuffers:
    """Device plan buffer (int64 slots ``[batch]``, int32 ``seq_meta [batch, 4]``,
    int32 ``work [work_cap, 4]``), the decode workspace, and a ring of pinned
    staging buffers reused once their copies have completed."""

    STAGING = 4

    def __init__(self, device, *, batch: int, work_cap: int, num_heads: int,
                 head_size: int) -> None:
        self.batch = batch
        self.work_cap = work_cap
        self.meta_off = -(-batch * 8 // 16) * 16
        self.work_off = self.meta_off + batch * 4 * 4
        self.nbytes = self.work_off + work_cap * 4 * 4
        self.plan = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        ws = _native.lib().kvq_int8_decode_workspace_bytes(max(1, work_cap), num_heads, head_size)
        self.workspace = torch.empty((ws + 3) // 4, dtype=torch.float32, device=device)
        self._host = [torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=True)
                      for _ in range(self.STAGING)]
        self._events = [torch.cuda.Event() for _ in range(self.STAGING)]
        self._used = [False] * self.STAGING
        self._next = 0

    def ptr(self, offset: int) -> int:
        return self.plan.data_ptr() + offset

    def stage(self, slots: np.ndarray | None, seq_lens: list[int], split_tokens: int, *,
              fixed: bool) -> int:
        """Stage a step's plan; returns the number of work items to launch
        (``work_cap`` when ``fixed``: the list is padded with empty items)."""
        i = self._next
        self._next = (i + 1) % self.STAGING
        if self._used[i] and not self._events[i].query():
            self._events[i].synchronize()  # the copy from four steps back
        h = self._host[i].numpy()
        b = len(seq_lens)
        if slots is not None:
            h[: 8 * b].view(np.int64)[:] = slots
        meta, work = plan_int8_work(seq_lens, split_tokens)
        n = work.shape[0]
        if n > self.work_cap or b > self.batch:
            raise RuntimeError("INT8 decode step: the plan exceeds the buffer capacity.")
        h[self.meta_off:self.meta_off + 16 * b].view(np.int32)[:] = meta.reshape(-1)
        w = h[self.work_off:self.nbytes].view(np.int32).reshape(self.work_cap, 4)
        w[:n] = work
        count = n
        if fixed:
            w[n:] = (0, 0, 0, 1)  # empty items: m = -inf into their own partial slot
            count = self.work_cap
        nbytes = self.work_off + 16 * count
        self.plan[:nbytes].copy_(self._host[i][:nbytes], non_blocking=True)
        self._events[i].record()
        self._used[i] = True
        return count


def launch_int8_step(impl, bufs: Int8StepBuffers, layer, query: torch.Tensor, key, value,
                     block_table: torch.Tensor, num_work: int, out: torch.Tensor) -> None:
    """Quantize + scatter the step's tokens (slots from the plan), then the
    fused decode and combine over the plan's work list."""
    lib = _native.lib()
    b, hq, d = query.shape
    kc, vc = impl.key_cache, impl.value_cache
    nb, bs = kc.shape[0], kc.shape[1]
    dtype = _native.dtype_code(query.dtype)
    stream = _native.stream_of(query)
    if key is not None:
        rc = lib.kvq_int8_quant_scatter(
            _native.ptr(key), _native.ptr(value), _native.dtype_code(key.dtype),
            _native.ptr(layer._int8_k_inv_scale), _native.ptr(layer._int8_v_inv_scale),
            bufs.ptr(0), _native.index_code(torch.int64), b, impl.num_kv_heads * d,
            _native.ptr(kc), _native.ptr(vc), nb, bs, stream)
        _native.check(rc, "kvq_int8_quant_scatter")
    rc = lib.kvq_int8_decode_attn(
        _native.ptr(query), dtype, b, hq, impl.num_kv_heads, d, float(impl.scale),
        _native.ptr(kc), _native.ptr(vc), nb, bs, _native.ptr(layer._int8_k_aq_scale),
        _native.ptr(layer._int8_v_aq_scale), _native.ptr(block_table), block_table.shape[1],
        bufs.ptr(bufs.meta_off), bufs.ptr(bufs.work_off), num_work, _native.ptr(bufs.workspace),
        _native.ptr(out), stream)
    _native.check(rc, "kvq_int8_decode_attn")


class Int8DecodeGraph:
    """An INT8 decode step of one layer, capturable once in a HIP graph.

    ``prepare(attn_metadata)`` stages the step's plan from host data (the
    slots from ``slot_mapping_cpu`` or ``slot_mapping``, the lengths from
    ``seq_lens_list``) and refreshes a persistent int32 copy of the block
    table; ``launch(query, key, value, output)`` quantizes and scatters the
    step's tokens and runs the decode over a work list of fixed capacity, so
    the launches captured once serve every later step with at most
    ``max_blocks * block_size`` positions per request.
    """

    def __init__(self, impl, layer, batch: int, *, max_blocks: int) -> None:
        kc = impl.key_cache
        if kc is None or not getattr(layer, "_int8_scales_ready", False):
            raise RuntimeError("INT8 decode graph: bind the cache and calibrate the scales first.")
        dev = kc.device
        bs = kc.shape[1]
        self.impl, self.layer, self.batch = impl, layer, batch
        self.max_len = max_blocks * bs
        # each step splits as an eager step does (int8_split_tokens, at
        # least 256 positions per item), so the capacity is the item count at
        # the smallest split
        work_cap = batch * (-(-self.max_len // 256)) + batch
        self.bufs = Int8StepBuffers(dev, batch=batch, work_cap=work_cap,
                                    num_heads=impl.num_heads, head_size=impl.head_size)
        self.table = torch.zeros((batch, max_blocks), dtype=torch.int32, device=dev)
        self.num_work = work_cap
        self.prepared = False

    def prepare(self, attn_metadata) -> None:
        from ...core.runtime import stream_capturing

        impl = self.impl
        if stream_capturing():
            raise RuntimeError(
                "INT8 decode graph: prepare() stages the step's plan from host memory and "
                "must run before a replay, not inside the capture."
            )
        lens = [int(x) for x in attn_metadata.seq_lens_list]
        if len(lens) != self.batch or max(lens) > self.max_len:
            raise RuntimeError("INT8 decode graph: the step does not fit the captured shape.")
        if attn_metadata.block_tables.shape[1] > self.table.shape[1]:
            raise RuntimeError("INT8 decode graph: block table wider than captured.")
        slots = impl._int8_host_slots(attn_metadata, len(lens))
        split = int8_split_tokens(sum(lens), impl.num_kv_heads, seq_lens=lens)
        self.num_work = self.bufs.stage(slots, lens, split, fixed=True)
        table = attn_metadata.block_tables[: self.batch]
        self.table[:, : table.shape[1]].copy_(table, non_blocking=True)
        self.prepared = True

    def launch(self, query, key, value, output) -> torch.Tensor:
        impl = self.impl
        if not self.prepared:
            raise RuntimeError("INT8 decode graph: call prepare() once before the capture.")
        b = self.batch
        q = query[:b].reshape(b, impl.num_heads, impl.head_size)
        out = output[:b].view(b, impl.num_heads, impl.head_size)
        launch_int8_step(impl, self.bufs, self.layer, q, key[:b], value[:b], self.table,
                         self.num_work, out)
        return output


__all__ = ["Int8DecodeGraph", "Int8StepBuffers", "launch_int8_step"]
