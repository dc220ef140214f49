# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 attention mixin (int4 paged history + full-precision residual window).

Role and behaviour follow ``AscendKiviInt4AttentionBackendMixin`` of the
reference (``pkg/methods/kivi_int4/attention_backend.py``, cited below as
``ab.py``): the adapter composes this mixin in front of the host's attention
implementation, ``forward`` owns the whole INT4 path, and every guard fails
closed with the reference's messages.  What changes is where the work runs:

* the residual windows live on the GPU (``KiviResidualRing``) with an exact
  host mirror, so the per-token window rules replay on the host without
  device reads and each step issues a few batched launches;
* packing, gather-dequant (with the residual overlay fused in), fused decode
  attention and dense prefill attention are the MI355X HIP kernels behind the
  ``_launch_*`` hooks (tests replace the hooks, the validations stay real).
"""

from __future__ import annotations

from contextlib import contextmanager
from typing import Any

import numpy as np
import torch

from ...core.runtime import stream_capturing
from .byte_cache import kivi_byte_cache_layout, kivi_caches_from_byte_tensors
from .geometry import validate_kivi_geometry
from .residual import KiviResidualRing, StorePlan
from .semantics import KiviInt4Semantics


def _attn_state_name(attn_metadata: Any) -> str:
    state = getattr(attn_metadata, "attn_state", None)
    if state is None:
        return "UNKNOWN"
    return getattr(state, "name", None) or str(state)


def _host_list(x: Any) -> list[int]:
    if isinstance(x, torch.Tensor):
        return [int(v) for v in x.tolist()]
    return [int(v) for v in x]


def _hook_replaced(impl: Any, name: str) -> bool:
    """True when ``name`` was overridden on the instance or by a subclass."""
    if name in vars(impl):
        return True
    return getattr(type(impl), name) is not getattr(AscendKiviInt4AttentionBackendMixin, name)


class _SharedStep:
    """The last decode step a layer planned, for the other layers of the step.

    A host calls every attention layer's ``forward`` with the same metadata
    object within one engine step, and layers that have seen the same steps
    hold the same window mirror, so the step's window plan, decode work list
    and staged device plan are the same for all of them; only the caches
    differ.  The layer that plans records what it planned from (``before``:
    the mirror and its row maps) and to (``after``), and the staged plan.  A
    later layer reuses the record only when the metadata object is the same,
    its geometry, dtypes, device and stream match, and its own mirror equals
    ``before`` exactly; it then takes ``after`` as its mirror and launches its
    own store and decode against the staged plan.
    """

    __slots__ = ("md", "sig", "before", "after", "bufs", "staged", "table", "b", "has_jobs")

    last: "_SharedStep | None" = None


def _gather_rows(src_a: Any, src_b: Any, src_index: Any) -> Any:
    """Rows ``src_index`` of ``[src_a ; src_b]`` (both viewed as ``[n, KVH, D]``)."""
    if src_index is None:
        return src_a
    n_a = src_a.shape[0]
    idx = src_index.long()
    out = torch.empty((idx.numel(), *src_a.shape[1:]), dtype=src_a.dtype, device=src_a.device)
    in_a = idx < n_a
    out[in_a] = src_a[idx[in_a]]
    if src_b is not None and not bool(in_a.all()):
        b = src_b.reshape(-1, *src_a.shape[1:]).to(src_a.dtype)
        out[~in_a] = b[idx[~in_a] - n_a]
    return out


class AscendKiviInt4AttentionBackendMixin:
    """KIVI INT4 (int4 history + full-precision residual window) attention path."""

    #: capturable decode steps by batch size (``kivi_decode_graph``)
    _kivi_capture_graphs: dict | None = None

    # ------------------------------------------------------------------
    # state (ab.py:50-133)
    # ------------------------------------------------------------------

    def _init_kivi_state(self, kv_cache_dtype: str | None, vllm_config: Any = None) -> None:
        self.enable_kivi = kv_cache_dtype in ("kivi_int4", "kivi")
        cache_config = getattr(vllm_config, "cache_config", None)
        group_size = getattr(cache_config, "kivi_group_size", 128)
        residual_length = getattr(cache_config, "kivi_residual_length", 128)
        self.kivi_group_size = group_size if isinstance(group_size, int) else 128
        self.kivi_residual_length = residual_length if isinstance(residual_length, int) else 128
        if self.enable_kivi:
            self._validate_kivi_geometry()
        self.kivi_bits = 4
        self.k_quant_cache = None
        self.k_scale_cache = None
        self.k_mn_cache = None
        self.v_quant_cache = None
        self.v_scale_cache = None
        self.v_mn_cache = None
        self._kivi_ring: KiviResidualRing | None = None
        self._kivi_bound_buffers = None
        scheduler_config = getattr(vllm_config, "scheduler_config", None)
        max_num_seqs = getattr(scheduler_config, "max_num_seqs", 128)
        self.kivi_max_num_seqs = (
            max_num_seqs if isinstance(max_num_seqs, int) and max_num_seqs > 0 else 128
        )
        self.kivi_residual_req_to_row: dict[str, int] = {}
        self.kivi_residual_row_to_req: list[str | None] = []
        self.kivi_residual_free_rows: list[int] = []
        # device-to-host reads of step metadata (0 while the host supplies
        # its own copies of slot_mapping and block_tables)
        self.kivi_host_reads = 0
        self._kivi_step_bufs = None
        self._kivi_capture_graphs = None

    def _validate_kivi_geometry(self) -> None:
        validate_kivi_geometry(
            head_size=self.head_size,
            group_size=self.kivi_group_size,
            residual_length=self.kivi_residual_length,
        )

    def _kivi_sem(self) -> KiviInt4Semantics:
        geometry = (self.head_size, self.kivi_group_size, self.kivi_residual_length)
        memo = getattr(self, "_kivi_sem_memo", None)
        if memo is not None and memo[0] == geometry:
            return memo[1]
        sem = KiviInt4Semantics(self)
        self._kivi_sem_memo = (geometry, sem)
        return sem

    def _kivi_caches(self) -> tuple[torch.Tensor, ...]:
        return (
            self.k_quant_cache,
            self.k_scale_cache,
            self.k_mn_cache,
            self.v_quant_cache,
            self.v_scale_cache,
            self.v_mn_cache,
        )

    def _check_kivi_cache_bound(self) -> None:
        if any(t is None for t in self._kivi_caches()):
            raise RuntimeError("KIVI cache tensors are not bound.")

    def _get_kivi_block_size(self) -> int:
        kq = self.k_quant_cache
        if kq is not None and kq is getattr(self, "_kivi_bs_of", None):
            return self._kivi_bs  # the bound key codes' page geometry, as last read
        self._check_kivi_cache_bound()
        self._kivi_bs, self._kivi_bs_of = kq.shape[-1] * 8, kq
        return self._kivi_bs

    # ------------------------------------------------------------------
    # cache binding (ab.py:135-175)
    # ------------------------------------------------------------------

    def _bind_kivi_cache(self, kv_cache: Any) -> None:
        """Bind the paged cache: two host byte buffers (sliced into six views) or six tensors."""
        if kv_cache is None:
            return
        if not isinstance(kv_cache, list | tuple):
            raise RuntimeError(
                "KIVI INT4 kv_cache must be a 2-tuple of byte buffers or a "
                f"6-tuple, got {type(kv_cache)}."
            )
        if len(kv_cache) == 0:
            return
        last = getattr(self, "_kivi_bound_objs", None)
        if (last is not None and len(kv_cache) == 2 and kv_cache[0] is last[0]
                and kv_cache[1] is last[1] and kv_cache[0].data_ptr() == last[2]
                and kv_cache[1].data_ptr() == last[3] and kv_cache[0].shape == last[4]
                and kv_cache[1].shape == last[5]
                and (self.num_kv_heads, self.head_size, self.kivi_group_size) == last[6]
                and self._kivi_ring is not None):
            return  # the very buffer objects bound last time, unchanged
        self._kivi_bound_objs = None
        if len(kv_cache) == 2:
            objs = (kv_cache[0], kv_cache[1], kv_cache[0].data_ptr(), kv_cache[1].data_ptr(),
                    kv_cache[0].shape, kv_cache[1].shape,
                    (self.num_kv_heads, self.head_size, self.kivi_group_size))
            # the same two buffers as the last call: the six views are still
            # bound (they hold the buffers' storage, so no other allocation
            # can have taken these addresses)
            bound = (kv_cache[0].data_ptr(), kv_cache[1].data_ptr(), tuple(kv_cache[0].shape),
                     tuple(kv_cache[1].shape), kv_cache[0].dtype, kv_cache[1].dtype,
                     self.num_kv_heads, self.head_size, self.kivi_group_size)
            if (bound == getattr(self, "_kivi_bound_buffers", None) and self._kivi_ring is not None
                    and all(t is not None for t in self._kivi_caches())):
                self._kivi_bound_objs = objs
                return
            layout = kivi_byte_cache_layout(
                kv_cache[0],
                kv_cache[1],
                num_kv_heads=self.num_kv_heads,
                head_size=self.head_size,
                group_size=self.kivi_group_size,
            )
            kv_cache = kivi_caches_from_byte_tensors(kv_cache[0], kv_cache[1], layout)
            self._kivi_bound_buffers = bound
        else:
            objs = None
            self._kivi_bound_buffers = None
        if len(kv_cache) != 6:
            raise RuntimeError(
                "KIVI INT4 kv_cache must be a 2-tuple of byte buffers or a "
                "6-tuple: (k_quant, k_scale, k_mn, v_quant, v_scale, v_mn)."
            )
        (
            self.k_quant_cache,
            self.k_scale_cache,
            self.k_mn_cache,
            self.v_quant_cache,
            self.v_scale_cache,
            self.v_mn_cache,
        ) = kv_cache
        self._ensure_kivi_residual_buffers()
        self._kivi_bound_objs = objs

    # ------------------------------------------------------------------
    # residual rows (ab.py:181-259)
    # ------------------------------------------------------------------

    def _ensure_kivi_residual_buffers(self) -> KiviResidualRing:
        if self._kivi_ring is not None:
            return self._kivi_ring
        self._check_kivi_cache_bound()
        rows = self.kivi_max_num_seqs
        self._kivi_ring = KiviResidualRing(
            rows,
            self.kivi_residual_length,
            self.num_kv_heads,
            self.head_size,
            device=self.k_quant_cache.device,
            dtype=self.k_scale_cache.dtype,
        )
        self.kivi_residual_req_to_row = {}
        self.kivi_residual_row_to_req = [None] * rows
        self.kivi_residual_free_rows = list(range(rows - 1, -1, -1))
        return self._kivi_ring

    # the ring tensors and window state under the reference's attribute names
    @property
    def kivi_residual_key_cache(self) -> torch.Tensor | None:
        return None if self._kivi_ring is None else self._kivi_ring.key

    @property
    def kivi_residual_value_cache(self) -> torch.Tensor | None:
        return None if self._kivi_ring is None else self._kivi_ring.value

    @property
    def kivi_residual_key_start(self) -> list[int]:
        return self._ensure_kivi_residual_buffers().start[True]

    @property
    def kivi_residual_key_len(self) -> list[int]:
        return self._ensure_kivi_residual_buffers().length[True]

    @property
    def kivi_residual_value_start(self) -> list[int]:
        return self._ensure_kivi_residual_buffers().start[False]

    @property
    def kivi_residual_value_len(self) -> list[int]:
        return self._ensure_kivi_residual_buffers().length[False]

    def _get_kivi_req_keys(self, req_ids: list[str] | None, num_reqs: int) -> list[str]:
        if req_ids is not None and len(req_ids) >= num_reqs:
            return [str(r) for r in req_ids[:num_reqs]]
        return [f"__kivi_batch_row_{i}" for i in range(num_reqs)]

    def _get_kivi_residual_row(self, req_key: str, *, create: bool) -> int | None:
        self._ensure_kivi_residual_buffers()
        row = self.kivi_residual_req_to_row.get(req_key)
        if row is not None or not create:
            return row
        if not self.kivi_residual_free_rows:
            raise RuntimeError(
                "KIVI residual rows are exhausted. "
                f"max_num_seqs={self.kivi_max_num_seqs}, req_id={req_key}."
            )
        row = self.kivi_residual_free_rows.pop()
        self.kivi_residual_req_to_row[req_key] = row
        self.kivi_residual_row_to_req[row] = req_key
        return row

    def _release_kivi_residual_row(self, req_key: str) -> None:
        row = self.kivi_residual_req_to_row.pop(req_key, None)
        if row is None:
            return
        self.kivi_residual_row_to_req[row] = None
        self._kivi_ring.reset_row(row)
        self.kivi_residual_free_rows.append(row)

    def _release_finished_kivi_residual_rows(self, finished_req_keys: set[str]) -> None:
        for key in finished_req_keys:
            self._release_kivi_residual_row(key)

    # ------------------------------------------------------------------
    # window queries (ab.py:286-326, 485-492)
    # ------------------------------------------------------------------

    def _get_kivi_residual_lanes(self, row_idx: int, *, is_key: bool) -> list[int]:
        return self._ensure_kivi_residual_buffers().lanes(row_idx, is_key=is_key)

    def _collect_kivi_residual_window(
        self,
        req_key: str,
        *,
        is_key: bool,
        target_dtype: Any | None = None,
        target_device: Any | None = None,
    ) -> tuple[list[int], torch.Tensor | None]:
        """``(slots, rows)`` of a request's window in FIFO order."""
        ring = self._ensure_kivi_residual_buffers()
        row = self._get_kivi_residual_row(req_key, create=False)
        if row is None:
            return [], None
        lanes = ring.lanes(row, is_key=is_key)
        if not lanes:
            return [], None
        lane_t = torch.tensor(lanes, dtype=torch.long, device=ring.device)
        rows = ring.tensor(is_key)[row].index_select(0, lane_t)
        if target_dtype is not None or target_device is not None:
            rows = rows.to(
                device=target_device or rows.device, dtype=target_dtype or rows.dtype
            )
        return ring.window_slots(row, is_key=is_key), rows

    def _has_kivi_residual_entry(self, slot: int, *, req_key: str, is_key: bool) -> bool:
        row = self._get_kivi_residual_row(req_key, create=False)
        if row is None:
            return False
        return self._kivi_ring.holds(row, int(slot), is_key=is_key)

    # ------------------------------------------------------------------
    # window writes (ab.py:377-462, 562-674)
    # ------------------------------------------------------------------

    def _kivi_mirror_snapshot(self) -> tuple:
        """The window mirror and the request-row maps, copied."""
        return (self._kivi_ring.snapshot(), dict(self.kivi_residual_req_to_row),
                list(self.kivi_residual_row_to_req), list(self.kivi_residual_free_rows))

    def _kivi_mirror_matches(self, snap: tuple) -> bool:
        ring, req_to_row, row_to_req, free_rows = snap
        return (self.kivi_residual_req_to_row == req_to_row
                and self.kivi_residual_row_to_req == row_to_req
                and self.kivi_residual_free_rows == free_rows and self._kivi_ring.matches(ring))

    def _kivi_mirror_load(self, snap: tuple) -> None:
        ring, req_to_row, row_to_req, free_rows = snap
        self._kivi_ring.load(ring)
        self.kivi_residual_req_to_row = dict(req_to_row)
        self.kivi_residual_row_to_req = list(row_to_req)
        self.kivi_residual_free_rows = list(free_rows)

    @contextmanager
    def _kivi_planning(self):
        """All-or-nothing planning of one store batch.

        When planning or launching raises, the ring mirror rows touched by
        the batch get their old state back and rows the batch created are
        released, so a caller that survives the error still sees the state
        the device holds.
        """
        ring = self._ensure_kivi_residual_buffers()
        before = set(self.kivi_residual_req_to_row)
        try:
            with ring.transaction():
                yield ring
        except BaseException:
            for key in set(self.kivi_residual_req_to_row) - before:
                self._release_kivi_residual_row(key)
            raise

    def _execute_kivi_plan(self, plan: StorePlan, key: Any, value: Any) -> None:
        if plan.empty():
            return
        # the one-launch store stands in for the three launch hooks below, so
        # it is used only while none of them (or the hooks they defer to) is
        # replaced
        hooks = ("_launch_kivi_key_pack", "_launch_kivi_value_pack",
                 "_launch_kivi_key_pack_rows", "_launch_kivi_value_pack_rows",
                 "_launch_kivi_ring_write", "_launch_kivi_store")
        store = None if any(_hook_replaced(self, h) for h in hooks) else self._launch_kivi_store
        self._kivi_ring.execute(
            plan,
            key,
            value,
            pack_key=self._launch_kivi_key_pack_rows,
            pack_value=self._launch_kivi_value_pack_rows,
            ring_write=self._launch_kivi_ring_write,
            store=store,
        )

    def _adopt_ring_dtype(self, *tensors: Any) -> None:
        ring = self._ensure_kivi_residual_buffers()
        for t in tensors:
            if t is not None:
                ring.adopt_dtype(t.dtype)

    def _store_kivi_residual_entries(
        self, values: torch.Tensor, slots: torch.Tensor, *, req_key: str, is_key: bool
    ) -> None:
        """Append tokens to a request's window; a full window flushes first.

        In-place overwrite for held slots; keys flush the whole window, values
        evict their single oldest entry (``ab.py:411-462``).
        """
        if values.numel() == 0 or slots.numel() == 0:
            return
        self._adopt_ring_dtype(values)
        slot_list = _host_list(slots)
        with self._kivi_planning() as ring:
            row = self._get_kivi_residual_row(req_key, create=True)
            plan = StorePlan()
            ring.plan_store(
                plan, row, slot_list, list(range(len(slot_list))), is_key=is_key,
                block_size=self._get_kivi_block_size(), group_size=self.kivi_group_size,
            )
            self._execute_kivi_plan(plan, values if is_key else None,
                                    None if is_key else values)

    def _flush_kivi_residual_prefix(self, req_key: str, *, is_key: bool, count: int) -> None:
        row = self._get_kivi_residual_row(req_key, create=False)
        if row is None:
            return
        with self._kivi_planning() as ring:
            plan = StorePlan()
            ring.flush_prefix(
                plan, row, count, is_key=is_key, block_size=self._get_kivi_block_size(),
                group_size=self.kivi_group_size,
            )
            self._execute_kivi_plan(plan, None, None)

    def _request_spans(self, slot_mapping: Any, actual_seq_qlen: Any
                       ) -> tuple[list[tuple[int, int]], int]:
        """``([(start, end)] per request, number of requests)`` from cumulative lengths.

        Same walk as ``ab.py:578-590``: spans stop at the slot mapping's end and
        empty spans keep their request index.
        """
        if isinstance(actual_seq_qlen, torch.Tensor):
            actual_seq_qlen = actual_seq_qlen.tolist()
        max_tokens = int(slot_mapping.shape[0])
        spans, prev = [], 0
        for q_end in actual_seq_qlen:
            q_end = min(int(q_end), max_tokens)
            if prev >= max_tokens:
                break
            spans.append((prev, q_end))
            prev = q_end
        return spans, len(actual_seq_qlen)

    @staticmethod
    def _span_positions(start: int, end: int, rows: list[int], seq_lens: Any,
                        i: int) -> list[int] | None:
        """Positions of a request's tokens when its length is known: the
        step's ``end - start`` tokens are the request's last ones."""
        if seq_lens is None or i >= len(seq_lens):
            return None
        first = int(seq_lens[i]) - (end - start)
        return [first + t - start for t in rows]

    def _write_kivi_cache(
        self, key: Any, value: Any, slot_mapping: Any, req_ids: list[str] | None,
        actual_seq_qlen: list[int] | Any, seq_lens: Any = None,
    ) -> None:
        """Token-by-token residual writes for every request of the step (``ab.py:562-606``).

        ``seq_lens`` (optional) gives each request's length after the step, so
        the mirror records every window token's position.
        """
        if key is None or value is None or slot_mapping is None:
            return
        spans, num_reqs = self._request_spans(slot_mapping, actual_seq_qlen)
        if not spans:
            return
        self._check_kivi_cache_bound()
        self._adopt_ring_dtype(key, value)
        slots = _host_list(slot_mapping)
        keys = self._get_kivi_req_keys(req_ids, num_reqs)
        bs, g = self._get_kivi_block_size(), self.kivi_group_size
        with self._kivi_planning() as ring:
            plan = StorePlan()
            for i, (start, end) in enumerate(spans):
                if end <= start:
                    continue
                rows = [t for t in range(start, end) if slots[t] >= 0]
                if not rows:
                    continue
                row = self._get_kivi_residual_row(keys[i], create=True)
                req_slots = [slots[t] for t in rows]
                pos = self._span_positions(start, end, rows, seq_lens, i)
                ring.plan_store(plan, row, req_slots, rows, is_key=True,
                                block_size=bs, group_size=g, positions=pos)
                ring.plan_store(plan, row, req_slots, rows, is_key=False,
                                block_size=bs, group_size=g, positions=pos)
            self._execute_kivi_plan(plan, key, value)

    def _write_kivi_prefill_cache(
        self, key: Any, value: Any, slot_mapping: Any, req_ids: list[str] | None,
        actual_seq_qlen: list[int] | Any, seq_lens: Any = None,
    ) -> None:
        """Bulk prefill: ``floor(n/R)*R`` tokens straight to history, the rest to the window.

        ``ab.py:608-674``.
        """
        if key is None or value is None or slot_mapping is None:
            return
        spans, num_reqs = self._request_spans(slot_mapping, actual_seq_qlen)
        if not spans:
            return
        self._check_kivi_cache_bound()
        slots = _host_list(slot_mapping)
        keys = self._get_kivi_req_keys(req_ids, num_reqs)
        r = self.kivi_residual_length
        bs, g = self._get_kivi_block_size(), self.kivi_group_size
        ring = self._ensure_kivi_residual_buffers()
        na = ring.rows * ring.ring_len
        self._adopt_ring_dtype(key, value)
        with self._kivi_planning():
            plan = StorePlan()
            for i, (start, end) in enumerate(spans):
                if end <= start:
                    continue
                rows = [t for t in range(start, end) if slots[t] >= 0]
                if not rows:
                    continue
                flush = (len(rows) // r) * r
                if flush:
                    self._check_key_flush(key, [slots[t] for t in rows[:flush]])
                    for side in (plan.key, plan.value):
                        side.pack_src.extend(na + t for t in rows[:flush])
                        side.pack_slots.extend(slots[t] for t in rows[:flush])
                if flush < len(rows):
                    row = self._get_kivi_residual_row(keys[i], create=True)
                    rest = rows[flush:]
                    rest_slots = [slots[t] for t in rest]
                    pos = self._span_positions(start, end, rest, seq_lens, i)
                    ring.plan_store(plan, row, rest_slots, rest, is_key=True, block_size=bs,
                                    group_size=g, positions=pos)
                    ring.plan_store(plan, row, rest_slots, rest, is_key=False, block_size=bs,
                                    group_size=g, positions=pos)
            self._execute_kivi_plan(plan, key, value)

    def _check_key_flush(self, key: Any, slots: list[int]) -> None:
        """Validation of a key flush before any launch (``ab.py:676-726``)."""
        if key.shape[-1] != self.head_size:
            raise RuntimeError(
                "KIVI INT4 key head_size must match attention head_size "
                f"({self.head_size}), got {key.shape[-1]}."
            )
        if len(slots) % self.kivi_group_size != 0:
            raise RuntimeError(
                "KIVI key flush must contain whole token groups, got "
                f"{len(slots)} tokens for group_size={self.kivi_group_size}."
            )
        if self.head_size % 8 != 0:
            raise RuntimeError(
                f"KIVI INT4 int32 packing requires head_size ({self.head_size}) "
                "to be divisible by 8."
            )
        if self.kivi_group_size % 8 != 0:
            raise RuntimeError(
                "KIVI INT4 key packing requires kivi_group_size "
                f"({self.kivi_group_size}) to be divisible by 8."
            )
        block_size = self._get_kivi_block_size()
        if block_size % self.kivi_group_size != 0:
            raise RuntimeError(
                f"KIVI INT4 key cache requires block_size ({block_size}) to be "
                f"divisible by kivi_group_size ({self.kivi_group_size})."
            )
        if not self._kivi_sem().is_aligned_key_window(slots, block_size):
            raise RuntimeError("KIVI key flush requires contiguous aligned token groups.")

    def _write_kivi_key_quant_cache(self, key: Any, slot_mapping: Any) -> None:
        """Pack whole key groups into history after the reference's checks."""
        self._check_kivi_cache_bound()
        if key is None or slot_mapping is None:
            return
        slots = _host_list(slot_mapping)
        keep = [i for i, s in enumerate(slots) if s >= 0]
        if not keep:
            return
        if len(keep) != len(slots):
            idx = torch.tensor(keep, dtype=torch.long, device=key.device)
            key = key.index_select(0, idx)
            slots = [slots[i] for i in keep]
        self._check_key_flush(key, slots)
        slot_t = torch.tensor(slots, dtype=torch.long).to(self.k_quant_cache.device)
        self._launch_kivi_key_pack(key.to(self.k_scale_cache.dtype).contiguous(), slot_t)

    def _write_kivi_value_quant_cache(self, value: Any, slot_mapping: Any) -> None:
        self._check_kivi_cache_bound()
        if value is None or slot_mapping is None:
            return
        slots = _host_list(slot_mapping)
        keep = [i for i, s in enumerate(slots) if s >= 0]
        if not keep:
            return
        head_size = value.shape[-1]
        if head_size != self.head_size:
            raise RuntimeError(
                "KIVI INT4 value head_size must match attention head_size "
                f"({self.head_size}), got {head_size}."
            )
        if head_size % self.kivi_group_size != 0:
            raise RuntimeError(
                f"KIVI INT4 value head_size ({head_size}) must be divisible by "
                f"kivi_group_size ({self.kivi_group_size})."
            )
        if head_size % 8 != 0:
            raise RuntimeError(
                f"KIVI INT4 int32 packing requires head_size ({head_size}) "
                "to be divisible by 8."
            )
        if self.kivi_group_size % 8 != 0:
            raise RuntimeError(
                "KIVI INT4 value packing requires kivi_group_size "
                f"({self.kivi_group_size}) to be divisible by 8."
            )
        if len(keep) != len(slots):
            idx = torch.tensor(keep, dtype=torch.long, device=value.device)
            value = value.index_select(0, idx)
            slots = [slots[i] for i in keep]
        slot_t = torch.tensor(slots, dtype=torch.long).to(self.v_quant_cache.device)
        self._launch_kivi_value_pack(value.to(self.v_scale_cache.dtype).contiguous(), slot_t)

    # ------------------------------------------------------------------
    # launch hooks (HIP kernels; tests replace them)
    # ------------------------------------------------------------------

    def _launch_kivi_key_pack(self, key: Any, slots: Any) -> None:
        """Pack ``key[T, KVH, D]`` into history at ``slots`` (``ab.py:728-739``)."""
        from ...ops.kivi_pack import kivi_pack_key_cache

        kivi_pack_key_cache(key, slots, self.k_quant_cache, self.k_scale_cache,
                            self.k_mn_cache, self.kivi_group_size)

    def _launch_kivi_value_pack(self, value: Any, slots: Any) -> None:
        """Pack ``value[T, KVH, D]`` into history at ``slots`` (``ab.py:779-790``)."""
        from ...ops.kivi_pack import kivi_pack_value_cache

        kivi_pack_value_cache(value, slots, self.v_quant_cache, self.v_scale_cache,
                              self.v_mn_cache, self.kivi_group_size)

    def _launch_kivi_key_pack_rows(self, src_a: Any, src_b: Any, src_index: Any,
                                   slots: Any) -> None:
        """Pack rows picked from ``[ring ; step input]`` in one launch (flush path).

        If the reference-signature hook ``_launch_kivi_key_pack`` has been
        replaced, the rows are materialized (cast to the scale dtype, as the
        reference hands them over) and passed to it instead.
        """
        if _hook_replaced(self, "_launch_kivi_key_pack"):
            rows = _gather_rows(src_a, src_b, src_index).to(self.k_scale_cache.dtype)
            return self._launch_kivi_key_pack(rows, slots)
        from ...ops.kivi_pack import pack_key_rows

        pack_key_rows(src_a, src_b, src_index, slots, self.k_quant_cache, self.k_scale_cache,
                      self.k_mn_cache, self.kivi_group_size)

    def _launch_kivi_value_pack_rows(self, src_a: Any, src_b: Any, src_index: Any,
                                     slots: Any) -> None:
        """Value counterpart of ``_launch_kivi_key_pack_rows``."""
        if _hook_replaced(self, "_launch_kivi_value_pack"):
            rows = _gather_rows(src_a, src_b, src_index).to(self.v_scale_cache.dtype)
            return self._launch_kivi_value_pack(rows, slots)
        from ...ops.kivi_pack import pack_value_rows

        pack_value_rows(src_a, src_b, src_index, slots, self.v_quant_cache, self.v_scale_cache,
                        self.v_mn_cache, self.kivi_group_size)

    def _launch_kivi_ring_write(self, src: Any, src_rows: Any, dst_rows: Any, is_key: bool) -> None:
        from ...ops.kivi_pack import ring_write

        ring_write(self._kivi_ring.tensor(is_key), src, src_rows, dst_rows)

    def _launch_kivi_store(self, key: Any, value: Any, jobs: Any, counts: Any) -> bool:
        """A whole hazard-free store batch in one launch (``kvq_kivi_store``);
        False when the geometry needs the separate pack and ring launches."""
        from ...ops.kivi_pack import kivi_store

        ring = self._kivi_ring
        caches = (self.k_quant_cache, self.k_scale_cache, self.k_mn_cache,
                  self.v_quant_cache, self.v_scale_cache, self.v_mn_cache)
        return kivi_store(key, value, ring.key, ring.value, jobs, counts, caches,
                          self.kivi_group_size)

    def _launch_kivi_gather(self, block_table: Any, cu_seqlens: Any, total: int,
                            target_dtype: Any, ring_meta: Any) -> tuple[Any, Any]:
        from ...ops.kivi_gather import gather_dequant_with_residual

        return gather_dequant_with_residual(
            self._kivi_caches(), block_table, cu_seqlens, total, target_dtype,
            self.kivi_group_size, ring_meta, self._kivi_ring.key, self._kivi_ring.value,
        )

    def _launch_kivi_decode(self, query: Any, block_table: Any, seqs: list, out: Any) -> Any:
        from ...ops.kivi_decode import kivi_decode_attention

        return kivi_decode_attention(
            query, self._kivi_caches(), block_table, seqs, self._kivi_ring.key,
            self._kivi_ring.value, self.scale, self.kivi_group_size, out=out,
        )

    def _launch_dense_attention(self, query: Any, key: Any, value: Any, q_lens: list[int],
                                kv_lens: list[int], causal: bool, out: Any) -> Any:
        from ...ops.attention import prefill_attention

        return prefill_attention(query, key, value, q_lens, kv_lens, self.scale, causal, out=out)

    # ------------------------------------------------------------------
    # per-step window sync (ab.py:813-836)
    # ------------------------------------------------------------------

    def _host_table(self, block_table: Any) -> np.ndarray:
        """The block table as a host int64 array (one device read when the
        caller hands over a device tensor)."""
        if isinstance(block_table, torch.Tensor):
            if block_table.device.type != "cpu":
                self.kivi_host_reads += 1
                block_table = block_table.cpu()
            return block_table.numpy().astype(np.int64, copy=False)
        return np.asarray(block_table, dtype=np.int64)

    def _host_array(self, attn_metadata: Any, name: str) -> np.ndarray:
        """A metadata field as a host array, preferring the host's own copy
        ``<name>_cpu`` (vLLM builds every step's slot mapping and block
        table on the host before copying them to the device), so that a
        step reads nothing back from the device."""
        host = getattr(attn_metadata, f"{name}_cpu", None)
        x = host if host is not None else getattr(attn_metadata, name)
        if isinstance(x, torch.Tensor):
            if x.device.type != "cpu":
                self.kivi_host_reads += 1
                x = x.cpu()
            return x.numpy()
        return np.asarray(x)

    def _sync_kivi_residual_windows(
        self, block_table: Any, seq_lens: list[int], req_ids: list[str] | None,
        finished_req_ids: set[str] | None = None,
    ) -> None:
        """Release finished rows and drop window entries a request no longer owns.

        An entry is live when the first table column holding its block, times
        the block size plus its offset, is below the request's length
        (``ab.py:813-836``).  Entries whose recorded position still maps to
        their slot are live (``KiviResidualRing.suspect_rows``); only the
        windows with other entries are checked entry by entry.
        """
        keys = self._get_kivi_req_keys(req_ids, len(seq_lens))
        if finished_req_ids:
            self._release_finished_kivi_residual_rows({str(r) for r in finished_req_ids})
        ring = self._ensure_kivi_residual_buffers()
        bs = self._get_kivi_block_size()
        idx, rows = [], []
        for i, key in enumerate(keys):
            row = self.kivi_residual_req_to_row.get(key)
            if row is not None and (ring.length[True][row] or ring.length[False][row]):
                idx.append(i)
                rows.append(row)
        if not rows:
            return
        table = self._host_table(block_table)
        lens = np.asarray([int(seq_lens[i]) for i in idx], dtype=np.int64)
        sub = np.full((len(idx), max(1, table.shape[1] if table.ndim == 2 else 1)), -1,
                      dtype=np.int64)
        for j, i in enumerate(idx):
            if i < len(table):
                sub[j, : table.shape[1]] = table[i]
        for j in ring.suspect_rows(np.asarray(rows), lens, sub, bs).tolist():
            self._check_window_entries(rows[j], sub[j], int(lens[j]), bs)

    def _check_window_entries(self, row: int, table_row: np.ndarray, n: int, bs: int) -> None:
        """The reference's per-entry liveness rule for one request's windows;
        live entries get their position recorded, dead ones are dropped."""
        ring = self._kivi_ring
        cols: dict[int, int] = {}
        for c, blk in enumerate(table_row.tolist()):
            if blk >= 0 and blk not in cols:
                cols[blk] = c
        for is_key in (True, False):
            keep = set()
            for lane in ring.lanes(row, is_key=is_key):
                slot = int(ring.lane_slot[is_key][row, lane])
                c = cols.get(slot // bs)
                if c is not None and c * bs + slot % bs < n:
                    keep.add(slot)
                    ring.lane_pos[is_key][row, lane] = c * bs + slot % bs
            if len(keep) != int(ring.length[is_key][row]):
                self._compact_kivi_window(row, keep, is_key=is_key)

    def _clear_stale_kivi_residual_entries(self, req_key: str, live_slots: set[int], *,
                                           is_key: bool) -> None:
        row = self._get_kivi_residual_row(req_key, create=False)
        if row is None:
            return
        self._compact_kivi_window(row, {int(s) for s in live_slots}, is_key=is_key)

    def _compact_kivi_window(self, row: int, keep: set[int], *, is_key: bool) -> None:
        ring = self._kivi_ring
        lanes_before = ring.lanes(row, is_key=is_key)
        slots_before = ring.window_slots(row, is_key=is_key)
        kept = [ln for ln, s in zip(lanes_before, slots_before) if s in keep]
        moves = ring.keep_only(row, keep, is_key=is_key)
        if not moves:
            return
        base = row * ring.ring_len
        flat = ring.tensor(is_key).view(-1, ring.num_kv_heads, ring.head_size)
        src_rows = torch.tensor([base + ln for ln in kept], dtype=torch.long, device=ring.device)
        staged = flat.index_select(0, src_rows)  # copy first: sources and targets overlap
        dst = torch.arange(base, base + len(kept), dtype=torch.long, device=ring.device)
        self._launch_kivi_ring_write(staged, None, dst, is_key)

    # ------------------------------------------------------------------
    # gather + overlay (ab.py:849-935)
    # ------------------------------------------------------------------

    def _request_rows(self, req_keys: list[str]) -> np.ndarray:
        """Ring row per request, -1 for requests without one."""
        get = self.kivi_residual_req_to_row.get
        return np.asarray([get(k, -1) for k in req_keys], dtype=np.int64)

    def _ring_meta_rows(self, seq_lens: list[int], req_keys: list[str]) -> np.ndarray:
        """``[row, k_first, k_tail, v_first, v_tail]`` per request (int32)."""
        ring = self._kivi_ring
        lens = np.asarray([int(n) for n in seq_lens], dtype=np.int64)
        rows = self._request_rows(req_keys)
        meta = np.zeros((lens.size, 5), dtype=np.int32)
        have = rows >= 0
        if have.any():
            kt, kf = ring.tails(rows[have], lens[have], is_key=True)
            vt, vf = ring.tails(rows[have], lens[have], is_key=False)
            meta[have] = np.stack([rows[have], kf, kt, vf, vt], axis=1)
        return meta

    def _gather_dequant_kivi_paged_cache(
        self, block_table: Any, seq_lens: list[int], target_dtype: Any,
        req_ids: list[str] | None = None,
    ) -> tuple[Any, Any]:
        """Dense TND K/V of every request: int4 history with the residual tail overlaid."""
        from ...ops.kivi_layout import check_gather_metadata_host

        self._ensure_kivi_residual_buffers()
        dev = self.k_quant_cache.device
        lens = [int(n) for n in seq_lens]
        batch = len(lens)
        bt = block_table[:batch].to(device=dev, dtype=torch.long).contiguous()
        check_gather_metadata_host(
            bt.to("cpu").tolist(), lens, max_blocks=bt.shape[1],
            num_blocks=self.k_quant_cache.shape[0], block_size=self._get_kivi_block_size(),
        )
        keys = self._get_kivi_req_keys(req_ids, batch)
        meta = torch.from_numpy(self._ring_meta_rows(lens, keys)).to(dev)
        cu = [0]
        for n in lens:
            cu.append(cu[-1] + n)
        cu_t = torch.tensor(cu, dtype=torch.int64).to(dev)
        return self._launch_kivi_gather(bt, cu_t, cu[-1], target_dtype, meta)

    # ------------------------------------------------------------------
    # attention paths (ab.py:937-1392)
    # ------------------------------------------------------------------

    def _decode_seq_array(self, seq_lens: Any, req_keys: list[str]) -> np.ndarray:
        """Decode geometry per request, int32 ``[B, 6]`` = ``{seq_len, k_hist,
        v_hist, ring_row, k_first, v_first}`` (no ring row: all int4)."""
        ring = self._kivi_ring
        lens = np.asarray([int(n) for n in seq_lens], dtype=np.int64)
        rows = self._request_rows(req_keys)
        out = np.zeros((lens.size, 6), dtype=np.int32)
        out[:, 0] = out[:, 1] = out[:, 2] = lens
        have = rows >= 0
        if have.any():
            kt, kf = ring.tails(rows[have], lens[have], is_key=True)
            vt, vf = ring.tails(rows[have], lens[have], is_key=False)
            out[have, 1] = lens[have] - kt
            out[have, 2] = lens[have] - vt
            out[have, 3] = rows[have]
            out[have, 4] = kf
            out[have, 5] = vf
        return out

    def _decode_seqs(self, seq_lens: list[int], req_keys: list[str]) -> list:
        from ...ops.kivi_decode import DecodeSeq

        return [DecodeSeq(*map(int, r)) for r in self._decode_seq_array(seq_lens, req_keys)]

    def _is_kivi_chunked_prefill_all_new(self, attn_metadata: Any) -> bool:
        qlen = attn_metadata.actual_seq_lengths_q
        for i in range(attn_metadata.num_decodes, len(attn_metadata.seq_lens_list)):
            q_start = qlen[i - 1] if i > 0 else 0
            if attn_metadata.seq_lens_list[i] > qlen[i] - q_start:
                return False
        return True

    def forward(
        self,
        layer: Any,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: Any,
        attn_metadata: Any,
        output: torch.Tensor | None = None,
        output_scale: torch.Tensor | None = None,
        output_block_scale: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """INT4 forward entry (``ab.py:972-1004``); bypasses the host cache writer."""
        assert output is not None, "Output tensor must be provided."
        if not getattr(self, "enable_kivi", False):
            raise RuntimeError(
                "the KIVI INT4 attention impl was instantiated without the "
                "kivi_int4 cache dtype; check the host get_impl_cls dispatch"
            )
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError(
                "fused output quantization is not yet supported for "
                "AscendKiviInt4AttentionBackendImpl"
            )
        if attn_metadata is None:
            return output.fill_(0)
        if stream_capturing():
            return self._forward_kivi_captured(query, key, value, attn_metadata, output)
        return self._forward_kivi_attention(query, key, value, attn_metadata, output, kv_cache)

    def _forward_kivi_captured(self, query: Any, key: Any, value: Any, attn_metadata: Any,
                               output: Any) -> Any:
        """``forward`` while the host records a HIP graph.

        The reference has no graph path for KIVI (it runs ``--enforce-eager``,
        ``docs/int4-host-integration.md:137-138``).  The eager step here
        stages a one-step plan (window flushes, slots, lengths) from host
        memory, and a recorded copy of it would replay that one step forever.
        Only a decode step whose capturable form the host created beforehand
        (``kivi_decode_graph``, whose ``prepare`` the host calls before every
        replay) is recorded; anything else is refused.
        """
        b = len(attn_metadata.seq_lens_list)
        graph = self._kivi_capture_graphs.get(b) if self._kivi_capture_graphs else None
        if _attn_state_name(attn_metadata) != "DecodeOnly" or graph is None:
            raise RuntimeError(
                "KIVI INT4 forward() was called under HIP graph capture: its eager step stages "
                "a one-step plan that every replay would reuse. Capture only decode steps, "
                f"after creating the batch-{b} capturable step with "
                "impl.kivi_decode_graph(batch, max_blocks=...), and call "
                "impl.prepare_kivi_graph_replay(attn_metadata, key, value) before every replay; "
                "or run the layer eagerly."
            )
        return graph.launch(query, key, value, output)

    def prepare_kivi_graph_replay(self, attn_metadata: Any, key: Any, value: Any) -> None:
        """Stage the plan of the step a captured ``forward`` will replay next
        (the batch's ``KiviDecodeGraph.prepare``)."""
        b = len(attn_metadata.seq_lens_list)
        graph = self._kivi_capture_graphs.get(b) if self._kivi_capture_graphs else None
        if graph is None:
            raise RuntimeError(f"KIVI decode graph: no capturable step for batch {b}.")
        graph.prepare(attn_metadata, key, value)

    def _forward_kivi_attention(
        self, query: Any, key: Any, value: Any, attn_metadata: Any, output: Any,
        kv_cache: Any = None,
    ) -> Any:
        """Dispatch by attention state (``ab.py:1006-1191``)."""
        self._bind_kivi_cache(kv_cache)
        finished = getattr(attn_metadata, "finished_req_ids", None)
        if finished:
            self._release_finished_kivi_residual_rows({str(r) for r in finished})

        state = _attn_state_name(attn_metadata)
        if state == "DecodeOnly":  # one query token per request
            qlen = list(range(1, len(attn_metadata.seq_lens_list) + 1))
        else:
            qlen = attn_metadata.actual_seq_lengths_q
        num_tokens = int(qlen[-1])
        query = query[:num_tokens]
        req_ids = getattr(attn_metadata, "req_ids", None)

        def actual(t: Any) -> int:
            return min(getattr(attn_metadata, "num_actual_tokens", t.shape[0]), t.shape[0])

        if state == "PrefillNoCache":
            if key is None or value is None:
                raise RuntimeError("KIVI PrefillNoCache requires dense key/value.")
            n = actual(key)
            self._write_kivi_prefill_cache(
                key[:n], value[:n], attn_metadata.slot_mapping[:n], req_ids,
                attn_metadata.actual_seq_lengths_q,
                KiviInt4Semantics.cu_seqlens_to_seq_lens(attn_metadata.actual_seq_lengths_q),
            )
            return self._forward_kivi_prefill(query, key, value, attn_metadata, output)

        if state == "ChunkedPrefill" and not self._is_kivi_chunked_prefill_all_new(attn_metadata):
            raise RuntimeError(
                "KIVI ChunkedPrefill does not support prefill requests with "
                "historical KV cache. Only decode rows plus all-new prefill "
                "prompts are supported."
            )

        seq_lens = attn_metadata.seq_lens_list
        if state == "DecodeOnly":
            if self._kivi_step_enabled(query, key, value):
                done = self._forward_kivi_decode_step(query, key, value, attn_metadata, output)
                if done is not None:
                    return done
            if key is not None and value is not None and actual(key) > 0:
                n = actual(key)
                self._write_kivi_cache(key[:n], value[:n], attn_metadata.slot_mapping[:n],
                                       req_ids, list(range(1, len(seq_lens) + 1)), seq_lens)
            self._sync_kivi_residual_windows(attn_metadata.block_tables, seq_lens, req_ids,
                                             finished)
            return self._forward_kivi_paged_decode_attention(
                query, attn_metadata.block_tables, seq_lens, req_ids, output
            )

        if state == "ChunkedPrefill":
            if key is not None and value is not None and actual(key) > 0:
                n = actual(key)
                slot_mapping = attn_metadata.slot_mapping[:n]
                nd = min(attn_metadata.num_decode_tokens, n)
                ndr = attn_metadata.num_decodes
                if nd > 0:
                    self._write_kivi_cache(
                        key[:nd], value[:nd], slot_mapping[:nd],
                        None if req_ids is None else req_ids[:ndr], list(range(1, ndr + 1)),
                        seq_lens[:ndr],
                    )
                if nd < n:
                    pq = [int(attn_metadata.actual_seq_lengths_q[i]) - nd
                          for i in range(ndr, len(attn_metadata.actual_seq_lengths_q))]
                    self._write_kivi_prefill_cache(
                        key[nd:n], value[nd:n], slot_mapping[nd:n],
                        None if req_ids is None else req_ids[ndr:], pq, seq_lens[ndr:],
                    )
            self._sync_kivi_residual_windows(attn_metadata.block_tables, seq_lens, req_ids,
                                             finished)
            return self._forward_kivi_chunked_prefill(query, key, value, attn_metadata, output)

        if key is not None and value is not None and actual(key) > 0:
            n = actual(key)
            self._write_kivi_cache(key[:n], value[:n], attn_metadata.slot_mapping[:n], req_ids,
                                   attn_metadata.actual_seq_lengths_q, seq_lens)
        self._sync_kivi_residual_windows(attn_metadata.block_tables, seq_lens, req_ids,
                                         finished)
        dense_k, dense_v = self._gather_dequant_kivi_paged_cache(
            attn_metadata.block_tables, seq_lens, query.dtype, req_ids
        )
        return self._forward_kivi_dense_attention(
            query, dense_k, dense_v, seq_lens, qlen, attn_metadata.causal, output
        )

    # ------------------------------------------------------------------
    # decode step from a host plan (sync-free, capturable launches)
    # ------------------------------------------------------------------

    def _kivi_step_enabled(self, query: Any, key: Any, value: Any) -> bool:
        """The planned decode step applies: GPU tensors, none of the launch
        hooks replaced, and a geometry the planned store and the pieces
        decode cover."""
        from .decode_step import step_geometry_ok

        hooks = ("_launch_kivi_key_pack", "_launch_kivi_value_pack",
                 "_launch_kivi_key_pack_rows", "_launch_kivi_value_pack_rows",
                 "_launch_kivi_ring_write", "_launch_kivi_store", "_launch_kivi_decode")
        if any(_hook_replaced(self, h) for h in hooks):
            return False
        if not isinstance(query, torch.Tensor) or query.device.type != "cuda":
            return False
        self._check_kivi_cache_bound()
        if key is not None and value is not None:
            self._adopt_ring_dtype(key, value)
        else:
            self._ensure_kivi_residual_buffers()
        return step_geometry_ok(self, query)

    def _plan_kivi_decode_step(self, attn_metadata: Any, key: Any, value: Any, *,
                               allow_compaction: bool = True):
        """Host half of a decode step: ``(jobs, seqs, block_table)`` or ``None``.

        Validates the block table, replays the window rules for one token per
        request on the mirror (``KiviResidualRing.plan_decode_step``) and
        returns the store jobs, the decode geometry (int32 ``[B, 6]``) and the
        device block table.  Reads nothing from the device when the metadata
        carries host copies (``slot_mapping_cpu``, ``block_tables_cpu``).

        Returns ``None`` with nothing changed when the step needs the general
        path: several tokens for a request, padding slots, a slot that does
        not follow the table at the request's last position, or a window
        entry that may no longer be live (its check, and any compaction,
        belongs after the store, which the general path orders).
        """
        ring = self._ensure_kivi_residual_buffers()
        bs = self._get_kivi_block_size()
        lens = np.asarray([int(x) for x in attn_metadata.seq_lens_list], dtype=np.int64)
        b = lens.size
        keys = self._get_kivi_req_keys(getattr(attn_metadata, "req_ids", None), b)
        table = self._host_array(attn_metadata, "block_tables")[:b].astype(np.int64, copy=False)
        # the gather's metadata gate and the window liveness, one native pass
        rows = self._request_rows(keys)
        suspect = ring.step_check(rows, lens, table, num_blocks=self.k_quant_cache.shape[0],
                                  block_size=bs)
        n = 0
        if key is not None and value is not None:
            n = min(int(getattr(attn_metadata, "num_actual_tokens", key.shape[0])), key.shape[0])
        slots = pos = None
        if n:
            if n != b:
                return None
            slots = self._host_array(attn_metadata, "slot_mapping")[:n].astype(np.int64)
            pos = lens - 1
            col = pos // bs
            if (slots < 0).any() or (pos < 0).any() or (col >= table.shape[1]).any():
                return None
            if ((table[np.arange(b), col] != slots // bs).any()
                    or (slots % bs != pos % bs).any()):
                return None
        if suspect.size:
            if not allow_compaction:
                raise RuntimeError(
                    "KIVI decode step: a window entry may no longer be live; run this "
                    "step eagerly (forward) so its check follows the store."
                )
            return None
        jobs = None
        if n:
            with self._kivi_planning():
                rows = np.asarray([self._get_kivi_residual_row(k, create=True) for k in keys],
                                  dtype=np.int64)
                jobs = ring.plan_decode_step(rows, slots, pos, np.arange(b, dtype=np.int64),
                                             block_size=bs, group_size=self.kivi_group_size)
            if jobs is None:
                if not allow_compaction:
                    raise RuntimeError("KIVI decode step: a slot is already held; run eagerly.")
                return None
        seqs = self._decode_seq_array(lens, keys)
        return jobs, seqs, attn_metadata.block_tables[:b]

    def _forward_kivi_decode_step(self, query: Any, key: Any, value: Any, attn_metadata: Any,
                                  output: Any) -> Any:
        """The decode step as two launches over one staged plan, or ``None``
        (nothing changed) when it needs the general path."""
        from ...ops.kivi_decode import _cu_count
        from .decode_step import (DecodeStepBuffers, KiviDecodeLauncher, eager_capacities,
                                  step_plan_mode)

        from ...ops import _native

        ring = self._ensure_kivi_residual_buffers()
        sig = (self.num_heads, self.num_kv_heads, self.head_size, self.kivi_group_size,
               self._get_kivi_block_size(), self.kivi_residual_length, ring.rows, ring.dtype,
               query.dtype, query.device, int(self.k_quant_cache.shape[0]),
               torch.cuda.current_stream(query.device).cuda_stream)
        shared = _SharedStep.last
        if (shared is not None and shared.md is attn_metadata and shared.sig == sig
                and self._kivi_mirror_matches(shared.before)):
            return self._replay_shared_kivi_step(shared, query, key, value, output)
        before = self._kivi_mirror_snapshot()
        # the window mirror advances in the planning; the transaction stays
        # open through staging and both launches, so an error anywhere before
        # the store is queued leaves the mirror describing the device
        with self._kivi_planning():
            plan = self._plan_kivi_decode_step(attn_metadata, key, value)
            if plan is None:
                return None
            jobs, seqs, table_dev = plan
            b = seqs.shape[0]
            dev = query.device
            cu = _cu_count(dev)
            work_cap, pieces_cap = eager_capacities(b, self.num_kv_heads, cu, seqs)
            bufs = self._kivi_step_bufs
            if bufs is None or not bufs.fits(b, work_cap, pieces_cap):
                # grow with headroom so a serving loop settles on one buffer
                bufs = DecodeStepBuffers(dev, batch=max(b, 2 * (bufs.batch if bufs else 0), 8),
                                         window=self.kivi_residual_length,
                                         num_heads=self.num_heads, head_size=self.head_size,
                                         work_cap=2 * work_cap, pieces_cap=2 * pieces_cap)
                self._kivi_step_bufs = bufs
            mode, tile = step_plan_mode(self, query, fixed=False)
            staged = bufs.stage(jobs, seqs, num_kv_heads=self.num_kv_heads, cu_count=cu,
                                mode=mode, fixed=False, tile=tile)
            launcher = KiviDecodeLauncher(self)
            q = query[:b].reshape(b, self.num_heads, self.head_size).contiguous()
            out = output[:b].view(b, self.num_heads, self.head_size)
            table = table_dev.to(device=dev, dtype=torch.int32).contiguous()
            if jobs is not None:
                ring = self._kivi_ring
                kin = key[:b].reshape(b, self.num_kv_heads, self.head_size).to(
                    ring.dtype).contiguous()
                vin = value[:b].reshape(b, self.num_kv_heads, self.head_size).to(
                    ring.dtype).contiguous()
                launcher.store(bufs, staged, kin, vin)
        launcher.decode(bufs, staged, q, table, out)
        rec = _SharedStep()
        rec.md, rec.sig, rec.before, rec.after = attn_metadata, sig, before, self._kivi_mirror_snapshot()
        rec.bufs, rec.staged, rec.table, rec.b, rec.has_jobs = bufs, staged, table, b, jobs is not None
        _SharedStep.last = rec
        return output

    def _replay_shared_kivi_step(self, rec: "_SharedStep", query: Any, key: Any, value: Any,
                                 output: Any) -> Any:
        """This layer's launches of a step another layer planned and staged
        (``_SharedStep``): the mirror takes the planned state, the store and
        the decode read the staged plan, this layer's caches and ring."""
        from .decode_step import KiviDecodeLauncher

        b = rec.b
        launcher = KiviDecodeLauncher(self)
        q = query[:b].reshape(b, self.num_heads, self.head_size).contiguous()
        out = output[:b].view(b, self.num_heads, self.head_size)
        self._kivi_mirror_load(rec.after)
        try:
            if rec.has_jobs:
                ring = self._kivi_ring
                kin = key[:b].reshape(b, self.num_kv_heads, self.head_size).to(
                    ring.dtype).contiguous()
                vin = value[:b].reshape(b, self.num_kv_heads, self.head_size).to(
                    ring.dtype).contiguous()
                launcher.store(rec.bufs, rec.staged, kin, vin)
        except BaseException:
            self._kivi_mirror_load(rec.before)  # nothing was queued
            raise
        launcher.decode(rec.bufs, rec.staged, q, rec.table, out)
        return output

    def kivi_decode_graph(self, batch: int, *, max_blocks: int, rounds: int = 1):
        """A ``KiviDecodeGraph`` for this layer: the decode step's launches,
        capturable once in a HIP graph and replayed every step after
        ``prepare`` stages that step's plan."""
        from .decode_step import KiviDecodeGraph

        graph = KiviDecodeGraph(self, batch, max_blocks=max_blocks, rounds=rounds)
        if self._kivi_capture_graphs is None:
            self._kivi_capture_graphs = {}
        self._kivi_capture_graphs[batch] = graph  # what a captured forward() launches
        return graph

    def _forward_kivi_paged_decode_attention(
        self, query: Any, block_table: Any, seq_lens: list[int], req_ids: list[str] | None,
        output: Any,
    ) -> Any:
        """One query token per request over int4 history + residual (``ab.py:1193-1230``)."""
        from ...ops.kivi_layout import check_gather_metadata_host

        batch = len(seq_lens)
        keys = self._get_kivi_req_keys(req_ids, batch)
        lens = [int(n) for n in seq_lens]
        seqs = self._decode_seqs(lens, keys)
        q = query[:batch].reshape(batch, self.num_heads, self.head_size)
        out_view = output[:batch].view(batch, self.num_heads, self.head_size)
        bt = block_table[:batch].to(device=q.device, dtype=torch.int32).contiguous()
        # the same live-block gate the reference's gather applies on this path
        # (pkg/ops/kivi_layout.py:205-238); one host copy of the table
        check_gather_metadata_host(
            bt.to("cpu").tolist(), lens, max_blocks=bt.shape[1],
            num_blocks=self.k_quant_cache.shape[0], block_size=self._get_kivi_block_size(),
        )
        got = self._launch_kivi_decode(q.contiguous(), bt, seqs, out_view)
        if got is not None and got is not out_view:
            out_view.copy_(got)
        return output

    def _forward_kivi_prefill(self, query: Any, key: Any, value: Any, attn_metadata: Any,
                              output: Any) -> Any:
        """Causal prefill on the raw prompt K/V (``ab.py:1232-1266``)."""
        lens = KiviInt4Semantics.cu_seqlens_to_seq_lens(attn_metadata.actual_seq_lengths_q)
        n = sum(lens)
        out = output[:n].view(n, self.num_heads, self.head_size)
        got = self._launch_dense_attention(
            query[:n].reshape(n, self.num_heads, self.head_size), key[:n], value[:n], lens, lens,
            bool(attn_metadata.causal), out,
        )
        if got is not None and got is not out:
            out.copy_(got)
        return output

    # reference name of the same path
    _forward_kivi_prefill_fia = _forward_kivi_prefill

    def _forward_kivi_chunked_prefill(self, query: Any, key: Any, value: Any,
                                      attn_metadata: Any, output: Any) -> Any:
        """Decode rows on the paged cache, all-new prompt rows on their own K/V.

        ``ab.py:1268-1339``.
        """
        nd = attn_metadata.num_decode_tokens
        ndr = attn_metadata.num_decodes
        qlen = attn_metadata.actual_seq_lengths_q
        num_tokens = int(qlen[-1])
        req_ids = getattr(attn_metadata, "req_ids", None)
        if nd > 0:
            self._forward_kivi_paged_decode_attention(
                query[:nd], attn_metadata.block_tables[:ndr], attn_metadata.seq_lens_list[:ndr],
                None if req_ids is None else req_ids[:ndr], output,
            )
        if attn_metadata.num_prefills <= 0:
            return output
        if key is None or value is None:
            raise RuntimeError(
                "KIVI ChunkedPrefill requires dense key/value for all-new prefill prompts."
            )
        if not self._is_kivi_chunked_prefill_all_new(attn_metadata):
            raise RuntimeError(
                "KIVI ChunkedPrefill prefill-with-history is disabled. Only "
                "all-new prompt prefills are supported."
            )
        lens = [int(qlen[i]) - (int(qlen[i - 1]) if i > 0 else 0) for i in range(ndr, len(qlen))]
        n = num_tokens - nd
        out = output[nd:num_tokens].view(n, self.num_heads, self.head_size)
        got = self._launch_dense_attention(
            query[nd:num_tokens].reshape(n, self.num_heads, self.head_size),
            key[nd:num_tokens], value[nd:num_tokens], lens, lens, bool(attn_metadata.causal), out,
        )
        if got is not None and got is not out:
            out.copy_(got)
        return output

    def _forward_kivi_dense_attention(self, query: Any, key: Any, value: Any,
                                      seq_lens: list[int], actual_seq_qlen: Any, causal: bool,
                                      output: Any) -> Any:
        """Attention of each request's queries over its dense K/V (``ab.py:1341-1392``)."""
        q_lens = KiviInt4Semantics.cu_seqlens_to_seq_lens(actual_seq_qlen)
        q_lens = q_lens[: len(seq_lens)]
        n = sum(q_lens)
        if n == 0:
            return output
        out = output[:n].view(n, self.num_heads, self.head_size)
        got = self._launch_dense_attention(
            query[:n].reshape(n, self.num_heads, self.head_size), key, value, q_lens,
            [int(x) for x in seq_lens], bool(causal), out,
        )
        if got is not None and got is not out:
            out.copy_(got)
        return output


__all__ = ["AscendKiviInt4AttentionBackendMixin"]
