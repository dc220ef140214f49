# SPDX-License-Identifier: Apache-2.0
"""Device-resident KIVI residual windows with a host mirror.

The reference keeps one full-precision ring row per request
(``[max_num_seqs, R, KVH, D]``) and drives it token by token from Python,
synchronising with the device for every slot lookup
(``pkg/methods/kivi_int4/attention_backend.py:181-462``).  Here the ring
tensors stay on the GPU and the host keeps an exact mirror of which slot
every lane holds, so the per-token rules can be replayed on the host without
reading the device:

* a slot already held is overwritten in place;
* otherwise, while the window is full, keys flush the whole window and values
  evict the single oldest lane (``:448-455``); then the token is appended.

A row has ``R + 1`` lanes for a window of ``R`` tokens: the free lane is where
the next token goes, so a step that evicts and appends never writes the lane
it packs, and the whole step can run as one launch.

The mirror is a set of numpy arrays (start, length, slot and token position
per lane), so a decode step -- one new token for each of a batch of requests
-- is planned for the whole batch at once (``plan_decode_step``), and the
per-step check that every window entry is still live needs a per-entry look
only where the token's recorded position no longer maps to its slot
(``suspect_rows``).

Replaying a batch of tokens yields a ``StorePlan``: packed-history writes
(sources are old ring lanes or rows of this step's input) and final ring-lane
writes.  ``execute`` issues them as one launch when no ring write of the batch
overwrites a lane the batch packs (every single-token step), otherwise as up
to three launches per side (key pack, value pack, ring write), in an order
that reads every old lane before it is overwritten.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field

import numpy as np
import torch

from ...ops.kivi_layout import key_slot_groups_error

_SIDES = (True, False)
_FLUSH_ERROR = "KIVI key flush requires contiguous aligned token groups."


@dataclass
class SideWrites:
    """Device work of one side (keys or values) for one store batch."""

    pack_src: list[int] = field(default_factory=list)  # source row per packed token
    pack_slots: list[int] = field(default_factory=list)  # history slot per packed token
    ring: dict[int, int] = field(default_factory=dict)  # ring row -> input row (last wins)
    lane_src: dict[int, int] = field(default_factory=dict)  # ring row -> current source row

    def empty(self) -> bool:
        return not self.pack_slots and not self.ring


@dataclass
class StorePlan:
    """Batched device work; source rows index ``[ring rows ; input rows]``."""

    key: SideWrites = field(default_factory=SideWrites)
    value: SideWrites = field(default_factory=SideWrites)

    def side(self, is_key: bool) -> SideWrites:
        return self.key if is_key else self.value

    def empty(self) -> bool:
        return self.key.empty() and self.value.empty()

    def one_launch_jobs(self) -> tuple[list[int], tuple[int, int, int, int]] | None:
        """``(jobs, counts)`` for a single store launch, or ``None``.

        ``jobs`` is key pack src | key pack slot | value pack src | value pack
        slot | key ring src | key ring dst | value ring src | value ring dst;
        ``counts`` the four lengths.  ``None`` when a ring write overwrites a
        ring row the same batch packs: the packs must then run first.
        """
        k, v = self.key, self.value
        for side in (k, v):
            if side.ring and side.pack_src and not side.ring.keys().isdisjoint(side.pack_src):
                return None
        jobs = (k.pack_src + k.pack_slots + v.pack_src + v.pack_slots
                + list(k.ring.values()) + list(k.ring.keys())
                + list(v.ring.values()) + list(v.ring.keys()))
        return jobs, (len(k.pack_src), len(v.pack_src), len(k.ring), len(v.ring))


@dataclass
class StepJobs:
    """A decode step's store work (one token per request), as int64 arrays.

    Pack sources index ``[ring rows ; input rows]``; ring sources are input
    rows and ring destinations ring rows.  No ring destination is a pack
    source of the same side, so the whole step is one launch.
    """

    key_pack_src: np.ndarray
    key_pack_slot: np.ndarray
    value_pack_src: np.ndarray
    value_pack_slot: np.ndarray
    key_ring_src: np.ndarray
    key_ring_dst: np.ndarray
    value_ring_src: np.ndarray
    value_ring_dst: np.ndarray


class KiviResidualRing:
    """Ring tensors ``[rows, R + 1, KVH, D]`` (keys, values) plus their host mirror.

    ``window`` is the residual length ``R``; ``ring_len = R + 1`` lanes per row.
    Mirror arrays, per side (``True`` = keys): ``start[side][row]``,
    ``length[side][row]``, ``lane_slot[side][row, lane]`` (-1 when free) and
    ``lane_pos[side][row, lane]`` (the token's position in its request, -1
    when the writer did not know it).
    """

    def __init__(
        self,
        rows: int,
        window: int,
        num_kv_heads: int,
        head_size: int,
        *,
        device,
        dtype=torch.float32,
    ) -> None:
        ring_len = window + 1
        self.rows = rows
        self.window = window
        self.ring_len = ring_len
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.device = device
        self.key = torch.zeros((rows, ring_len, num_kv_heads, head_size), dtype=dtype, device=device)
        self.value = torch.zeros_like(self.key)
        self.written = False
        # the whole mirror is one int64 block; the per-side arrays are views
        # into it, so a snapshot, a comparison or a restore is one operation
        per_side = 2 * rows + 2 * rows * ring_len
        self._mirror = np.empty(2 * per_side, dtype=np.int64)
        self.start, self.length, self.lane_slot, self.lane_pos = {}, {}, {}, {}
        off = 0
        for s in _SIDES:
            self.start[s] = self._mirror[off:off + rows]
            self.length[s] = self._mirror[off + rows:off + 2 * rows]
            off += 2 * rows
            self.lane_slot[s] = self._mirror[off:off + rows * ring_len].reshape(rows, ring_len)
            off += rows * ring_len
            self.lane_pos[s] = self._mirror[off:off + rows * ring_len].reshape(rows, ring_len)
            off += rows * ring_len
            self.start[s][:] = 0
            self.length[s][:] = 0
            self.lane_slot[s][:] = -1
            self.lane_pos[s][:] = -1
        self._saved: dict[int, tuple] | None = None
        # vectorized snapshots of whole batches of rows: (rows, per-side arrays)
        self._saved_batches: list[tuple[np.ndarray, tuple]] = []

    # -- all-or-nothing planning ----------------------------------------------

    @contextmanager
    def transaction(self):
        """Undo the mirror changes made inside the block when it raises.

        A batch is planned request by request, and every request updates the
        mirror as it goes; the launches come after the whole batch is planned.
        When a later request is rejected (an unaligned key flush), nothing is
        launched, so the earlier requests' mirror changes are rolled back too
        and the mirror keeps describing what the device holds.
        """
        if self._saved is not None:  # nested: the outer block restores
            yield
            return
        self._saved = {}
        self._saved_batches = []
        try:
            yield
        except BaseException:
            for row, state in self._saved.items():
                if state is not None:
                    self._restore(row, state)
            for rows, snap in self._saved_batches:
                for k, (start, length, ls, lp) in zip(_SIDES, snap):
                    self.start[k][rows] = start
                    self.length[k][rows] = length
                    self.lane_slot[k][rows] = ls
                    self.lane_pos[k][rows] = lp
            raise
        finally:
            self._saved = None
            self._saved_batches = []

    def _touch_rows(self, rows: np.ndarray) -> None:
        """``_touch`` for a batch of distinct rows, as one vectorized copy.

        Rows already saved keep their earlier snapshot; the rest are marked
        saved (the per-row map holds ``None`` for them) so later touches do
        not snapshot them again.
        """
        if self._saved is None:
            return
        new = [r for r in rows.tolist() if r not in self._saved]
        if not new:
            return
        idx = np.asarray(new, dtype=np.int64)
        self._saved_batches.append((idx, tuple(
            (self.start[k][idx].copy(), self.length[k][idx].copy(),
             self.lane_slot[k][idx].copy(), self.lane_pos[k][idx].copy())
            for k in _SIDES)))
        for r in new:
            self._saved[r] = None

    def _touch(self, row: int) -> None:
        if self._saved is not None and row not in self._saved:
            self._saved[row] = tuple(
                (int(self.start[k][row]), int(self.length[k][row]),
                 self.lane_slot[k][row].copy(), self.lane_pos[k][row].copy())
                for k in _SIDES
            )

    def _restore(self, row: int, state: tuple) -> None:
        for k, (start, length, ls, lp) in zip(_SIDES, state):
            self.start[k][row] = start
            self.length[k][row] = length
            self.lane_slot[k][row] = ls
            self.lane_pos[k][row] = lp

    def snapshot(self) -> np.ndarray:
        """A copy of the whole mirror (start, length, lane_slot, lane_pos of
        both sides)."""
        return self._mirror.copy()

    def matches(self, snap: np.ndarray) -> bool:
        """The mirror equals ``snap`` (a ``snapshot`` of a ring of this shape)."""
        return snap.shape == self._mirror.shape and bool((self._mirror == snap).all())

    def load(self, snap: np.ndarray) -> None:
        """Set the mirror to ``snap`` (copied in; ``snap`` stays unchanged)."""
        np.copyto(self._mirror, snap)

    def state(self) -> tuple:
        """The whole mirror as nested tuples of ints (for comparisons)."""
        return tuple(
            (tuple(self.start[k].tolist()), tuple(self.length[k].tolist()),
             tuple(map(tuple, self.lane_slot[k].tolist())))
            for k in _SIDES
        )

    # -- dtype ----------------------------------------------------------------

    @property
    def dtype(self):
        return self.key.dtype

    def adopt_dtype(self, dtype) -> None:
        """Match the ring to the activations so pack and overlay stay exact.

        An untouched ring takes the activation dtype; a ring that already
        holds data and meets a different dtype widens to fp32 (lossless for
        every 16-bit input).
        """
        if dtype == self.key.dtype:
            return
        if not self.written:
            self.key = torch.zeros(self.key.shape, dtype=dtype, device=self.device)
            self.value = torch.zeros_like(self.key)
        elif self.key.dtype != torch.float32:
            self.key = self.key.float()
            self.value = self.value.float()

    def tensor(self, is_key: bool) -> torch.Tensor:
        return self.key if is_key else self.value

    # -- host mirror queries -----------------------------------------------

    def lanes(self, row: int, *, is_key: bool) -> list[int]:
        """Occupied lanes of ``row`` in FIFO order (wrapping past R)."""
        n = int(self.length[is_key][row])
        s = int(self.start[is_key][row])
        return [(s + i) % self.ring_len for i in range(n)]

    def window_slots(self, row: int, *, is_key: bool) -> list[int]:
        ls = self.lane_slot[is_key][row]
        return [int(ls[lane]) for lane in self.lanes(row, is_key=is_key)]

    def holds(self, row: int, slot: int, *, is_key: bool) -> bool:
        return bool((self.lane_slot[is_key][row] == slot).any())

    def tail(self, row: int, seq_len: int, *, is_key: bool) -> tuple[int, int]:
        """``(tail_len, first_lane)`` of the overlay for a sequence of ``seq_len``.

        The last ``min(seq_len, len)`` window entries replace the sequence's
        last positions (``attention_backend.py:899-923``).
        """
        n = int(self.length[is_key][row])
        t = min(int(seq_len), n)
        first = (int(self.start[is_key][row]) + n - t) % self.ring_len
        return t, first

    def tails(self, rows: np.ndarray, seq_lens: np.ndarray, *, is_key: bool
              ) -> tuple[np.ndarray, np.ndarray]:
        """``tail`` for many rows at once: ``(tail_len, first_lane)`` arrays."""
        n = self.length[is_key][rows]
        t = np.minimum(seq_lens, n)
        first = (self.start[is_key][rows] + n - t) % self.ring_len
        return t, first

    def suspect_rows(self, rows: np.ndarray, seq_lens: np.ndarray, table: np.ndarray,
                     block_size: int) -> np.ndarray:
        """Indices into ``rows`` whose windows need the per-entry liveness check.

        An entry written at position ``p`` with slot ``s`` is live for the
        reference (``attention_backend.py:813-836``: the first column holding
        ``s``'s block, times the block size plus ``s``'s offset, is below the
        sequence length) whenever ``p < seq_len`` and the request's table
        still has ``s``'s block at column ``p // block_size``: that column is
        then the first holder or comes after it.  Rows where some entry fails
        this test (or has no recorded position) are returned; every entry of
        the other rows is live.
        """
        if rows.size == 0:
            return np.zeros(0, dtype=np.int64)
        suspect = np.zeros(rows.shape[0], dtype=bool)
        maxb = table.shape[1]
        n = seq_lens[:, None]
        req = np.arange(rows.shape[0])[:, None]
        for k in _SIDES:
            ls = self.lane_slot[k][rows]
            lp = self.lane_pos[k][rows]
            occ = ls >= 0
            col = lp // block_size
            ok = (lp >= 0) & (lp < n) & (col < maxb)
            tb = table[req, np.clip(col, 0, maxb - 1)]
            ok &= tb == ls // block_size
            suspect |= (occ & ~ok).any(axis=1)
        return np.flatnonzero(suspect)

    def step_check(self, rows: np.ndarray, seq_lens: np.ndarray, table: np.ndarray, *,
                   num_blocks: int, block_size: int) -> np.ndarray:
        """A decode step's host checks in one native pass
        (``kvq_kivi_step_check``): the gather's metadata gate, raising as
        ``check_gather_metadata_host`` does, then ``suspect_rows`` for the
        requests with a row (``rows[i] >= 0``).  Returns the indices into
        ``rows`` of the suspect requests."""
        from ...ops import _native

        table = np.ascontiguousarray(table, dtype=np.int64)
        lens = np.ascontiguousarray(seq_lens, dtype=np.int64)
        rows = np.ascontiguousarray(rows, dtype=np.int64)
        b, maxb = table.shape
        if lens.size != b or rows.size != b:
            raise ValueError("step_check: table, seq_lens and rows must have one entry per request")
        k_slot, k_pos, v_slot, v_pos = (np.ascontiguousarray(a) for a in (
            self.lane_slot[True], self.lane_pos[True], self.lane_slot[False],
            self.lane_pos[False]))
        suspect = np.zeros(b, dtype=np.int32)
        kind = np.zeros(1, dtype=np.int32)
        r = _native.lib().kvq_kivi_step_check(
            table.ctypes.data, b, maxb, lens.ctypes.data, int(num_blocks), int(block_size),
            rows.ctypes.data, k_slot.ctypes.data, k_pos.ctypes.data, v_slot.ctypes.data,
            v_pos.ctypes.data, self.rows, self.ring_len, suspect.ctypes.data, kind.ctypes.data)
        _native.check(int(r) if r < 0 else 0, "kvq_kivi_step_check")
        if kind[0] == 3:
            raise RuntimeError(
                "block_table does not cover the longest KIVI sequence: "
                f"max_seq_len={int(lens.max())}, max_blocks={maxb}, block_size={block_size}."
            )
        if kind[0] == 1:
            raise RuntimeError("KIVI block_table has invalid block ids for live tokens.")
        if kind[0] == 2:
            raise RuntimeError("KIVI block_table references blocks outside the int4 cache.")
        return np.flatnonzero(suspect)

    # -- mutation ----------------------------------------------------------

    def load_row(self, row: int, *, is_key: bool, slots: list[int],
                 positions: list[int] | None = None) -> None:
        """Describe a window the caller wrote to lanes ``0..len(slots)-1`` itself
        (a state restored or built outside the store path)."""
        n = len(slots)
        if n > self.window:
            raise ValueError(f"a window holds at most {self.window} tokens, got {n}")
        self._touch(row)
        self.start[is_key][row] = 0
        self.length[is_key][row] = n
        self.lane_slot[is_key][row] = -1
        self.lane_pos[is_key][row] = -1
        self.lane_slot[is_key][row, :n] = slots
        if positions is not None:
            self.lane_pos[is_key][row, :n] = positions

    def reset_row(self, row: int) -> None:
        self._touch(row)
        for is_key in _SIDES:
            self.start[is_key][row] = 0
            self.length[is_key][row] = 0
            self.lane_slot[is_key][row] = -1
            self.lane_pos[is_key][row] = -1

    def keep_only(self, row: int, keep_slots: set[int], *, is_key: bool) -> list[tuple[int, int]]:
        """Drop lanes whose slot is not in ``keep_slots``; compact to lane 0.

        Returns the ``(dst_lane, src_lane)`` moves the device copy must perform
        (the reference rewrites the kept entries from lane 0 on,
        ``attention_backend.py:328-356``).
        """
        self._touch(row)
        lanes = self.lanes(row, is_key=is_key)
        ls = self.lane_slot[is_key][row]
        lp = self.lane_pos[is_key][row]
        kept = [lane for lane in lanes if int(ls[lane]) in keep_slots]
        if len(kept) == len(lanes):
            return []
        slots = ls[kept].copy()
        pos = lp[kept].copy()
        self.start[is_key][row] = 0
        self.length[is_key][row] = len(kept)
        ls[:] = -1
        lp[:] = -1
        ls[: len(kept)] = slots
        lp[: len(kept)] = pos
        return [(i, src) for i, src in enumerate(kept) if i != src]

    def plan_store(
        self,
        plan: StorePlan,
        row: int,
        slots: list[int],
        input_rows: list[int],
        *,
        is_key: bool,
        block_size: int,
        group_size: int,
        positions: list[int] | None = None,
    ) -> None:
        """Replay ``_store_kivi_residual_entries`` for one request and side.

        ``input_rows[i]`` is the row (in the step's input) of the token with
        slot ``slots[i]``, and ``positions[i]`` its position in the request
        when the caller knows it.  Updates the mirror and appends the device
        work to ``plan``; raises before any launch if a key flush would break
        the pack kernel's aligned-group contract.

        A run of distinct slots none of which the window holds (a prompt
        chunk, a decode token) is planned in closed form (``_plan_run``);
        anything else replays token by token (``_plan_tokens``).  Both give
        the same plan and mirror.
        """
        self._touch(row)
        if len(slots) > 1 and len(set(slots)) == len(slots) and not np.isin(
                self.lane_slot[is_key][row], slots).any():
            self._plan_run(plan, row, slots, input_rows, positions, is_key=is_key,
                           block_size=block_size, group_size=group_size)
        else:
            self._plan_tokens(plan, row, slots, input_rows, positions, is_key=is_key,
                              block_size=block_size, group_size=group_size)

    def _evict(self, side: SideWrites, row: int, ev: list[int], *, is_key: bool) -> None:
        base = row * self.ring_len
        ls = self.lane_slot[is_key][row]
        side.pack_src.extend(side.lane_src.get(base + lane, base + lane) for lane in ev)
        side.pack_slots.extend(int(ls[lane]) for lane in ev)
        for lane in ev:
            side.ring.pop(base + lane, None)
            side.lane_src.pop(base + lane, None)
        ls[ev] = -1
        self.lane_pos[is_key][row, ev] = -1

    def _plan_run(self, plan: StorePlan, row: int, slots: list[int], input_rows: list[int],
                  positions: list[int] | None = None, *, is_key: bool, block_size: int,
                  group_size: int) -> None:
        """``plan_store`` for new, distinct slots without a per-token walk.

        With ``l0`` entries in the window and ``n`` new ones, the per-token
        rules evict ``((l0 + n - 1) // R) * R`` entries on the key side (whole
        windows) and ``max(0, l0 + n - R)`` on the value side (one per token
        past a full window), oldest first; every eviction moves the start one
        lane per evicted entry, and the survivors stay contiguous from the
        start.  New tokens evicted inside the run are packed straight from the
        input and never written to the ring.
        """
        side = plan.side(is_key)
        r, cap = self.ring_len, self.window
        na, base = self.rows * r, row * r
        ls = self.lane_slot[is_key][row]
        lp = self.lane_pos[is_key][row]
        n = len(slots)
        if positions is None:
            positions = [-1] * n
        s0, l0 = int(self.start[is_key][row]), int(self.length[is_key][row])
        evict = ((l0 + n - 1) // cap) * cap if is_key else max(0, l0 + n - cap)
        ev_old = [(s0 + j) % r for j in range(min(evict, l0))]
        ev_new = evict - len(ev_old)
        if evict:
            ev_slots = [int(ls[lane]) for lane in ev_old] + list(slots[:ev_new])
            if is_key:
                for w in range(0, evict, cap):
                    if key_slot_groups_error(ev_slots[w:w + cap], block_size=block_size,
                                             group_size=group_size) is not None:
                        raise RuntimeError(_FLUSH_ERROR)
            self._evict(side, row, ev_old, is_key=is_key)
            side.pack_src.extend(na + irow for irow in input_rows[:ev_new])
            side.pack_slots.extend(slots[:ev_new])
        start = (s0 + evict) % r
        kept_old = l0 - len(ev_old)
        for j in range(ev_new, n):
            lane = (start + kept_old + j - ev_new) % r
            ls[lane] = slots[j]
            lp[lane] = positions[j]
            side.lane_src[base + lane] = na + input_rows[j]
            side.ring[base + lane] = input_rows[j]
        self.start[is_key][row] = start
        self.length[is_key][row] = kept_old + n - ev_new

    def _plan_tokens(self, plan: StorePlan, row: int, slots: list[int], input_rows: list[int],
                     positions: list[int] | None = None, *, is_key: bool, block_size: int,
                     group_size: int) -> None:
        """``plan_store`` token by token: the reference's loop (``ab.py:411-462``)."""
        side = plan.side(is_key)
        r = self.ring_len
        cap = self.window
        na = self.rows * r
        base = row * r
        ls = self.lane_slot[is_key][row]
        lp = self.lane_pos[is_key][row]
        if positions is None:
            positions = [-1] * len(slots)
        for slot, irow, pos in zip(slots, input_rows, positions):
            held = np.flatnonzero(ls == slot)
            if held.size:
                lane = int(held[0])
                side.lane_src[base + lane] = na + irow
                side.ring[base + lane] = irow
                continue
            while self.length[is_key][row] >= cap:
                count = cap if is_key else 1
                ev = self.lanes(row, is_key=is_key)[:count]
                if is_key:
                    err = key_slot_groups_error([int(ls[lane]) for lane in ev],
                                                block_size=block_size, group_size=group_size)
                    if err is not None:
                        raise RuntimeError(_FLUSH_ERROR)
                self._evict(side, row, ev, is_key=is_key)
                # the start moves past the evicted lanes even when the window
                # empties, so the append below lands on the lane that was free
                # before this flush, never on one it packs
                self.length[is_key][row] -= count
                self.start[is_key][row] = (self.start[is_key][row] + count) % r
            tail = int((self.start[is_key][row] + self.length[is_key][row]) % r)
            ls[tail] = slot
            lp[tail] = pos
            side.lane_src[base + tail] = na + irow
            side.ring[base + tail] = irow
            self.length[is_key][row] += 1

    def plan_decode_step(self, rows: np.ndarray, slots: np.ndarray, positions: np.ndarray,
                         input_rows: np.ndarray, *, block_size: int,
                         group_size: int) -> StepJobs | None:
        """One new token for each of a batch of requests, planned for the whole
        batch at once; ``None`` (nothing changed) when the batch does not fit
        the closed form -- repeated rows, or a slot a window already holds --
        and the caller replays it token by token instead.

        For each row and side the per-token rule is: a full window evicts
        (keys: the whole window, checked for aligned groups first; values:
        the oldest lane), then the token goes to lane ``start + length``.
        Every key window is checked before any row changes, so a rejected
        batch leaves the mirror as it was.
        """
        if rows.size == 0 or np.unique(rows).size != rows.size:
            return None
        for k in _SIDES:
            if (self.lane_slot[k][rows] == slots[:, None]).any():
                return None
        r, cap = self.ring_len, self.window
        full_k = self.length[True][rows] >= cap
        fk = rows[full_k]
        k_lanes = (self.start[True][fk][:, None] + np.arange(cap)) % r
        k_ev = self.lane_slot[True][fk[:, None], k_lanes]
        if fk.size and not self._aligned_windows(k_ev, block_size, group_size):
            raise RuntimeError(_FLUSH_ERROR)
        # inside a transaction the rows are snapshotted, so an error after the
        # planning (staging, a launch) still rolls the whole batch back
        self._touch_rows(rows)
        # keys: flush whole windows
        kp_src = (fk[:, None] * r + k_lanes).ravel()
        kp_slot = k_ev.ravel()
        self.lane_slot[True][fk[:, None], k_lanes] = -1
        self.lane_pos[True][fk[:, None], k_lanes] = -1
        self.start[True][fk] = (self.start[True][fk] + cap) % r
        self.length[True][fk] = 0
        # values: evict the oldest lane of each full window
        fv = rows[self.length[False][rows] >= cap]
        v_lane = self.start[False][fv]
        vp_src = fv * r + v_lane
        vp_slot = self.lane_slot[False][fv, v_lane].copy()
        self.lane_slot[False][fv, v_lane] = -1
        self.lane_pos[False][fv, v_lane] = -1
        self.start[False][fv] = (v_lane + 1) % r
        self.length[False][fv] -= 1
        # the new token goes to lane start + length on both sides
        dst = {}
        for k in _SIDES:
            tail = (self.start[k][rows] + self.length[k][rows]) % r
            self.lane_slot[k][rows, tail] = slots
            self.lane_pos[k][rows, tail] = positions
            self.length[k][rows] += 1
            dst[k] = rows * r + tail
        src = input_rows.astype(np.int64)
        return StepJobs(kp_src.astype(np.int64), kp_slot.astype(np.int64),
                        vp_src.astype(np.int64), vp_slot.astype(np.int64), src, dst[True], src,
                        dst[False])

    @staticmethod
    def _aligned_windows(windows: np.ndarray, block_size: int, group_size: int) -> bool:
        """Every row of ``windows`` passes ``key_slot_groups_error``."""
        n, w = windows.shape
        if (windows < 0).any() or w % group_size:
            return False
        g = windows.reshape(n, w // group_size, group_size)
        if not (np.diff(g, axis=2) == 1).all():
            return False
        if (g[:, :, 0] % group_size).any():
            return False
        return bool((g[:, :, 0] // block_size == g[:, :, -1] // block_size).all())

    def flush_prefix(self, plan: StorePlan, row: int, count: int, *, is_key: bool,
                     block_size: int, group_size: int) -> None:
        """Move the ``count`` oldest entries of a window to int4 history."""
        self._touch(row)
        n = int(self.length[is_key][row])
        count = min(count, n)
        if count <= 0:
            return
        ev = self.lanes(row, is_key=is_key)[:count]
        ls = self.lane_slot[is_key][row]
        if is_key:
            err = key_slot_groups_error([int(ls[lane]) for lane in ev], block_size=block_size,
                                        group_size=group_size)
            if err is not None or count % group_size:
                raise RuntimeError(_FLUSH_ERROR)
        self._evict(plan.side(is_key), row, ev, is_key=is_key)
        self.length[is_key][row] = n - count
        self.start[is_key][row] = (self.start[is_key][row] + count) % self.ring_len

    # -- execution ---------------------------------------------------------

    def execute(
        self,
        plan: StorePlan,
        key_input: torch.Tensor | None,
        value_input: torch.Tensor | None,
        *,
        pack_key,
        pack_value,
        ring_write,
        store=None,
    ) -> None:
        """Issue a plan: one launch when the plan allows it, else history packs
        first (they read old lanes), then ring writes.

        ``pack_key/pack_value(src_a, src_b, src_index, slots)`` and
        ``ring_write(src, src_rows, dst_rows, is_key)`` are the launch hooks;
        ``src_a`` is the ring viewed as ``[rows*(R+1), KVH, D]``, ``src_b`` the
        step's input converted to the ring dtype.  ``store(key_input,
        value_input, jobs, counts)`` (optional) issues a whole hazard-free plan
        (``StorePlan.one_launch_jobs``) and returns False when it cannot.
        """
        dev = self.key.device
        if store is not None:
            one = plan.one_launch_jobs()
            if one is not None:
                jobs, counts = one
                kin, vin = (
                    None if x is None else x.to(self.dtype).contiguous()
                    for x in (key_input, value_input)
                )
                jt = torch.tensor(jobs, dtype=torch.int64).to(dev, non_blocking=True)
                if store(kin, vin, jt, counts):
                    if counts[2] or counts[3]:
                        self.written = True
                    return
        inputs = {True: key_input, False: value_input}
        for is_key in _SIDES:
            side = plan.side(is_key)
            if not side.pack_slots:
                continue
            inp = inputs[is_key]
            if inp is not None and inp.dtype != self.dtype:
                inp = inp.to(self.dtype)
            flat = self.tensor(is_key).view(-1, self.num_kv_heads, self.head_size)
            idx = torch.tensor(side.pack_src, dtype=torch.int64).to(dev, non_blocking=True)
            slots = torch.tensor(side.pack_slots, dtype=torch.int64).to(dev, non_blocking=True)
            (pack_key if is_key else pack_value)(flat, inp, idx, slots)
        for is_key in _SIDES:
            side = plan.side(is_key)
            if not side.ring:
                continue
            dst = torch.tensor(list(side.ring.keys()), dtype=torch.int64).to(dev, non_blocking=True)
            src = torch.tensor(list(side.ring.values()), dtype=torch.int64).to(dev, non_blocking=True)
            ring_write(inputs[is_key], src, dst, is_key)
            self.written = True


__all__ = ["KiviResidualRing", "SideWrites", "StepJobs", "StorePlan"]
