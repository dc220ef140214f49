# SPDX-License-Identifier: Apache-2.0
"""CPU oracle for the quantized-KV hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(the ``vllm_ascend_quantized_kv_cache`` package and its HIP library) never
imports, links or calls anything under ``oracle/``.

Every function restates one piece of the reference algorithm in vectorized
torch-CPU code (the reference itself is torch, so torch-CPU reproduces its
IEEE fp32 and bf16 rounding exactly).  Each docstring cites the reference
lines it follows; paths are relative to ``/root/reference`` with
``pkg/ = src/vllm_ascend_quantized_kv_cache/``.

How each function is pinned (checked by ``tests/test_oracle.py``):

* ``group_scale`` / ``quantize_group`` / ``pack_int4`` / ``unpack_int4`` --
  the reference's known-answer tests (``tests/test_kivi_int4.py:1140-1171``,
  ``:76-81``) and the independent scalar C restatement ``oracle/kvq_ref.c``.
* ``pack_key_cache`` / ``pack_value_cache`` / ``dequant_gather`` -- the C
  restatement (bit-exact, element by element), the round trip against
  ``fake_quant_key``/``fake_quant_value`` (``tests/test_kivi_int4.py:561-632``),
  and hand-computed words for a tiny input.
* ``int8_calc_scales`` / ``int8_quantize`` / ``int8_paged_dequant`` -- the C
  restatement with explicit bf16 round-to-nearest-even, closed forms
  (``inv = 127/amax``), round-half-even known answers, and every positive
  bf16 amax against the two-step ``bf16(bf16(1/amax)*127)``, which differs
  from a single rounded division on some of them.
* ``attention`` -- textbook softmax attention; checked against a float64
  brute-force loop and against ``torch.nn.functional.scaled_dot_product_attention``.
* ``KiviWindowModel`` -- closed forms of the incremental rule
  (``hist_k = ((L-1)//R)*R``, ``hist_v = max(0, L-R)``;
  ``tests/test_kivi_int4.py:1730-1734``), overwrite-without-eviction, FIFO
  value eviction and the bulk-prefill flush.
"""

from __future__ import annotations

import math

import torch

# ---------------------------------------------------------------------------
# a3: KIVI int4 quantization math
# ---------------------------------------------------------------------------


def group_scale(mn: torch.Tensor, mx: torch.Tensor) -> torch.Tensor:
    """``max((mx - mn) / 15, 1e-6)``; pkg/methods/kivi_int4/semantics.py:86-93."""
    return ((mx - mn) / 15).clamp(min=1e-6)


def quantize_group(x: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``clamp(floor((x - mn)/scale + 0.5), 0, 15)`` as int32; semantics.py:95-111."""
    return torch.clamp(torch.floor((x - mn) / scale + 0.5), 0, 15).to(torch.int32)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """Eight int4 lanes (last dim) -> one int32, lane L at bits 4L; semantics.py:76-83."""
    q = q.to(torch.int64) & 0xF
    word = torch.zeros(q.shape[:-1], dtype=torch.int64)
    for lane in range(8):
        word |= q[..., lane] << (4 * lane)
    # reinterpret the low 32 bits as signed int32 (lane 7 >= 8 sets the sign bit)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


def unpack_int4(words: torch.Tensor) -> torch.Tensor:
    """int32 -> eight lanes as float32 (new last dim); semantics.py:63-74."""
    w = words.to(torch.int32)
    return torch.stack([(w >> (4 * lane)) & 0xF for lane in range(8)], dim=-1).to(
        torch.float32
    )


def fake_quant_key(key: torch.Tensor, group_size: int) -> torch.Tensor:
    """Token-group quantize+dequantize ``[T, H, D]``; semantics.py:113-135."""
    if key.numel() == 0:
        return key
    t = key.shape[0]
    pad = (group_size - t % group_size) % group_size
    work = key.to(torch.float32)
    if pad:
        work = torch.cat([work, work[-1:].expand(pad, -1, -1)], dim=0)
    grouped = work.view(-1, group_size, *key.shape[1:])
    mn = grouped.amin(dim=1, keepdim=True)
    mx = grouped.amax(dim=1, keepdim=True)
    scale = group_scale(mn, mx)
    q = quantize_group(grouped, mn, scale)
    deq = (q.to(torch.float32) * scale + mn).view(-1, *key.shape[1:])
    return deq[:t].to(key.dtype)


def fake_quant_value(value: torch.Tensor, group_size: int) -> torch.Tensor:
    """Head-dim-group quantize+dequantize ``[T, H, D]``; semantics.py:137-154."""
    if value.numel() == 0:
        return value
    d = value.shape[-1]
    work = value.to(torch.float32)
    grouped = work.view(*work.shape[:-1], -1, group_size)
    mn = grouped.amin(dim=-1, keepdim=True)
    mx = grouped.amax(dim=-1, keepdim=True)
    scale = group_scale(mn, mx)
    q = quantize_group(grouped, mn, scale)
    deq = (q.to(torch.float32) * scale + mn).view(*work.shape)
    return deq[..., :d].to(value.dtype)


# ---------------------------------------------------------------------------
# a4 / a5: pack kernels (index math of pkg/ops/triton/kivi_pack.py)
# ---------------------------------------------------------------------------


def pack_key_cache(
    key: torch.Tensor,
    slots: torch.Tensor,
    k_quant: torch.Tensor,
    k_scale: torch.Tensor,
    k_mn: torch.Tensor,
    group_size: int,
) -> None:
    """Token-group key pack into ``k_quant[NB,KVH,D,Bs/8]`` (in place).

    Follows ``pkg/ops/triton/kivi_pack.py:161-226``: per group of G tokens the
    first slot picks (block, offset); min/max run over the G tokens per
    (head, dim); word ``(offset + 8j)/8`` packs tokens ``8j..8j+7`` with lane =
    token % 8; scale and min land at ``[blk, h, d, offset/G]``.  Groups whose
    first slot is negative are skipped (``:171``).
    """
    t, kvh, d = key.shape
    if t == 0:
        return
    g = group_size
    bs = k_quant.shape[-1] * 8
    x = key.to(torch.float32).reshape(t // g, g, kvh, d)
    first = slots.reshape(t // g, g)[:, 0].to(torch.int64)
    live = first >= 0
    x, first = x[live], first[live]
    if first.numel() == 0:
        return
    blk = first // bs
    off = first % bs
    mn = x.amin(dim=1)  # [n, KVH, D]
    mx = x.amax(dim=1)
    scale = group_scale(mn, mx)
    q = quantize_group(x, mn.unsqueeze(1), scale.unsqueeze(1))  # [n, G, KVH, D]
    words = pack_int4(q.view(-1, g // 8, 8, kvh, d).permute(0, 3, 4, 1, 2))  # [n,KVH,D,G/8]
    for i in range(first.numel()):
        b, o = int(blk[i]), int(off[i])
        k_quant[b, :, :, o // 8 : o // 8 + g // 8] = words[i]
        k_scale[b, :, :, o // g] = scale[i]
        k_mn[b, :, :, o // g] = mn[i]


def pack_value_cache(
    value: torch.Tensor,
    slots: torch.Tensor,
    v_quant: torch.Tensor,
    v_scale: torch.Tensor,
    v_mn: torch.Tensor,
    group_size: int,
) -> None:
    """Head-dim-group value pack into ``v_quant[NB,Bs,KVH,D/8]`` (in place).

    Follows ``pkg/ops/triton/kivi_pack.py:84-131``: per (token, head, dim group)
    min/max/scale at ``[blk, off, h, g]``; word ``d/8`` packs dims ``8j..8j+7``
    with lane = dim % 8.  Tokens with a negative slot are skipped (``:90``).
    """
    t, kvh, d = value.shape
    if t == 0:
        return
    g = group_size
    bs = v_quant.shape[1]
    s = slots.to(torch.int64)
    live = s >= 0
    x = value.to(torch.float32)[live].reshape(-1, kvh, d // g, g)
    s = s[live]
    if s.numel() == 0:
        return
    mn = x.amin(dim=-1)
    mx = x.amax(dim=-1)
    scale = group_scale(mn, mx)
    q = quantize_group(x, mn.unsqueeze(-1), scale.unsqueeze(-1)).reshape(-1, kvh, d)
    words = pack_int4(q.view(-1, kvh, d // 8, 8))
    blk, off = s // bs, s % bs
    v_quant[blk, off] = words
    v_scale[blk, off] = scale
    v_mn[blk, off] = mn


# ---------------------------------------------------------------------------
# a7 / a8: gather-dequant and residual overlay
# ---------------------------------------------------------------------------


def dequant_gather(
    k_quant: torch.Tensor,
    k_scale: torch.Tensor,
    k_mn: torch.Tensor,
    v_quant: torch.Tensor,
    v_scale: torch.Tensor,
    v_mn: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    target_dtype: torch.dtype,
    group_size: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged int4 history -> dense TND; ``pkg/ops/kivi_gather.py:108-156``.

    Negative block ids read block 0 (``clamp_min(0)``, ``:109``) and are then
    masked away by ``seq_lens``.  Dequant is ``q*scale`` then ``+mn`` as two
    fp32 roundings (``:126``, ``:140``), then a cast to ``target_dtype``.
    """
    nb, kvh, d, pbs = k_quant.shape
    bs = pbs * 8
    batch, maxb = block_table.shape
    ids = block_table.reshape(-1).clamp_min(0).long()
    kq = unpack_int4(k_quant[ids]).view(batch, maxb, kvh, d, bs)
    ks = k_scale[ids].view(batch, maxb, kvh, d, bs // group_size)
    km = k_mn[ids].view(batch, maxb, kvh, d, bs // group_size)
    kb = (kq * ks.repeat_interleave(group_size, -1) + km.repeat_interleave(group_size, -1))
    kb = kb.permute(0, 1, 4, 2, 3)
    vq = unpack_int4(v_quant[ids]).view(batch, maxb, bs, kvh, d)
    vs = v_scale[ids].view(batch, maxb, bs, kvh, d // group_size)
    vm = v_mn[ids].view(batch, maxb, bs, kvh, d // group_size)
    vb = vq * vs.repeat_interleave(group_size, -1) + vm.repeat_interleave(group_size, -1)
    pos = torch.arange(maxb * bs)
    valid = pos.unsqueeze(0) < seq_lens.to(torch.long).unsqueeze(1)
    dk = kb.reshape(batch, maxb * bs, kvh, d)[valid]
    dv = vb.reshape(batch, maxb * bs, kvh, d)[valid]
    return dk.to(target_dtype).contiguous(), dv.to(target_dtype).contiguous()


def overlay_residual(
    dense: torch.Tensor,
    seq_lens: list[int],
    windows: list[torch.Tensor | None],
) -> torch.Tensor:
    """Replace each request's tail by its residual window (FIFO order).

    ``pkg/methods/kivi_int4/attention_backend.py:889-923``: the last
    ``min(L, len(window))`` rows of the request take the window's last rows,
    cast to the dense dtype.
    """
    out = dense.clone()
    start = 0
    for length, win in zip(seq_lens, windows):
        if win is not None and win.shape[0] > 0 and length > 0:
            tail = min(length, win.shape[0])
            out[start + length - tail : start + length] = win[-tail:].to(dense.dtype)
        start += length
    return out


# ---------------------------------------------------------------------------
# a9 / a10 / a13: attention (fp32 SDPA over the dequantized K/V)
# ---------------------------------------------------------------------------


def attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    q_lens: list[int],
    kv_lens: list[int],
    scale: float,
    causal: bool,
) -> torch.Tensor:
    """Per-request ``softmax(q K^T * scale + mask) V`` in fp32, GQA by repeat.

    Same math as the dense path ``attention_backend.py:1341-1392`` (with
    ``_repeat_kv`` ``:941-944`` and the mask of ``semantics.py:285-299``: query
    rows are the last ``q_len`` positions, kv positions past them are masked),
    evaluated in fp32 throughout as the parity criterion asks.
    Inputs are TND: ``query [sum q, Hq, D]``, ``key/value [sum kv, KVH, D]``.
    """
    hq = query.shape[1]
    kvh = key.shape[1]
    rep = hq // kvh
    out = torch.zeros(query.shape, dtype=torch.float32)
    qs = ks = 0
    for ql, kl in zip(q_lens, kv_lens):
        if ql > 0:
            q = query[qs : qs + ql].float().transpose(0, 1)  # [Hq, ql, D]
            k = key[ks : ks + kl].float().repeat_interleave(rep, dim=1).transpose(0, 1)
            v = value[ks : ks + kl].float().repeat_interleave(rep, dim=1).transpose(0, 1)
            s = torch.matmul(q, k.transpose(1, 2)) * scale
            if causal:
                qpos = torch.arange(kl - ql, kl).unsqueeze(1)
                kpos = torch.arange(kl).unsqueeze(0)
                s = s.masked_fill((kpos > qpos).unsqueeze(0), float("-inf"))
            p = torch.softmax(s, dim=-1)
            out[qs : qs + ql] = torch.matmul(p, v).transpose(0, 1)
        qs += ql
        ks += kl
    return out


# ---------------------------------------------------------------------------
# a11 / a12 / a14: INT8 dynamic per-channel
# ---------------------------------------------------------------------------


def int8_calc_scales(key: torch.Tensor, value: torch.Tensor):
    """First-K/V scales in the activation dtype; i8ab.py:130-150.

    Returns ``(k_inv, v_inv, k_aq, v_aq)`` shaped ``[1, KVH, D]`` with
    ``inv = 127 / amax`` (torch evaluates it as ``amax.reciprocal() * 127``,
    each step rounded to the activation dtype) and ``aq = 1 / inv``.
    """
    k_max = key.abs().amax(dim=0, keepdim=True).clamp(min=1e-12)
    v_max = value.abs().amax(dim=0, keepdim=True).clamp(min=1e-12)
    k_inv = 127.0 / k_max
    v_inv = 127.0 / v_max
    return k_inv, v_inv, 1.0 / k_inv, 1.0 / v_inv


def int8_quantize(x: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """``clamp(round(x*inv + 0), -128, 127)`` as int8; i8ab.py:152-171."""
    offset = torch.zeros_like(inv)
    return torch.clamp(torch.round(x * inv + offset), -128, 127).to(torch.int8)


def int8_reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_inv: torch.Tensor,
    v_inv: torch.Tensor,
    slots: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
) -> None:
    """Quantize and scatter into ``[NB, Bs, KVH, D]`` int8 pages by slot.

    The quantize is ``i8ab.py:152-171``; the scatter is the host
    ``reshape_and_cache`` it hands the codes to (``i8ab.py:86-88``): slot
    ``s`` goes to ``[s // Bs, s % Bs]``, negative slots are padding.
    """
    bs = key_cache.shape[1]
    kq = int8_quantize(key, k_inv)
    vq = int8_quantize(value, v_inv)
    s = slots.to(torch.int64)
    live = s >= 0
    key_cache[s[live] // bs, s[live] % bs] = kq[live]
    value_cache[s[live] // bs, s[live] % bs] = vq[live]


def int8_paged_dequant(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    target_dtype: torch.dtype,
    k_inv: torch.Tensor,
    v_inv: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged int8 -> dense TND; i8ab.py:370-404 (``(x - 0) * (1/inv)``).

    With ``target_dtype`` equal to the activation dtype this is the dense
    dequant of the prefill branches.  With ``torch.float32`` it is the
    per-channel antiquant of the fused decode (``i8ab.py:183-199``,
    ``antiquant_mode=0``): ``code * aq`` with ``aq = 1/inv`` still rounded to
    the activation dtype, the product kept in fp32.
    """
    nb, bs, kvh, d = key_cache.shape
    batch, maxb = block_table.shape
    ids = block_table.reshape(-1).long()
    gk = key_cache[ids].view(batch, maxb * bs, kvh * d)
    gv = value_cache[ids].view(batch, maxb * bs, kvh * d)
    pos = torch.arange(maxb * bs)
    valid = (pos.unsqueeze(0) < torch.tensor(seq_lens).unsqueeze(1)).view(-1)
    dk = gk.view(-1, kvh * d)[valid].view(-1, kvh, d)
    dv = gv.view(-1, kvh * d)[valid].view(-1, kvh, d)
    k_off = torch.zeros_like(k_inv)
    v_off = torch.zeros_like(v_inv)
    dk = (dk.to(target_dtype) - k_off) * (1.0 / k_inv)
    dv = (dv.to(target_dtype) - v_off) * (1.0 / v_inv)
    return dk, dv


# ---------------------------------------------------------------------------
# f4: fp8_per_token_head (E4M3 codes, one fp32 scale per (token, head))
# ---------------------------------------------------------------------------

FP8_E4M3_MAX = 448.0


def fp8_pth_scale(x: torch.Tensor) -> torch.Tensor:
    """``[T, KVH, D] -> [T, KVH, 1]``: ``max(amax|x| / 448, 1e-6)`` in fp32;
    pkg/methods/fp8_per_token_head/semantics.py:52-55."""
    amax = x.to(torch.float32).abs().amax(dim=-1, keepdim=True)
    return (amax / FP8_E4M3_MAX).clamp(min=1e-6)


def fp8_pth_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(codes uint8 [T, KVH, D], scale fp32 [T, KVH, 1])``: the E4M3 bytes of
    ``clamp(x / scale, -448, 448)`` (torch's e4m3fn cast, round to nearest
    even); semantics.py:57-61."""
    scale = fp8_pth_scale(x)
    q = (x.to(torch.float32) / scale).clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX)
    return q.to(torch.float8_e4m3fn).view(torch.uint8), scale


def fp8_pth_dequantize(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``float(code) * scale`` in fp32; semantics.py:63-65."""
    return codes.view(torch.float8_e4m3fn).to(torch.float32) * scale


def fp8_pth_store(
    key: torch.Tensor,
    value: torch.Tensor,
    slots: torch.Tensor,
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
) -> None:
    """Quantize ``[T, KVH, D]`` K/V and write codes and scales by slot into the
    ``[NB, Bs, KVH, D]`` / ``[NB, Bs, KVH, 1]`` views; slot ``s`` is page
    ``s // Bs`` row ``s % Bs`` and negative slots are skipped
    (pkg/ops/triton/per_token_head_store.py:163-218)."""
    bs = k_data.shape[1]
    s = slots.to(torch.int64)
    live = s >= 0
    for x, data, scale in ((key, k_data, k_scale), (value, v_data, v_scale)):
        codes, sc = fp8_pth_quantize(x)
        data[s[live] // bs, s[live] % bs] = codes[live]
        scale[s[live] // bs, s[live] % bs] = sc[live]


def fp8_pth_gather(
    k_data: torch.Tensor,
    k_scale: torch.Tensor,
    v_data: torch.Tensor,
    v_scale: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: list[int],
    target_dtype: torch.dtype,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Paged codes -> dense TND ``[sum L, KVH, D]``: ``dequantize`` then
    ``.to(target_dtype)``, as ``fake_quant`` reads a code back
    (semantics.py:63-70), for positions ``p < L`` of each request at slot
    ``table[b, p // Bs] * Bs + p % Bs``; negative ids read page 0 as the
    KIVI gather does (pkg/ops/kivi_gather.py:109)."""
    bs = k_data.shape[1]
    outs = []
    for data, scale in ((k_data, k_scale), (v_data, v_scale)):
        rows = []
        for b, n in enumerate(seq_lens):
            p = torch.arange(int(n))
            blk = block_table[b, p // bs].to(torch.int64).clamp(min=0)
            rows.append(fp8_pth_dequantize(data[blk, p % bs], scale[blk, p % bs]))
        dense = torch.cat(rows) if rows else data.new_zeros((0,) + data.shape[2:])
        outs.append(dense.to(target_dtype))
    return outs[0], outs[1]


# ---------------------------------------------------------------------------
# a6: residual window state (incremental rule) -- a reference-free model
# ---------------------------------------------------------------------------


class KiviWindowModel:
    """Sequential model of one request's residual windows.

    Restates the per-slot semantics of ``_store_kivi_residual_entries``
    (``attention_backend.py:411-462``): a slot already held is overwritten in
    place; otherwise, while the window is full, keys flush the whole window
    and values evict the single oldest entry (``:448-455``); then the token is
    appended.  The bulk prefill writer (``:608-674``) flushes
    ``floor(n/R)*R`` tokens straight to history first.  ``history_k`` /
    ``history_v`` record ``(slot, row)`` pairs in flush order.
    """

    def __init__(self, residual_length: int) -> None:
        self.r = residual_length
        self.win = {True: [], False: []}  # is_key -> list of (slot, row)
        self.history = {True: [], False: []}

    def store(self, rows: torch.Tensor, slots: list[int], *, is_key: bool) -> None:
        win = self.win[is_key]
        for i, slot in enumerate(slots):
            held = [j for j, (s, _) in enumerate(win) if s == slot]
            if held:
                win[held[0]] = (slot, rows[i])
                continue
            while len(win) >= self.r:
                count = self.r if is_key else 1
                self.history[is_key].extend(win[:count])
                del win[:count]
            win.append((slot, rows[i]))

    def write(self, key: torch.Tensor, value: torch.Tensor, slots: list[int]) -> None:
        self.store(key, slots, is_key=True)
        self.store(value, slots, is_key=False)

    def write_prefill(self, key: torch.Tensor, value: torch.Tensor, slots: list[int]) -> None:
        n = len(slots)
        flush = (n // self.r) * self.r
        for i in range(flush):
            self.history[True].append((slots[i], key[i]))
            self.history[False].append((slots[i], value[i]))
        if flush < n:
            self.write(key[flush:], value[flush:], slots[flush:])


def incremental_split(length: int, residual_length: int) -> tuple[int, int]:
    """``(hist_k, hist_v)`` after ``length`` one-token writes.

    Closed form of the incremental rule (``tests/test_kivi_int4.py:1730-1734``).
    """
    r = residual_length
    return ((length - 1) // r) * r if length > 0 else 0, max(0, length - r)


def algorithmic_bytes_int4_decode(
    hist_k: int, hist_v: int, res_k: int, res_v: int, kvh: int, d: int, g: int,
    hq: int, bs: int, res_elem: int = 2, q_elem: int = 2,
) -> int:
    """Bytes one request's INT4 decode must move (per the measurement plan)."""
    s = d // 2 + 8 * d // g
    length = hist_k + res_k
    return (
        (hist_k + hist_v) * kvh * s
        + (res_k + res_v) * kvh * d * res_elem
        + 2 * hq * d * q_elem
        + 4 * math.ceil(length / bs)
    )


__all__ = [
    "KiviWindowModel",
    "algorithmic_bytes_int4_decode",
    "attention",
    "dequant_gather",
    "fake_quant_key",
    "fake_quant_value",
    "group_scale",
    "incremental_split",
    "int8_calc_scales",
    "int8_paged_dequant",
    "int8_quantize",
    "int8_reshape_and_cache",
    "overlay_residual",
    "pack_int4",
    "pack_key_cache",
    "pack_value_cache",
    "quantize_group",
    "unpack_int4",
]
