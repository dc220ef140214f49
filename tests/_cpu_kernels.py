# SPDX-License-Identifier: Apache-2.0
"""CPU stand-ins for the mixins' kernel launch hooks, built on the oracle.

Tests only: they let the host state machine (window bookkeeping, flush
planning, metadata) run end to end without a GPU, the way the reference's
tests swap its triton launches for CPU packers
(``tests/test_kivi_int4.py:703-745``).  The real validations stay active.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

from oracle import kvq_oracle as ref

ROOT = Path(__file__).resolve().parents[1]


def install_cpu_kernels(impl) -> dict[str, list]:
    """Replace the KIVI mixin's launch hooks with oracle-backed CPU versions.

    The pack hooks are replaced through their reference signature
    ``(rows, slots)``, so the mixin's flush path hands them materialized rows.
    Returns call logs keyed by hook name.
    """
    calls: dict[str, list] = {"key_pack": [], "value_pack": [], "ring": [], "gather": [],
                              "decode": [], "dense": []}

    def pack_key(key, slots):
        calls["key_pack"].append((key.clone(), slots.clone()))
        ref.pack_key_cache(key, slots, impl.k_quant_cache, impl.k_scale_cache,
                           impl.k_mn_cache, impl.kivi_group_size)

    def pack_value(value, slots):
        calls["value_pack"].append((value.clone(), slots.clone()))
        ref.pack_value_cache(value, slots, impl.v_quant_cache, impl.v_scale_cache,
                             impl.v_mn_cache, impl.kivi_group_size)

    def ring_write(src, src_rows, dst_rows, is_key):
        ring = impl._kivi_ring.tensor(is_key)
        flat = ring.view(-1, *ring.shape[-2:])
        rows = src.reshape(-1, *src.shape[-2:])
        rows = rows if src_rows is None else rows[src_rows.long()]
        calls["ring"].append((is_key, dst_rows.clone()))
        flat[dst_rows.long()] = rows.to(ring.dtype)

    def gather(block_table, cu, total, target_dtype, ring_meta):
        lens = [int(cu[i + 1] - cu[i]) for i in range(len(cu) - 1)]
        calls["gather"].append(lens)
        dk, dv = ref.dequant_gather(*impl._kivi_caches(), block_table, torch.tensor(lens),
                                    target_dtype, impl.kivi_group_size)
        wk, wv = windows_from_meta(impl, ring_meta, lens)
        return ref.overlay_residual(dk, lens, wk), ref.overlay_residual(dv, lens, wv)

    def decode(query, block_table, seqs, out):
        lens = [s.seq_len for s in seqs]
        calls["decode"].append(seqs)
        meta = torch.tensor([[s.ring_row, s.k_first, s.seq_len - s.k_hist, s.v_first,
                              s.seq_len - s.v_hist] for s in seqs])
        dk, dv = ref.dequant_gather(*impl._kivi_caches(), block_table, torch.tensor(lens),
                                    torch.float32, impl.kivi_group_size)
        wk, wv = windows_from_meta(impl, meta, lens)
        dk = ref.overlay_residual(dk, lens, wk)
        dv = ref.overlay_residual(dv, lens, wv)
        res = ref.attention(query, dk, dv, [1] * len(lens), lens, impl.scale, causal=True)
        out.copy_(res.to(out.dtype))
        return out

    def dense(q, k, v, q_lens, kv_lens, causal, out):
        calls["dense"].append((list(q_lens), list(kv_lens), causal))
        res = ref.attention(q, k, v, q_lens, kv_lens, impl.scale, causal)
        out.copy_(res.to(out.dtype))
        return out

    impl._launch_kivi_key_pack = pack_key
    impl._launch_kivi_value_pack = pack_value
    impl._launch_kivi_ring_write = ring_write
    impl._launch_kivi_gather = gather
    impl._launch_kivi_decode = decode
    impl._launch_dense_attention = dense
    return calls


def windows_from_meta(impl, ring_meta, lens):
    """Residual tails named by ``[row, k_first, k_tail, v_first, v_tail]`` rows."""
    ring = impl._kivi_ring
    wk, wv = [], []
    for i in range(len(lens)):
        row, kf, kt, vf, vt = (int(x) for x in ring_meta[i])
        r = ring.ring_len
        wk.append(ring.key[row, [(kf + j) % r for j in range(kt)]] if kt else None)
        wv.append(ring.value[row, [(vf + j) % r for j in range(vt)]] if vt else None)
    return wk, wv


# ---------------------------------------------------------------------------
# the scalar C restatement (oracle/kvq_ref.c), built on demand
# ---------------------------------------------------------------------------

_C = None


def c_oracle() -> ctypes.CDLL:
    global _C
    if _C is None:
        lib = ROOT / "oracle" / "_build" / "libkvq_ref.so"
        if not lib.exists():
            subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
        _C = ctypes.CDLL(str(lib))
    return _C


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def c_pack_key(key_f32, slots, caches, g, bs):
    kq, ks, km = caches
    c_oracle().ref_pack_key(_p(key_f32), ctypes.c_int64(key_f32.shape[0]),
                            ctypes.c_int(key_f32.shape[1]), ctypes.c_int(key_f32.shape[2]),
                            _p(slots), ctypes.c_int(g), ctypes.c_int(bs), _p(kq), _p(ks), _p(km))


def c_pack_value(value_f32, slots, caches, g, bs):
    vq, vs, vm = caches
    c_oracle().ref_pack_value(_p(value_f32), ctypes.c_int64(value_f32.shape[0]),
                              ctypes.c_int(value_f32.shape[1]), ctypes.c_int(value_f32.shape[2]),
                              _p(slots), ctypes.c_int(g), ctypes.c_int(bs), _p(vq), _p(vs), _p(vm))


def c_gather(caches, bs, kvh, d, g, table, seq_lens):
    kq, ks, km, vq, vs, vm = caches
    total = int(seq_lens.sum())
    ok = torch.empty(total, kvh, d)
    ov = torch.empty(total, kvh, d)
    c_oracle().ref_gather(_p(kq), _p(ks), _p(km), _p(vq), _p(vs), _p(vm), ctypes.c_int(bs),
                          ctypes.c_int(kvh), ctypes.c_int(d), ctypes.c_int(g), _p(table),
                          ctypes.c_int64(table.shape[0]), ctypes.c_int64(table.shape[1]),
                          _p(seq_lens), _p(ok), _p(ov))
    return ok, ov


def c_int8_scales_bf16(x_f32):
    t, c = x_f32.shape
    inv = torch.empty(c)
    aq = torch.empty(c)
    c_oracle().ref_int8_scales_bf16(_p(x_f32), ctypes.c_int64(t), ctypes.c_int64(c), _p(inv),
                                    _p(aq))
    return inv, aq


def c_int8_quant_bf16(x_f32, inv):
    t, c = x_f32.shape
    out = torch.empty(t, c, dtype=torch.int8)
    c_oracle().ref_int8_quant_bf16(_p(x_f32), ctypes.c_int64(t), ctypes.c_int64(c), _p(inv),
                                   _p(out))
    return out
