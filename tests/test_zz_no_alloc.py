# SPDX-License-Identifier: Apache-2.0
"""The allocation-free decode entry point ``kvq_kivi_decode_attn_noalloc``.

It must give exactly what ``kvq_kivi_decode_attn`` gives with a caller
workspace (same kernels, same plan), on two calls in a row -- the second
smaller, over the partials the first left in the shared static scratch --
and refuse a work list whose partials exceed the scratch before launching.
"""

from __future__ import annotations

import pytest
import torch

from tests._util import to_dev
from tests.test_gpu_kivi_kernels import _ring_case
from vllm_ascend_quantized_kv_cache.ops import _native
from vllm_ascend_quantized_kv_cache.ops.kivi_decode import (
    DecodeSeq,
    kivi_decode_attention,
    plan_decode,
)

pytestmark = pytest.mark.gpu


def _noalloc(q, caches, table, meta, work, pieces, ring_k, ring_v, scale, g, out):
    kq, ks, km, vq, vs, vm = caches
    batch, hq, d = q.shape
    nb, kvh, _, pbs = kq.shape
    return _native.lib().kvq_kivi_decode_attn_noalloc(
        _native.ptr(q), _native.dtype_code(q.dtype), batch, hq, kvh, d, float(scale),
        _native.ptr(kq), _native.ptr(ks), _native.ptr(km), _native.ptr(vq), _native.ptr(vs),
        _native.ptr(vm), nb, pbs * 8, g, _native.ptr(table), table.shape[1], _native.ptr(meta),
        _native.ptr(work), work.shape[0], _native.ptr(pieces),
        0 if pieces is None else pieces.numel() - 1, _native.ptr(ring_k), _native.ptr(ring_v),
        _native.dtype_code(ring_k.dtype), ring_k.shape[1], _native.ptr(out),
        _native.stream_of(q),
    )


def _case(dev, lens, seed, hq_per_kv=5, kvh=8, g=128, bs=128):
    d, r_len = 128, 128
    cpu, table, ring_k, ring_v, seqs, *_ = _ring_case(dev, d, kvh, g, bs, r_len, lens, seed=seed,
                                                     ring_dtype=torch.bfloat16)
    hq = kvh * hq_per_kv
    q = torch.randn(len(lens), hq, d, generator=torch.Generator().manual_seed(seed)).to(
        torch.bfloat16)
    dseqs = [DecodeSeq(*s) for s in seqs]
    meta, work, pieces = plan_decode(dseqs, kvh, torch.cuda.get_device_properties(dev)
                                     .multi_processor_count)
    return dict(q=q.to(dev), caches=to_dev(cpu, dev), table=table.to(dev),
                meta=torch.from_numpy(meta).to(dev), work=torch.from_numpy(work).to(dev),
                pieces=None if pieces is None else torch.from_numpy(pieces).to(dev),
                ring_k=ring_k.to(dev), ring_v=ring_v.to(dev), scale=d ** -0.5, g=g)


def test_noalloc_decode_equals_workspace_entry_point_twice(gpu_device):
    big = _case(gpu_device, [3000, 129, 1700, 640, 2049, 77], seed=11)
    small = _case(gpu_device, [300, 1030], seed=12)
    for c in (big, small):
        want = kivi_decode_attention(c["q"], c["caches"], c["table"], [], c["ring_k"],
                                     c["ring_v"], c["scale"], c["g"],
                                     plan=(c["meta"], c["work"], c["pieces"]))
        got = torch.full_like(c["q"], float("nan"))
        rc = _noalloc(c["q"], c["caches"], c["table"], c["meta"], c["work"], c["pieces"],
                      c["ring_k"], c["ring_v"], c["scale"], c["g"], got)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_decode_refuses_work_beyond_scratch(gpu_device):
    c = _case(gpu_device, [200], seed=13)
    d, hq = 128, c["q"].shape[1]
    per_item = _native.lib().kvq_kivi_decode_workspace_bytes(1, hq, d)
    too_many = _native.KVQ_DECODE_SCRATCH_BYTES // per_item + 1
    assert _native.lib().kvq_kivi_decode_workspace_bytes(too_many, hq, d) > \
        _native.KVQ_DECODE_SCRATCH_BYTES
    # the size check comes first: nothing is launched, so the short work list
    # is never read past its end
    out = torch.zeros_like(c["q"])
    work = c["work"]
    rc = _native.lib().kvq_kivi_decode_attn_noalloc(
        _native.ptr(c["q"]), _native.dtype_code(c["q"].dtype), 1, hq, 8, d, c["scale"],
        *[_native.ptr(t) for t in c["caches"]], c["caches"][0].shape[0], 128, c["g"],
        _native.ptr(c["table"]), c["table"].shape[1], _native.ptr(c["meta"]), _native.ptr(work),
        too_many, None, 0, _native.ptr(c["ring_k"]), _native.ptr(c["ring_v"]),
        _native.dtype_code(c["ring_k"].dtype), c["ring_k"].shape[1], _native.ptr(out),
        _native.stream_of(c["q"]))
    assert rc == _native.KVQ_ERR_SCRATCH
    torch.cuda.synchronize()
    assert not out.any()
