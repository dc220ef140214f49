# SPDX-License-Identifier: Apache-2.0
"""Dense TND attention on MFMA (HIP kernel ``kvq_prefill_attn``).

Stands in for the NPU fused-attention calls with ``input_layout="TND"`` of the
reference (prefill, chunked prompt rows and the dense fallback of
``pkg/methods/kivi_int4/attention_backend.py:1232-1392``; the INT8 prefill
paths of ``pkg/methods/int8_dynamic/attention_backend.py:207-368``).
"""

from __future__ import annotations

import torch

from . import _native


def prefill_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    q_lens: list[int],
    kv_lens: list[int],
    scale: float,
    causal: bool,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-request attention over TND tensors.

    ``query [sum q_lens, Hq, D]``, ``key/value [sum kv_lens, KVH, D]``; query
    row ``i`` of a request is kv position ``kv_len - q_len + i``.
    """
    tq, hq, d = query.shape
    kvh = key.shape[1]
    if out is None:
        out = torch.empty_like(query)
    if tq == 0 or not q_lens:
        return out
    _native.require_gpu_tensors("prefill_attention", query, key, value, out)
    dev = query.device
    cu_q = [0]
    for n in q_lens:
        cu_q.append(cu_q[-1] + int(n))
    cu_k = [0]
    for n in kv_lens:
        cu_k.append(cu_k[-1] + int(n))
    cu = torch.tensor([cu_q, cu_k], dtype=torch.int32).to(dev, non_blocking=True)
    q = query.contiguous()
    k = key.contiguous()
    v = value.to(key.dtype).contiguous()
    if q.dtype != k.dtype:
        k = k.to(q.dtype)
        v = v.to(q.dtype)
    target = out if out.is_contiguous() and out.dtype == q.dtype else torch.empty_like(q)
    rc = _native.lib().kvq_prefill_attn(
        _native.ptr(q), _native.ptr(k), _native.ptr(v), _native.dtype_code(q.dtype),
        _native.ptr(cu[0]), _native.ptr(cu[1]), len(q_lens), max(int(x) for x in q_lens),
        hq, kvh, d, float(scale), 1 if causal else 0, _native.ptr(target),
        _native.stream_of(q),
    )
    _native.check(rc, "kvq_prefill_attn")
    if target is not out:
        out.copy_(target)
    return out


__all__ = ["prefill_attention"]
