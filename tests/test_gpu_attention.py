# SPDX-License-Identifier: Apache-2.0
"""GPU parity of the MFMA dense (prefill / chunked) attention kernel.

Checked against the oracle's fp32 softmax attention within atol/rtol 1e-2 on
ragged batches, GQA ratios, causal and full masks, and query chunks that sit
at the end of a longer key range (chunked prefill with history).
"""

from __future__ import annotations

import pytest
import torch

from oracle import kvq_oracle as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,kvh", [(8, 8), (40, 8), (8, 1)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_matches_oracle(gpu_device, d, hq, kvh, causal, dtype):
    from vllm_ascend_quantized_kv_cache.ops.attention import prefill_attention

    g = torch.Generator().manual_seed(d + hq)
    q_lens = [1, 37, 130, 64]
    kv_lens = [1, 37, 300, 64] if causal else [5, 37, 300, 64]  # request 2: chunk with history
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(dtype)
    k = (torch.randn(sum(kv_lens), kvh, d, generator=g) * 2).to(dtype)
    v = torch.randn(sum(kv_lens), kvh, d, generator=g).to(dtype)
    scale = d ** -0.5
    want = ref.attention(q, k, v, q_lens, kv_lens, scale, causal)
    got = prefill_attention(
        q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), q_lens, kv_lens, scale, causal
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)


def test_prefill_attention_chunk_after_int4_history(gpu_device):
    """Config-4 shape in miniature: a new chunk attending to a longer prefix."""
    from vllm_ascend_quantized_kv_cache.ops.attention import prefill_attention

    g = torch.Generator().manual_seed(3)
    hq, kvh, d = 40, 8, 128
    q_lens = [256, 128]
    kv_lens = [1280, 640]
    q = torch.randn(sum(q_lens), hq, d, generator=g).to(torch.bfloat16)
    k = (torch.randn(sum(kv_lens), kvh, d, generator=g) * torch.exp(torch.randn(kvh, d, generator=g)))
    k = k.to(torch.bfloat16)
    v = torch.randn(sum(kv_lens), kvh, d, generator=g).to(torch.bfloat16)
    want = ref.attention(q, k, v, q_lens, kv_lens, d ** -0.5, True)
    got = prefill_attention(
        q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), q_lens, kv_lens, d ** -0.5, True
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)
