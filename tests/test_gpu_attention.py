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


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_growing_and_shrinking_row_maxima(gpu_device, d, dtype):
    """Scores that climb by more than the lazy-offset threshold (8 in log2
    units) every 64-key block for half the heads, and fall for the others:
    the rescale branch runs on almost every block of the first half, never
    after the first block of the second, and both match the oracle."""
    from vllm_ascend_quantized_kv_cache.ops.attention import prefill_attention

    g = torch.Generator().manual_seed(11 + d)
    hq, kvh = 8, 2
    q_lens = [96, 200]
    kv_lens = [300, 200]
    n = sum(kv_lens)
    u = torch.randn(kvh, d, generator=g)
    u = u / u.norm(dim=1, keepdim=True)  # unit direction per kv head
    pos = torch.cat([torch.arange(L, dtype=torch.float32) for L in kv_lens])
    # raw score of key j against a query along u: 8 * (+-0.5 j + noise); with
    # scale d^-0.5 that moves the log2 exponent by about 23 / sqrt(d / 64) per block
    sign = torch.tensor([1.0, -1.0])
    k = (u[None] * (sign[None, :, None] * 0.5 * pos[:, None, None])
         + 0.05 * torch.randn(n, kvh, d, generator=g))
    q = 8.0 * u.repeat_interleave(hq // kvh, dim=0)[None] + 0.05 * torch.randn(
        sum(q_lens), hq, d, generator=g)
    v = torch.randn(n, kvh, d, generator=g)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    scale = d ** -0.5
    want = ref.attention(q, k, v, q_lens, kv_lens, scale, True)
    got = prefill_attention(
        q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), q_lens, kv_lens, scale, True
    )
    torch.testing.assert_close(got.float().cpu(), want, atol=1e-2, rtol=1e-2)
