# SPDX-License-Identifier: Apache-2.0
"""Quantization methods: importing this package registers their metadata.

The registry knows the reference's three schemes
(``src/vllm_ascend_quantized_kv_cache/methods/__init__.py:17``); two of them
are routable through the host adapter (``bootstrap.REGISTERED_METHODS``,
``src/vllm_ascend_quantized_kv_cache/bootstrap.py:15``): ``int8_dynamic`` and
``kivi_int4``.  ``fp8_per_token_head`` has its HIP store and read path but,
as in the reference, no host adapter.
"""

from . import fp8_per_token_head, int8_dynamic, kivi_int4  # noqa: F401  (registration side effect)

__all__ = ["fp8_per_token_head", "int8_dynamic", "kivi_int4"]
