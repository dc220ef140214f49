# SPDX-License-Identifier: Apache-2.0
"""Quantization methods: importing this package registers their metadata.

Only the two routable schemes of the reference are built here
(``src/vllm_ascend_quantized_kv_cache/bootstrap.py:15``): ``int8_dynamic`` and
``kivi_int4``.
"""

from . import int8_dynamic, kivi_int4  # noqa: F401  (registration side effect)

__all__ = ["int8_dynamic", "kivi_int4"]
