# SPDX-License-Identifier: Apache-2.0
"""Release version of the MI355X build of the quantized-KV plugin.

The manifest's ``bundle_version`` and the packaging metadata both read this
value (reference: ``src/vllm_ascend_quantized_kv_cache/_version.py:9``).
"""

__version__ = "0.2.0rc4+mi355x"
