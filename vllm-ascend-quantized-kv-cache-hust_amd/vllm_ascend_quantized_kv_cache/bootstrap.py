# SPDX-License-Identifier: Apache-2.0
"""``vllm.general_plugins`` hook.

Installs the cache-dtype dispatch on the host attention backend; quantization
itself turns on only with ``--kv-cache-dtype int8`` or ``kivi_int4``.  Same
behaviour as ``src/vllm_ascend_quantized_kv_cache/bootstrap.py:20-35``: a no-op
in processes without the host stack.
"""

from __future__ import annotations

from .core.hosts import VLLM_ASCEND_HUST, detect_host

REGISTERED_METHODS = ("int8_dynamic", "kivi_int4")


def register_plugins() -> list[str]:
    if detect_host() != VLLM_ASCEND_HUST:
        return []
    from .core import activation

    for name in REGISTERED_METHODS:
        activation.activate(name, host=VLLM_ASCEND_HUST)
    print(
        "[vllm-ascend-quantized-kv] registered quantized KV attention backends "
        "(MI355X HIP kernels); enable one with --kv-cache-dtype "
        f"{', '.join(REGISTERED_METHODS)}",
        flush=True,
    )
    return list(REGISTERED_METHODS)


__all__ = ["REGISTERED_METHODS", "detect_host", "register_plugins"]
