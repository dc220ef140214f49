# SPDX-License-Identifier: Apache-2.0
"""Single activation pipeline: method name -> host adapter -> ``register()``.

Same contract as ``src/vllm_ascend_quantized_kv_cache/core/activation.py:17-38``:
unknown names, bad configs, unknown or missing hosts all raise immediately.
"""

from __future__ import annotations

from typing import Any


def activate(name: str, *, host: str | None = None, **config: Any) -> dict[str, Any]:
    from ..methods.registry import get_method
    from .hosts import ALL_HOSTS, require_host_stack

    if host is None:
        host = require_host_stack(f"activating method {name!r}")
    elif host not in ALL_HOSTS:
        raise ValueError(f"unknown host {host!r}; known hosts: {', '.join(ALL_HOSTS)}")
    method = get_method(name, **config)
    info = dict(method.host_adapter(host).register())
    info.setdefault("host", host)
    info["method"] = name
    return info


__all__ = ["activate"]
