# SPDX-License-Identifier: Apache-2.0
"""Shared adapter type: binds one method to one host stack.

Host imports happen only inside methods, never at module import
(``src/vllm_ascend_quantized_kv_cache/adapters/base.py:11-44``).
"""

from __future__ import annotations

import importlib.util
from typing import Any


class HostAdapter:
    host: str = ""
    host_module: str = ""

    def __init__(self, method: Any) -> None:
        self.method = method

    @classmethod
    def available(cls) -> bool:
        try:
            return importlib.util.find_spec(cls.host_module) is not None
        except (ImportError, ValueError):
            return False

    def require_host(self) -> None:
        if not self.available():
            raise RuntimeError(
                f"host adapter {type(self).__name__} requires "
                f"{self.host_module!r}, which is not importable in this environment"
            )

    def register(self, **options: Any) -> dict[str, Any]:
        raise NotImplementedError


__all__ = ["HostAdapter"]
