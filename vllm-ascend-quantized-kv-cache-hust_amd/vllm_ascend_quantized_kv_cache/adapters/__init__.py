# SPDX-License-Identifier: Apache-2.0
"""Host adapters (lazy: the vllm-ascend-hust subpackage pulls torch)."""

from __future__ import annotations

from .base import HostAdapter


def adapter_for(host: str) -> type[HostAdapter]:
    if host == "vllm_ascend_hust":
        from .vllm_ascend_hust import AscendHustAdapter

        return AscendHustAdapter
    from ..core.hosts import ALL_HOSTS

    raise ValueError(f"unknown host {host!r}; known hosts: {', '.join(ALL_HOSTS)}")


__all__ = ["HostAdapter", "adapter_for"]
