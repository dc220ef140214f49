# SPDX-License-Identifier: Apache-2.0
"""Method model: immutable config, static spec and the per-method handle.

Torch-free on purpose (discovery must work without a device stack).  The
shape of these types is the plugin's discovery interface, kept as in
``src/vllm_ascend_quantized_kv_cache/methods/base.py:22-181``.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass, field, replace
from typing import Any

from ..core.hosts import ALL_HOSTS
from ..dtypes import KVCacheLayout, KVQuantMode, resolve_layout


@dataclass(frozen=True)
class MethodConfig:
    """Geometry shared by every method (defaults: the production geometry)."""

    head_size: int = 128
    num_kv_heads: int = 8
    num_heads: int = 32
    block_size: int = 128
    group_size: int = 128
    residual_length: int = 128

    def validated(self) -> MethodConfig:
        for name in ("head_size", "num_kv_heads", "block_size", "group_size"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive, got {getattr(self, name)}")
        if self.num_heads < self.num_kv_heads:
            raise ValueError(
                "num_heads must be >= num_kv_heads, got "
                f"{self.num_heads} < {self.num_kv_heads}"
            )
        if self.residual_length < 0:
            raise ValueError(
                f"residual_length must be non-negative, got {self.residual_length}"
            )
        return self


_CONFIG_FIELDS = (
    "head_size",
    "num_kv_heads",
    "num_heads",
    "block_size",
    "group_size",
    "residual_length",
)


@dataclass(frozen=True)
class MethodSpec:
    """Static descriptor of one method; holds only lazy references."""

    name: str
    dtype: str
    summary: str
    provenance: str
    quant_mode: KVQuantMode
    supports: tuple[str, ...]
    requires_gpu_kernels: bool = True
    config_validator: Callable[[MethodConfig], None] | None = None
    semantics_loader: Callable[[Any], Any] | None = None
    adapter_factories: Mapping[str, Callable[[Any], Any]] = field(default_factory=dict)

    def describe(self) -> dict[str, Any]:
        return {
            "name": self.name,
            "dtype": self.dtype,
            "quant_mode": int(self.quant_mode),
            "summary": self.summary,
            "provenance": self.provenance,
            "requires_gpu_kernels": self.requires_gpu_kernels,
            "supports": list(self.supports),
        }


class KvQuantMethod:
    """A configured method: layout contract, semantics and host adapter."""

    def __init__(self, spec: MethodSpec, config: MethodConfig) -> None:
        if spec.config_validator is not None:
            spec.config_validator(config)
        self.spec = spec
        self.config = config.validated()

    @property
    def name(self) -> str:
        return self.spec.name

    @property
    def descriptor(self) -> dict[str, Any]:
        payload = self.spec.describe()
        payload["config"] = {f: getattr(self.config, f) for f in _CONFIG_FIELDS}
        return payload

    def supports(self, host: str) -> bool:
        return host in self.spec.supports

    def resolve_layout(self) -> KVCacheLayout:
        return resolve_layout(self.spec.dtype, self.config.head_size)

    @property
    def semantics(self) -> Any:
        if self.spec.semantics_loader is None:
            raise ValueError(f"method {self.spec.name!r} exposes no semantics module")
        return self.spec.semantics_loader(self.config)

    def host_adapter(self, host: str) -> Any:
        if host not in ALL_HOSTS:
            raise ValueError(f"unknown host {host!r}; known hosts: {', '.join(ALL_HOSTS)}")
        if not self.supports(host):
            raise ValueError(
                f"method {self.spec.name!r} does not support host {host!r} "
                f"(supports: {', '.join(self.spec.supports) or 'none'})"
            )
        factory = self.spec.adapter_factories.get(host)
        if factory is None:
            raise ValueError(
                f"method {self.spec.name!r} has no adapter wired for host {host!r} yet"
            )
        return factory(self)

    def with_config(self, **overrides: Any) -> KvQuantMethod:
        return KvQuantMethod(self.spec, replace(self.config, **overrides))


__all__ = ["KvQuantMethod", "MethodConfig", "MethodSpec"]
