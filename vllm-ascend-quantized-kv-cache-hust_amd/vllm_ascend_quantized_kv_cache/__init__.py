# SPDX-License-Identifier: Apache-2.0
"""Quantized KV-cache plugin for vLLM, rebuilt for AMD MI355X (gfx950).

Importing the package is lazy: no torch, no host modules, no device library.
The public surface mirrors the reference plugin
(``src/vllm_ascend_quantized_kv_cache/__init__.py:34-126``)::

    from vllm_ascend_quantized_kv_cache import kv_methods
    kv_methods.list()
    kv_methods.get("kivi_int4", group_size=64, residual_length=64)
    kv_methods.activate("kivi_int4", host="vllm_ascend_hust")

Device work (pack, gather-dequant, fused decode and prefill attention) runs in
the in-tree HIP library ``_lib/libkvq_hip.so`` reached through ``ops``.
"""

from ._version import __version__
from .core import VLLM_ASCEND_HUST
from .dtypes import (
    KVCacheLayout,
    KVQuantMode,
    get_kv_quant_mode,
    is_quantized_kv_cache,
    resolve_layout,
)
from .methods.base import KvQuantMethod


def _load_methods() -> None:
    from . import methods  # noqa: F401  (registration side effect)


class _KvMethodsFacade:
    """Discovery / configuration / activation entry points."""

    @staticmethod
    def get(name: str, **config) -> KvQuantMethod:
        _load_methods()
        from .methods.registry import get_method

        return get_method(name, **config)

    @staticmethod
    def list(host: str | None = None) -> list[str]:
        _load_methods()
        from .methods.registry import list_methods

        return list(list_methods(host))

    @staticmethod
    def describe(name: str) -> dict:
        _load_methods()
        from .methods.registry import get_spec

        return get_spec(name).describe()

    @staticmethod
    def describe_all(host: str | None = None) -> dict[str, dict]:
        _load_methods()
        from .methods.registry import get_spec, list_methods

        return {n: get_spec(n).describe() for n in list_methods(host)}

    @staticmethod
    def reset() -> None:
        from .methods.registry import reset_registry

        reset_registry()

    @staticmethod
    def activate(name: str, *, host: str | None = None, **config) -> dict:
        _load_methods()
        from .core.activation import activate as _activate

        return _activate(name, host=host, **config)


kv_methods = _KvMethodsFacade()

__all__ = [
    "KVCacheLayout",
    "KVQuantMode",
    "KvQuantMethod",
    "VLLM_ASCEND_HUST",
    "__version__",
    "get_kv_quant_mode",
    "is_quantized_kv_cache",
    "kv_methods",
    "resolve_layout",
]
