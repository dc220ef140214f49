# SPDX-License-Identifier: Apache-2.0
"""Cache-dtype dispatch on the host attention backend.

One patched ``get_impl_cls`` serves both quantized schemes: the
``--kv-cache-dtype`` literal picks the plugin implementation and every other
literal goes to the host's original factory.  The dispatch contract (marker
attribute, idempotence, context-parallel refusal, mixin-before-host MRO) is
the one of ``src/vllm_ascend_quantized_kv_cache/adapters/vllm_ascend_hust/backend.py:15-190``;
the mixins it composes call the MI355X HIP kernels instead of NPU operators.
"""

from __future__ import annotations

import importlib
from collections.abc import Callable
from functools import cache
from typing import Any

_DISPATCH_MARKER = "_quantized_kv_plugin_dispatch_installed"
_ORIGINAL_IMPL_GETTER = "_quantized_kv_original_get_impl_cls"

_INT8_CACHE_DTYPE = "int8"
_KIVI_CACHE_DTYPE = "kivi_int4"


def _require_cache_dtype(expected: str) -> None:
    from vllm.config import get_current_vllm_config

    cache_dtype = get_current_vllm_config().cache_config.cache_dtype
    if cache_dtype != expected:
        raise RuntimeError(
            f"the quantized KV plugin backend {expected!r} is selected only by "
            f"--kv-cache-dtype {expected}; got {cache_dtype!r}"
        )


def _host_attention_v1():
    """The host's ``attention_v1`` module.

    ``vllm_ascend.ops`` is imported first: on the pinned host revision the
    attention module cannot be the first ``vllm_ascend`` import (circular
    import through its device-op layer).
    """
    importlib.import_module("vllm_ascend.ops")
    return importlib.import_module("vllm_ascend.attention.attention_v1")


def _context_parallel_enabled() -> bool:
    """Host context-parallel state across host revisions.

    Older hosts expose ``enable_cp()``; newer ones split it into
    ``enable_dcp()`` / ``enable_pcp()``.  Neither present is an error.
    """
    from vllm_ascend.attention import utils as attention_utils

    enable_cp = getattr(attention_utils, "enable_cp", None)
    if enable_cp is not None:
        return bool(enable_cp())
    probes = [
        getattr(attention_utils, n)
        for n in ("enable_dcp", "enable_pcp")
        if hasattr(attention_utils, n)
    ]
    if not probes:
        raise RuntimeError(
            "Cannot detect context parallel: vllm_ascend.attention.utils "
            "exposes neither enable_cp() nor enable_dcp()/enable_pcp()."
        )
    return any(bool(fn()) for fn in probes)


@cache
def _build_int8_impl_cls() -> type:
    host_impl = _host_attention_v1().AscendAttentionBackendImpl
    from ...methods.int8_dynamic.attention_backend import (
        AscendInt8AttentionBackendMixin,
    )

    class AscendInt8KvAttentionImpl(AscendInt8AttentionBackendMixin, host_impl):
        """INT8 KV attention: plugin mixin over the live host implementation."""

    return AscendInt8KvAttentionImpl


@cache
def _build_kivi_impl_cls() -> type:
    """INT4 mixin over the host impl; KIVI state reads the host vllm_config."""
    host_impl = _host_attention_v1().AscendAttentionBackendImpl
    from ...methods.kivi_int4.attention_backend import (
        AscendKiviInt4AttentionBackendMixin,
    )

    class AscendKiviInt4KvAttentionImpl(AscendKiviInt4AttentionBackendMixin, host_impl):
        """KIVI INT4 KV attention: plugin mixin over the live host implementation."""

        def __init__(self, *args: Any, **kwargs: Any) -> None:
            super().__init__(*args, **kwargs)
            self._init_kivi_state(_KIVI_CACHE_DTYPE, getattr(self, "vllm_config", None))

    return AscendKiviInt4KvAttentionImpl


_IMPL_BUILDERS: dict[str, Callable[[], type]] = {
    _INT8_CACHE_DTYPE: _build_int8_impl_cls,
    _KIVI_CACHE_DTYPE: _build_kivi_impl_cls,
}


def install_kv_impl_dispatch() -> type:
    """Patch ``AscendAttentionBackend.get_impl_cls`` once (idempotent)."""
    from vllm.config import get_current_vllm_config

    backend_cls = _host_attention_v1().AscendAttentionBackend
    if getattr(backend_cls, _DISPATCH_MARKER, False):
        return backend_cls

    original = backend_cls.get_impl_cls

    def get_impl_cls() -> type:
        cache_dtype = get_current_vllm_config().cache_config.cache_dtype
        builder = _IMPL_BUILDERS.get(cache_dtype)
        if builder is None:
            return original()
        if _context_parallel_enabled():
            raise NotImplementedError(
                f"KV cache {cache_dtype} does not support context parallel yet."
            )
        return builder()

    setattr(backend_cls, _ORIGINAL_IMPL_GETTER, original)
    backend_cls.get_impl_cls = staticmethod(get_impl_cls)
    setattr(backend_cls, _DISPATCH_MARKER, True)
    return backend_cls


def _build_backend_cls(cache_dtype: str, class_name: str) -> type:
    base = _host_attention_v1().AscendAttentionBackend

    class _KvAttentionBackend(base):
        @staticmethod
        def get_impl_cls() -> type:
            _require_cache_dtype(cache_dtype)
            return _IMPL_BUILDERS[cache_dtype]()

    _KvAttentionBackend.__name__ = class_name
    _KvAttentionBackend.__qualname__ = class_name
    _KvAttentionBackend.__doc__ = (
        f"Backend activated exclusively by ``--kv-cache-dtype {cache_dtype}``."
    )
    return _KvAttentionBackend


_BACKENDS_BY_CLASS_NAME = {
    "AscendInt8KvAttentionBackend": _INT8_CACHE_DTYPE,
    "AscendKiviInt4KvAttentionBackend": _KIVI_CACHE_DTYPE,
}


def __getattr__(name: str) -> Any:
    cache_dtype = _BACKENDS_BY_CLASS_NAME.get(name)
    if cache_dtype is not None:
        return _build_backend_cls(cache_dtype, name)
    raise AttributeError(name)


__all__ = ["install_kv_impl_dispatch"]
