# SPDX-License-Identifier: Apache-2.0
"""Plugin surface: discovery, layout contract and host dispatch (no GPU, no vLLM).

Mirrors the reference's ``tests/test_plugin.py``: the host modules the
dispatcher touches are installed as stubs, so the dispatch table -- the
plugin's only runtime switch -- stays under test without a host install.
"""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest

from vllm_ascend_quantized_kv_cache import KVQuantMode, bootstrap, kv_methods, resolve_layout
from vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.register import (
    BACKEND_CLASS_PATH_BY_DTYPE,
)

PKG = Path(__file__).resolve().parents[1] / "vllm-ascend-quantized-kv-cache-hust_amd"
#: every method the registry knows, including the scheme with no host adapter
KNOWN = ["fp8_per_token_head", "int8_dynamic", "kivi_int4"]
#: the methods bootstrap routes (adapter wired, literal selectable)
ROUTABLE = ["int8_dynamic", "kivi_int4"]


def test_published_methods_and_dtypes():
    assert kv_methods.list() == KNOWN
    assert kv_methods.list(host="vllm_ascend_hust") == KNOWN
    assert kv_methods.describe("int8_dynamic")["dtype"] == "int8"
    assert kv_methods.describe("kivi_int4")["dtype"] == "kivi_int4"
    with pytest.raises(ValueError, match="unknown quantized KV method"):
        kv_methods.get("fp8_e4m3")


def test_layout_contract():
    layout = resolve_layout("int8", 128)
    assert (layout.storage_dtype, layout.packed_last_dim) == ("int8", 128)
    assert layout.quant_mode is KVQuantMode.INT8_PER_TENSOR
    layout = resolve_layout("kivi_int4", 128)
    assert (layout.storage_dtype, layout.packed_last_dim) == ("uint8", 64)
    assert layout.quant_mode is KVQuantMode.KIVI_INT4
    with pytest.raises(ValueError, match="positive even"):
        resolve_layout("kivi_int4", 127)
    with pytest.raises(ValueError, match="not a registered"):
        resolve_layout("int4", 128)


def test_kivi_method_config_validators_are_wired():
    method = kv_methods.get("kivi_int4", head_size=64, group_size=32)
    assert method.descriptor["config"]["residual_length"] == 128
    with pytest.raises(ValueError, match="divisible by 8"):
        kv_methods.get("kivi_int4", head_size=12)
    with pytest.raises(ValueError, match="residual_length"):
        kv_methods.get("kivi_int4", group_size=64, residual_length=32)


def test_bootstrap_is_noop_without_host(monkeypatch):
    monkeypatch.setattr(bootstrap, "detect_host", lambda: None)
    assert bootstrap.register_plugins() == []


def test_bootstrap_registers_every_quantized_kv_backend(monkeypatch):
    import vllm_ascend_quantized_kv_cache.core.activation as activation

    calls = []
    monkeypatch.setattr(bootstrap, "detect_host", lambda: bootstrap.VLLM_ASCEND_HUST)
    monkeypatch.setattr(activation, "activate",
                        lambda name, host: calls.append((name, host)) or {})
    assert bootstrap.register_plugins() == ROUTABLE
    assert calls == [(n, "vllm_ascend_hust") for n in ROUTABLE]


@pytest.mark.parametrize("method_name", ROUTABLE)
def test_adapter_installs_host_impl_dispatch(method_name, monkeypatch):
    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    class HostBackend:
        pass

    installed = []
    monkeypatch.setattr(backend, "install_kv_impl_dispatch",
                        lambda: installed.append(True) or HostBackend)
    method = kv_methods.get(method_name)
    adapter = method.host_adapter("vllm_ascend_hust")
    monkeypatch.setattr(adapter, "require_host", lambda: None)
    info = adapter.register()
    assert installed == [True]
    assert info["integration"] == "host_get_impl_cls_dispatch"
    assert info["method"] == method_name
    dtype = method.spec.dtype
    assert info["cache_dtype_literal"] == dtype
    assert info["backend_class_path"] == BACKEND_CLASS_PATH_BY_DTYPE[dtype]
    assert f"--kv-cache-dtype {dtype}" in info["usage"]


@pytest.fixture
def host_stack(monkeypatch):
    import types

    def stub(name):
        module = types.ModuleType(name)
        monkeypatch.setitem(sys.modules, name, module)
        return module

    vllm = stub("vllm")
    vllm.config = stub("vllm.config")
    stub("vllm_ascend")
    stub("vllm_ascend.attention")
    stub("vllm_ascend.ops")
    attention_v1 = stub("vllm_ascend.attention.attention_v1")
    utils = stub("vllm_ascend.attention.utils")

    class HostImpl:
        pass

    class HostBackend:
        @staticmethod
        def get_impl_cls():
            return HostImpl

    attention_v1.AscendAttentionBackend = HostBackend
    cache_config = SimpleNamespace(cache_dtype="auto")
    vllm.config.get_current_vllm_config = lambda: SimpleNamespace(cache_config=cache_config)
    utils.enable_cp = lambda: False
    return SimpleNamespace(backend=HostBackend, host_impl=HostImpl, cache_config=cache_config)


def test_dispatch_selects_plugin_only_for_quantized_dtypes(monkeypatch, host_stack):
    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    class Int8Impl:
        pass

    class KiviImpl:
        pass

    monkeypatch.setitem(backend._IMPL_BUILDERS, "int8", lambda: Int8Impl)
    monkeypatch.setitem(backend._IMPL_BUILDERS, "kivi_int4", lambda: KiviImpl)
    assert backend.install_kv_impl_dispatch() is host_stack.backend
    host_stack.cache_config.cache_dtype = "int8"
    assert host_stack.backend.get_impl_cls() is Int8Impl
    host_stack.cache_config.cache_dtype = "kivi_int4"
    assert host_stack.backend.get_impl_cls() is KiviImpl
    host_stack.cache_config.cache_dtype = "auto"
    assert host_stack.backend.get_impl_cls() is host_stack.host_impl
    # loading the plugin again must not stack wrappers
    assert backend.install_kv_impl_dispatch() is host_stack.backend
    assert host_stack.backend.get_impl_cls() is host_stack.host_impl


def test_dispatch_rejects_context_parallel(monkeypatch, host_stack):
    import vllm_ascend.attention.utils as attention_utils

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    host_stack.cache_config.cache_dtype = "kivi_int4"
    monkeypatch.setattr(attention_utils, "enable_cp", lambda: True)
    backend.install_kv_impl_dispatch()
    with pytest.raises(NotImplementedError, match="context parallel"):
        host_stack.backend.get_impl_cls()


def test_dispatch_uses_split_context_parallel_helpers(monkeypatch, host_stack):
    import vllm_ascend.attention.utils as attention_utils

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    class KiviImpl:
        pass

    monkeypatch.setitem(backend._IMPL_BUILDERS, "kivi_int4", lambda: KiviImpl)
    monkeypatch.delattr(attention_utils, "enable_cp")
    monkeypatch.setattr(attention_utils, "enable_dcp", lambda: False, raising=False)
    monkeypatch.setattr(attention_utils, "enable_pcp", lambda: False, raising=False)
    host_stack.cache_config.cache_dtype = "kivi_int4"
    backend.install_kv_impl_dispatch()
    assert host_stack.backend.get_impl_cls() is KiviImpl
    monkeypatch.setattr(attention_utils, "enable_pcp", lambda: True)
    with pytest.raises(NotImplementedError, match="context parallel"):
        host_stack.backend.get_impl_cls()
    host_stack.cache_config.cache_dtype = "auto"
    assert host_stack.backend.get_impl_cls() is host_stack.host_impl


def test_context_parallel_probe_fails_closed_without_helpers(monkeypatch, host_stack):
    import vllm_ascend.attention.utils as attention_utils

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    monkeypatch.delattr(attention_utils, "enable_cp")
    with pytest.raises(RuntimeError, match="enable_dcp"):
        backend._context_parallel_enabled()


def test_registration_imports_host_ops_before_attention_module(monkeypatch, host_stack):
    import importlib

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    touched = []
    real = importlib.import_module

    def spy(name, *args, **kwargs):
        touched.append(name)
        return real(name, *args, **kwargs)

    monkeypatch.setattr(importlib, "import_module", spy)
    module = backend._host_attention_v1()
    assert touched == ["vllm_ascend.ops", "vllm_ascend.attention.attention_v1"]
    assert module.AscendAttentionBackend is host_stack.backend


def test_kivi_impl_composition_turns_on_kivi_state(monkeypatch, host_stack):
    import vllm_ascend.attention.attention_v1 as attention_v1

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    class HostAttentionImpl:
        num_kv_heads = 8
        head_size = 128

        def __init__(self, *args, **kwargs):
            self.host_args = (args, kwargs)
            self.vllm_config = SimpleNamespace(
                cache_config=SimpleNamespace(kivi_group_size=64, kivi_residual_length=64),
                scheduler_config=SimpleNamespace(max_num_seqs=4),
            )

    monkeypatch.setattr(attention_v1, "AscendAttentionBackendImpl", HostAttentionImpl,
                        raising=False)
    backend._build_kivi_impl_cls.cache_clear()
    try:
        impl = backend._build_kivi_impl_cls()()
        assert impl.enable_kivi is True
        assert (impl.kivi_group_size, impl.kivi_residual_length) == (64, 64)
        assert impl.kivi_max_num_seqs == 4
        assert impl.host_args == ((), {})
    finally:
        backend._build_kivi_impl_cls.cache_clear()


def test_shipped_dispatch_maps_each_dtype_to_its_own_mixin(monkeypatch, host_stack):
    import vllm_ascend.attention.attention_v1 as attention_v1

    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend
    from vllm_ascend_quantized_kv_cache.methods.int8_dynamic.attention_backend import (
        AscendInt8AttentionBackendMixin,
    )
    from vllm_ascend_quantized_kv_cache.methods.kivi_int4.attention_backend import (
        AscendKiviInt4AttentionBackendMixin,
    )

    assert backend._IMPL_BUILDERS == {"int8": backend._build_int8_impl_cls,
                                      "kivi_int4": backend._build_kivi_impl_cls}

    class HostAttentionImpl:
        def forward(self, *args, **kwargs):
            raise AssertionError("host forward must not run")

        def __init__(self, *args, **kwargs):
            self.vllm_config = None

    monkeypatch.setattr(attention_v1, "AscendAttentionBackendImpl", HostAttentionImpl,
                        raising=False)
    backend._build_kivi_impl_cls.cache_clear()
    backend._build_int8_impl_cls.cache_clear()
    try:
        kivi_cls = backend._build_kivi_impl_cls()
        int8_cls = backend._build_int8_impl_cls()
        assert issubclass(kivi_cls, AscendKiviInt4AttentionBackendMixin)
        assert kivi_cls.forward is AscendKiviInt4AttentionBackendMixin.forward
        assert issubclass(int8_cls, AscendInt8AttentionBackendMixin)
        assert int8_cls.forward is AscendInt8AttentionBackendMixin.forward
        # mixin before the host impl in the MRO
        assert kivi_cls.__mro__.index(AscendKiviInt4AttentionBackendMixin) < \
            kivi_cls.__mro__.index(HostAttentionImpl)
    finally:
        backend._build_kivi_impl_cls.cache_clear()
        backend._build_int8_impl_cls.cache_clear()


def test_backend_classes_resolve_through_module_getattr(monkeypatch, host_stack):
    import vllm_ascend_quantized_kv_cache.adapters.vllm_ascend_hust.backend as backend

    cls = backend.AscendKiviInt4KvAttentionBackend
    assert issubclass(cls, host_stack.backend)
    host_stack.cache_config.cache_dtype = "int8"
    with pytest.raises(RuntimeError, match="--kv-cache-dtype kivi_int4"):
        cls.get_impl_cls()
    with pytest.raises(AttributeError):
        backend.NotABackend  # noqa: B018


def test_bundle_manifest_publishes_both_backends():
    from vllm_ascend_quantized_kv_cache import __version__

    path = PKG / "vllm_ascend_quantized_kv_cache/manifests/vllm-hust-extension-v1.json"
    payload = json.loads(path.read_text())
    assert payload["schema_version"] == "1.0"
    assert payload["host"] == {"provider": "vllm", "name": "vllm-ascend-hust"}
    assert payload["bundle_version"] == __version__
    refs = {c["component_id"]: c["implementation_ref"] for c in payload["components"]}
    assert refs["int8-kv-attention-backend"].endswith(":AscendInt8KvAttentionBackend")
    assert refs["kivi-int4-kv-attention-backend"].endswith(":AscendKiviInt4KvAttentionBackend")


def test_entry_point_is_the_reference_plugin_hook():
    try:
        import tomllib
    except ModuleNotFoundError:
        import tomli as tomllib
    project = tomllib.loads((PKG / "pyproject.toml").read_text())["project"]
    assert project["entry-points"]["vllm.general_plugins"] == {
        "vllm-ascend-quantized-kv-cache": "vllm_ascend_quantized_kv_cache.bootstrap:register_plugins"
    }


def test_lazy_kernel_imports_resolve():
    """Every ``from ...ops.X import`` inside the mixins names a real module."""
    import ast
    import importlib.util

    targets = set()
    for method in ("kivi_int4", "int8_dynamic"):
        src = (PKG / f"vllm_ascend_quantized_kv_cache/methods/{method}/attention_backend.py")
        for node in ast.walk(ast.parse(src.read_text())):
            if isinstance(node, ast.ImportFrom) and node.level == 3 and node.module:
                targets.add(f"vllm_ascend_quantized_kv_cache.{node.module}")
    assert targets
    for module in sorted(targets):
        assert importlib.util.find_spec(module) is not None, module


def test_method_discovery_needs_no_torch():
    program = """
import sys
class _BlockTorch:
    def find_spec(self, name, path=None, target=None):
        if name == "torch" or name.startswith("torch."):
            raise ImportError("torch is blocked")
        return None
sys.meta_path.insert(0, _BlockTorch())
from vllm_ascend_quantized_kv_cache import kv_methods
for name in ("int8_dynamic", "kivi_int4"):
    method = kv_methods.get(name, head_size=128, group_size=64)
    assert method.resolve_layout().packed_last_dim > 0
assert "torch" not in sys.modules
"""
    done = subprocess.run([sys.executable, "-c", program], capture_output=True, text=True,
                          env={"PYTHONPATH": str(PKG), "PATH": "/usr/bin:/bin"})
    assert done.returncode == 0, done.stderr
