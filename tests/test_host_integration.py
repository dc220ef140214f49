# SPDX-License-Identifier: Apache-2.0
"""Host page-budget and KV-shape integration of ``kivi_int4`` (CPU).

The host checkouts (vllm-hust, vllm-ascend-hust) are not installed here, so,
as the reference's tests stub the host, small stand-in modules carry the
constructs the four host edits change (``docs/int4-host-integration.md:20-77``
and the serve-time fixes of ``docs/serving-verification-20261003.md:31-45``).
The edits are applied to them, the patched modules are imported, and the
published numbers are checked: S = 72 B and a 147,456-byte page at block 128,
8 kv heads, head and group 128; shape ``(2, NB, Bs, KVH, S)``; two equal
uint8 regions that the KIVI mixin slices into its six views, aliasing the
host's allocation.
"""

from __future__ import annotations

import importlib.util
import sys
import textwrap
from pathlib import Path
from typing import get_args

import pytest
import torch

from vllm_ascend_quantized_kv_cache import host_integration as hi
from vllm_ascend_quantized_kv_cache.methods.kivi_int4 import attention_backend as ab
from vllm_ascend_quantized_kv_cache.methods.kivi_int4.byte_cache import KiviByteCacheLayout

STUBS = {
    ("vllm", "vllm/config/cache.py"): '''
        from typing import Literal

        CacheDType = Literal[
            "auto",
            "bfloat16",
            "fp8",
            "int8",
            "nvfp4",
            "nvfp4_4over6",
        ]
    ''',
    ("vllm", "vllm/utils/torch_utils.py"): '''
        import torch

        STR_DTYPE_TO_TORCH_DTYPE = {
            "float32": torch.float32,
            "half": torch.half,
            "bfloat16": torch.bfloat16,
            "int8": torch.int8,
            "fp8": torch.uint8,
        }


        def is_quantized_kv_cache(kv_cache_dtype: str) -> bool:
            """True for a cache dtype that stores codes, not activations."""
            return (
                kv_cache_dtype.startswith("fp8")
                or kv_cache_dtype == "int8"
                or kv_cache_dtype.startswith("nvfp4")
            )
    ''',
    ("vllm", "vllm/v1/kv_cache_interface.py"): '''
        import enum
        from dataclasses import dataclass


        class KVQuantMode(enum.IntEnum):
            NONE = 0
            INT8_PER_TENSOR = 1
            INT4_PER_TOKEN_HEAD = 9
            NVFP4_DS_MLA = 10  # opaque-bytes NVFP4 DS-MLA layouts (FlashMLA sparse)


        def get_kv_quant_mode(kv_cache_dtype: str) -> KVQuantMode:
            if kv_cache_dtype == "int4_per_token_head":
                return KVQuantMode.INT4_PER_TOKEN_HEAD
            return KVQuantMode.NONE


        @dataclass(frozen=True)
        class FullAttentionSpec:
            block_size: int
            num_kv_heads: int
            head_size: int
            head_size_v: int
            dtype_size: int
            kv_quant_mode: KVQuantMode = KVQuantMode.NONE

            @property
            def real_page_size_bytes(self) -> int:
                if self.kv_quant_mode == KVQuantMode.NONE:
                    last_dim = self.head_size + self.head_size_v
                elif self.kv_quant_mode == KVQuantMode.INT4_PER_TOKEN_HEAD:
                    last_dim = self.head_size // 2 + self.head_size_v // 2
                else:
                    last_dim = self.head_size + self.head_size_v
                return self.block_size * self.num_kv_heads * last_dim * self.dtype_size
    ''',
    ("ascend", "vllm_ascend/attention/attention_v1.py"): '''
        from dataclasses import dataclass, replace


        def get_dtype_size(dtype):
            return 2


        @dataclass(frozen=True)
        class Spec:
            num_kv_heads: int
            head_size: int
            dtype: str
            kv_quant_mode: object = None
            num_head_slots: int = 1
            state_content_bytes: int = 0


        class AscendAttentionBackend:
            @staticmethod
            def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size,
                                   cache_dtype_str="auto"):
                return (2, num_blocks, block_size, num_kv_heads, head_size)

            @staticmethod
            def customize_spec(spec):
                plane_size_bytes = spec.num_kv_heads * spec.head_size * get_dtype_size(spec.dtype)
                return replace(spec, state_content_bytes=plane_size_bytes)
    ''',
    ("ascend", "vllm_ascend/worker/model_runner_v1.py"): '''
        class Runner:
            def __init__(self, vllm_config):
                self.vllm_config = vllm_config

            def kv_shapes(self, attn_backend, current_kv_cache_spec, num_blocks, hybrid=False,
                          block_size_chunk=1, block_size=16):
                if hybrid:
                    if True:
                        kv_cache_shape = attn_backend.get_kv_cache_shape(
                            num_blocks * block_size_chunk,
                            block_size,
                            current_kv_cache_spec.num_kv_heads,
                            current_kv_cache_spec.head_size,
                        )
                else:
                    if True:
                        kv_cache_shape = attn_backend.get_kv_cache_shape(
                            num_blocks,
                            current_kv_cache_spec.block_size,
                            current_kv_cache_spec.num_kv_heads,
                            current_kv_cache_spec.head_size,
                        )
                k_shape = kv_cache_shape[1:]
                v_shape = k_shape
                if hasattr(current_kv_cache_spec, "head_size_v"):
                    v_shape = (*kv_cache_shape[1:-1], current_kv_cache_spec.head_size_v)
                return k_shape, v_shape
    ''',
}


def _trees(tmp: Path) -> tuple[Path, Path]:
    roots = {"vllm": tmp / "vllm-hust", "ascend": tmp / "vllm-ascend-hust"}
    for (tree, rel), body in STUBS.items():
        path = roots[tree] / rel
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(textwrap.dedent(body).lstrip())
    return roots["vllm"], roots["ascend"]


def _load(path: Path, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def test_page_budget_numbers():
    assert hi.kivi_int4_bytes_per_token_head(128, 128) == 72
    assert hi.kivi_int4_bytes_per_token_head(128, 64) == 80
    assert hi.kivi_int4_bytes_per_token_head(256, 128) == 144
    assert hi.kivi_int4_page_size_bytes(128, 8, 128, 128) == 147_456
    assert hi.kivi_int4_kv_cache_shape(7, 128, 8, 128, 128) == (2, 7, 128, 8, 72)
    # the plugin's own layout agrees for every geometry the validators accept
    for d, g, bs, kvh in ((128, 128, 128, 8), (128, 64, 128, 4), (64, 32, 64, 2), (32, 8, 16, 2)):
        lay = KiviByteCacheLayout(5, bs, kvh, d, g)
        assert lay.bytes_per_token_head == hi.kivi_int4_bytes_per_token_head(d, g)
        assert 5 * hi.kivi_int4_page_size_bytes(bs, kvh, d, g) == 2 * lay.region_bytes
    with pytest.raises(ValueError, match="group_size"):
        hi.kivi_int4_bytes_per_token_head(128, 12)


def test_group_size_comes_from_the_environment(monkeypatch):
    monkeypatch.setenv(hi.GROUP_SIZE_ENV, "64")
    assert hi.kivi_int4_kv_cache_shape(3, 128, 8, 128) == (2, 3, 128, 8, 80)


def test_host_edits_apply_and_the_host_allocates_plugin_pages(tmp_path):
    vllm_root, ascend_root = _trees(tmp_path)
    hi.apply_host_edits(vllm_root, ascend_root, check=True)  # verify only
    assert "kivi_int4" not in (vllm_root / "vllm/config/cache.py").read_text()
    changed = hi.apply_host_edits(vllm_root, ascend_root)
    assert len(changed) == 5

    cache = _load(vllm_root / "vllm/config/cache.py", "stub_cache")
    assert "kivi_int4" in get_args(cache.CacheDType)
    assert "fp8" in get_args(cache.CacheDType)

    tu = _load(vllm_root / "vllm/utils/torch_utils.py", "stub_torch_utils")
    assert tu.STR_DTYPE_TO_TORCH_DTYPE["kivi_int4"] is torch.uint8
    assert tu.is_quantized_kv_cache("kivi_int4") and tu.is_quantized_kv_cache("int8")
    assert not tu.is_quantized_kv_cache("auto")

    iface = _load(vllm_root / "vllm/v1/kv_cache_interface.py", "stub_iface")
    mode = iface.get_kv_quant_mode("kivi_int4")
    assert mode is iface.KVQuantMode.KIVI_INT4 and int(mode) == 11
    assert iface.get_kv_quant_mode("int4_per_token_head") is iface.KVQuantMode.INT4_PER_TOKEN_HEAD
    spec = iface.FullAttentionSpec(128, 8, 128, 128, 1, mode)
    assert spec.real_page_size_bytes == 147_456
    dense = iface.FullAttentionSpec(128, 8, 128, 128, 2)
    assert dense.real_page_size_bytes == 128 * 8 * 256 * 2

    attn = _load(ascend_root / "vllm_ascend/attention/attention_v1.py", "stub_attn")
    backend = attn.AscendAttentionBackend
    assert backend.get_kv_cache_shape(7, 128, 8, 128, "kivi_int4") == (2, 7, 128, 8, 72)
    assert backend.get_kv_cache_shape(7, 128, 8, 128, "auto") == (2, 7, 128, 8, 128)
    s = backend.customize_spec(attn.Spec(8, 128, "uint8", mode))
    assert (s.num_head_slots, s.state_content_bytes) == (2, 8 * 72)
    assert backend.customize_spec(attn.Spec(8, 128, "bf16")).state_content_bytes == 8 * 128 * 2

    runner_mod = _load(ascend_root / "vllm_ascend/worker/model_runner_v1.py", "stub_runner")
    calls = []

    class Backend:
        @staticmethod
        def get_kv_cache_shape(*args, **kw):
            calls.append(kw.get("cache_dtype_str"))
            return backend.get_kv_cache_shape(*args, **kw)

    cfg = type("Cfg", (), {"cache_config": type("CC", (), {"cache_dtype": "kivi_int4"})()})()
    kv_spec = type("S", (), dict(block_size=128, num_kv_heads=8, head_size=128,
                                 head_size_v=128))()
    runner = runner_mod.Runner(cfg)
    for hybrid in (False, True):
        k_shape, v_shape = runner.kv_shapes(Backend, kv_spec, 7, hybrid=hybrid, block_size=128)
        assert k_shape == v_shape == (7, 128, 8, 72)
    assert calls == ["kivi_int4", "kivi_int4"]

    # the host's allocation, sliced as the runner slices it, binds the mixin's
    # six views over the host's own bytes
    shape = backend.get_kv_cache_shape(7, 128, 8, 128, "kivi_int4")
    raw = torch.zeros(spec.real_page_size_bytes * 7, dtype=torch.uint8)
    kv = raw.view(shape)

    class Impl(ab.AscendKiviInt4AttentionBackendMixin):
        pass

    impl = Impl()
    impl.num_heads = impl.num_kv_heads = 8
    impl.head_size = 128
    impl._init_kivi_state("kivi_int4")
    impl._bind_kivi_cache((kv[0], kv[1]))
    assert impl.k_quant_cache.shape == (7, 8, 128, 16)
    assert impl.v_scale_cache.shape == (7, 128, 8, 1)
    impl.v_scale_cache[0, 0, 0, 0] = 2.5
    off = kv[0].numel() + impl.v_quant_cache.numel() * 4
    assert raw[off:off + 4].tolist() == [0, 0, 0x20, 0x40]


def test_host_edits_reverse_exactly_and_refuse_twice(tmp_path):
    vllm_root, ascend_root = _trees(tmp_path)
    before = {p: p.read_text() for p in sorted(tmp_path.rglob("*.py"))}
    hi.apply_host_edits(vllm_root, ascend_root)
    with pytest.raises(hi.HostPatchError, match="already applied"):
        hi.apply_host_edits(vllm_root, ascend_root)
    hi.apply_host_edits(vllm_root, ascend_root, reverse=True)
    assert {p: p.read_text() for p in sorted(tmp_path.rglob("*.py"))} == before
    assert not list(tmp_path.rglob("*.orig"))
    # a file edited after the patch is not reverted over
    hi.apply_host_edits(vllm_root, ascend_root)
    target = vllm_root / "vllm/config/cache.py"
    target.write_text(target.read_text() + "\n# local change\n")
    with pytest.raises(hi.HostPatchError, match="changed since"):
        hi.apply_host_edits(vllm_root, ascend_root, reverse=True)


def test_host_edits_are_all_or_nothing(tmp_path):
    vllm_root, ascend_root = _trees(tmp_path)
    runner = ascend_root / "vllm_ascend/worker/model_runner_v1.py"
    runner.write_text(runner.read_text().replace('hasattr(current_kv_cache_spec, "head_size_v")',
                                                 "current_kv_cache_spec.v"))
    before = {p: p.read_text() for p in sorted(tmp_path.rglob("*.py"))}
    with pytest.raises(hi.HostPatchError, match="head_size_v override: construct matched 0"):
        hi.apply_host_edits(vllm_root, ascend_root)
    assert {p: p.read_text() for p in sorted(tmp_path.rglob("*.py"))} == before
    assert not list(tmp_path.rglob("*.orig"))


def test_host_edits_refuse_installed_packages(tmp_path):
    vllm_root, ascend_root = _trees(tmp_path / "lib" / "site-packages")
    with pytest.raises(hi.HostPatchError, match="installed package"):
        hi.apply_host_edits(vllm_root, ascend_root)


def test_command_line(tmp_path, capsys):
    vllm_root, ascend_root = _trees(tmp_path)
    args = ["--vllm", str(vllm_root), "--ascend", str(ascend_root)]
    assert hi.main(args + ["--check"]) == 0
    assert hi.main(args) == 0
    assert hi.main(args) == 1
    assert hi.main(args + ["--reverse"]) == 0
    assert "RESULT: host edits reverted" in capsys.readouterr().out
