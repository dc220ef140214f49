# SPDX-License-Identifier: Apache-2.0
"""KIVI INT4 KV cache: int4 paged history plus a full-precision residual window.

Registers metadata only; torch and the HIP library load lazily
(``src/vllm_ascend_quantized_kv_cache/methods/kivi_int4/__init__.py:18-74``).
"""

from __future__ import annotations

from ...core.hosts import VLLM_ASCEND_HUST
from ...dtypes import KVQuantMode
from ..base import MethodConfig, MethodSpec
from ..registry import register_method

PROVENANCE = "ascend-pr-116/0003-0009 (MI355X HIP rebuild)"


def _validate_config(config: MethodConfig) -> None:
    from .geometry import validate_kivi_config

    validate_kivi_config(config)


def _load_semantics(config):
    from .semantics import KiviInt4Semantics

    return KiviInt4Semantics(config)


def _ascend_adapter(method):
    from ...adapters.vllm_ascend_hust import AscendHustAdapter

    return AscendHustAdapter(method)


METHOD_SPEC = register_method(
    MethodSpec(
        name="kivi_int4",
        dtype="kivi_int4",
        summary=(
            "KIVI INT4: the newest residual_length tokens of each request stay "
            "full precision; older tokens are packed into a paged int4 history "
            "by HIP kernels (keys grouped along tokens, values along head_dim) "
            "and read back by a fused dequant-attention kernel."
        ),
        provenance=PROVENANCE,
        quant_mode=KVQuantMode.KIVI_INT4,
        supports=(VLLM_ASCEND_HUST,),
        config_validator=_validate_config,
        semantics_loader=_load_semantics,
        adapter_factories={VLLM_ASCEND_HUST: _ascend_adapter},
    )
)

__all__ = ["METHOD_SPEC"]
