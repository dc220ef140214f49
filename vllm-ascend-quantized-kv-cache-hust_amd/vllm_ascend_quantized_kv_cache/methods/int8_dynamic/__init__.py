# SPDX-License-Identifier: Apache-2.0
"""Dynamic per-channel INT8 KV cache (scales from the first K/V a layer sees).

Registers metadata only (``src/vllm_ascend_quantized_kv_cache/methods/int8_dynamic/__init__.py:17-74``).
"""

from __future__ import annotations

from ...core.hosts import VLLM_ASCEND_HUST
from ...dtypes import KVQuantMode
from ..base import MethodConfig, MethodSpec
from ..registry import register_method

PROVENANCE = "ascend-pr-116/0001 (MI355X HIP rebuild)"


def _validate_config(config: MethodConfig) -> None:
    if config.head_size % 8:
        raise ValueError(
            "int8_dynamic expects head_size divisible by 8 for the fused "
            f"attention path, got {config.head_size}"
        )


def _load_semantics(config):
    from .semantics import Int8DynamicSemantics

    return Int8DynamicSemantics(config)


def _ascend_adapter(method):
    from ...adapters.vllm_ascend_hust import AscendHustAdapter

    return AscendHustAdapter(method)


METHOD_SPEC = register_method(
    MethodSpec(
        name="int8_dynamic",
        dtype="int8",
        summary=(
            "Dynamic per-channel INT8 KV cache: token-axis amax of the first K/V "
            "sets symmetric scales; decode dequantizes in registers inside a "
            "fused HIP attention kernel."
        ),
        provenance=PROVENANCE,
        quant_mode=KVQuantMode.INT8_PER_TENSOR,
        supports=(VLLM_ASCEND_HUST,),
        config_validator=_validate_config,
        semantics_loader=_load_semantics,
        adapter_factories={VLLM_ASCEND_HUST: _ascend_adapter},
    )
)

__all__ = ["METHOD_SPEC"]
