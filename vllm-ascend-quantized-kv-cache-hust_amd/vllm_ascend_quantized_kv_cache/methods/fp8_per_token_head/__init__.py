# SPDX-License-Identifier: Apache-2.0
"""fp8_per_token_head KV cache: E4M3 codes plus a dynamic fp32 scale per (token, head).

Registers metadata only; torch and the HIP library load lazily
(``src/vllm_ascend_quantized_kv_cache/methods/fp8_per_token_head/__init__.py:1-84``).
The store (``ops.fp8_ops.fp8_per_token_head_store``) and the read path
(``fp8_per_token_head_dequant_gather`` / ``fp8_per_token_head_attention``)
run as HIP kernels.  As in the reference, no host adapter is wired: the host
cannot select the literal through this plugin yet, and ``host_adapter``
fails closed with "no adapter wired".
"""

from __future__ import annotations

from ...core.hosts import VLLM_ASCEND_HUST
from ...dtypes import KVQuantMode
from ..base import MethodConfig, MethodSpec
from ..registry import register_method

PROVENANCE = "host-triton-per-token-head-contract (MI355X HIP rebuild)"


def _validate_config(config: MethodConfig) -> None:
    if config.head_size <= 0 or config.head_size % 4:
        raise ValueError(
            "fp8_per_token_head requires head_size positive and divisible "
            f"by 4 (fp32 scale alignment), got {config.head_size}"
        )


def _load_semantics(config):
    from .semantics import Fp8PerTokenHeadSemantics

    return Fp8PerTokenHeadSemantics(config)


METHOD_SPEC = register_method(
    MethodSpec(
        name="fp8_per_token_head",
        dtype="fp8_per_token_head",
        summary=(
            "Per-token-head dynamic-scale E4M3 storage: each (token, head) keeps "
            "head_size E4M3 bytes plus one fp32 scale computed online at write "
            "time.  A HIP store kernel writes the paged codes and a HIP gather "
            "reads them back into dense rows for the MFMA attention kernel; no "
            "host adapter is wired, so the literal is not selectable yet."
        ),
        provenance=PROVENANCE,
        quant_mode=KVQuantMode.FP8_PER_TOKEN_HEAD,
        supports=(VLLM_ASCEND_HUST,),
        config_validator=_validate_config,
        semantics_loader=_load_semantics,
    )
)

__all__ = ["METHOD_SPEC"]
