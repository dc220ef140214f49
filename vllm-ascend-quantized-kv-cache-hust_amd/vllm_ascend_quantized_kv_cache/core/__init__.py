# SPDX-License-Identifier: Apache-2.0
"""Cross-cutting layer: host list and detection, activation, device guards."""

from .activation import activate
from .hosts import ALL_HOSTS, VLLM_ASCEND_HUST, detect_host, require_host_stack
from .runtime import gpu_available, require_gpu

__all__ = [
    "ALL_HOSTS",
    "VLLM_ASCEND_HUST",
    "activate",
    "detect_host",
    "gpu_available",
    "require_gpu",
    "require_host_stack",
]
