# SPDX-License-Identifier: Apache-2.0
"""Adapter for the vllm-ascend-hust attention backend."""

from .register import BACKEND_CLASS_PATH_BY_DTYPE, AscendHustAdapter

__all__ = ["BACKEND_CLASS_PATH_BY_DTYPE", "AscendHustAdapter"]
