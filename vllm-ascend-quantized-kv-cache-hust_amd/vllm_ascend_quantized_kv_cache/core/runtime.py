# SPDX-License-Identifier: Apache-2.0
"""Device-capability guards for the kernel layer (safe to import anywhere).

The reference guards its NPU paths the same way
(``src/vllm_ascend_quantized_kv_cache/core/runtime.py:36-62``); here the device
is a ROCm GPU driven through the in-tree HIP library, and every guard raises a
``RuntimeError`` naming the caller instead of silently falling back.
"""

from __future__ import annotations

import importlib
import importlib.util


def module_available(name: str) -> bool:
    try:
        return importlib.util.find_spec(name) is not None
    except (ImportError, ValueError):
        return False


def import_torch(what: str = "this code path"):
    try:
        return importlib.import_module("torch")
    except ImportError as exc:
        raise RuntimeError(f"{what} requires torch, which is not installed") from exc


def gpu_available() -> bool:
    """True when torch sees a ROCm device."""
    try:
        torch = importlib.import_module("torch")
    except ImportError:
        return False
    try:
        return bool(torch.version.hip) and torch.cuda.is_available()
    except Exception:
        return False


def stream_capturing() -> bool:
    """True while the caller's current HIP stream is recording a graph.

    Checked at the entry of each mixin's ``forward``: a step that stages a
    one-step plan from host memory must not be recorded into a graph that
    later replays it with other sequence lengths and slots.
    """
    try:
        torch = importlib.import_module("torch")
    except ImportError:
        return False
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def require_gpu(what: str) -> None:
    if not gpu_available():
        raise RuntimeError(
            f"{what} requires a ROCm GPU (MI355X / gfx950), but none is visible. "
            "The quantized-KV kernel layer runs on the GPU only; the pure "
            "semantics API works on any machine."
        )


__all__ = ["gpu_available", "import_torch", "module_available", "require_gpu",
           "stream_capturing"]
