# SPDX-License-Identifier: Apache-2.0
"""ctypes binding of ``libkvq_hip.so`` (the C ABI declared in ``include/kvq_hip.h``).

The library is built in-tree (``build_native.py``) and loaded from
``vllm_ascend_quantized_kv_cache/_lib``.  There is no fallback: if the library
is missing, or a tensor handed to a kernel is not on a ROCm device, the call
raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Any

_LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / "libkvq_hip.so"
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double

#: name -> (restype, argtypes); must match include/kvq_hip.h
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "kvq_abi_version": (_I, []),
    "kvq_kivi_pack_key": (
        _I,
        [_P, _I64, _P, _P, _I, _P, _I, _I64, _I, _I, _I, _I, _P, _P, _P, _P],
    ),
    "kvq_kivi_pack_value": (
        _I,
        [_P, _I64, _P, _P, _I, _P, _I, _I64, _I, _I, _I, _I, _P, _P, _P, _P],
    ),
    "kvq_kivi_ring_write": (_I, [_P, _I, _P, _P, _I64, _I, _P, _I, _P]),
    "kvq_kivi_store": (
        _I,
        [_P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _I64, _I64, _I64, _I64,
         _P, _P, _P, _P, _P, _P, _P],
    ),
    "kvq_kivi_gather_dequant": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _P, _I, _I64, _P, _I64,
         _P, _P, _P, _I, _I, _P, _P, _I, _P],
    ),
    "kvq_kivi_decode_workspace_bytes": (_I64, [_I64, _I, _I]),
    "kvq_kivi_decode_attn": (
        _I,
        [_P, _I, _I64, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _P, _I64,
         _P, _P, _I64, _P, _I64, _P, _P, _I, _I, _P, _P, _P],
    ),
    "kvq_kivi_decode_attn_noalloc": (
        _I,
        [_P, _I, _I64, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _P, _I64,
         _P, _P, _I64, _P, _I64, _P, _P, _I, _I, _P, _P],
    ),
    "kvq_plan_kivi_decode": (
        _I64, [_P, _I64, _I, _I, _I, _I64, _D, _P, _P, _I64, _P, _I64, _P]
    ),
    "kvq_kivi_step_check": (
        _I64,
        [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, _P, _P],
    ),
    "kvq_kivi_store_planned": (
        _I,
        [_P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _P, _I64, _I64, _I64,
         _P, _P, _P, _P, _P, _P, _P],
    ),
    "kvq_prefill_attn": (
        _I, [_P, _P, _P, _I, _P, _P, _I64, _I64, _I, _I, _I, _F, _I, _P, _P]
    ),
    "kvq_int8_calc_scales": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "kvq_int8_quant_scatter": (
        _I,
        [_P, _P, _I, _P, _P, _P, _I, _I64, _I64, _P, _P, _I64, _I, _P],
    ),
    "kvq_int8_dequant_gather": (
        _I,
        [_P, _P, _I64, _I, _I, _I, _P, _P, _I, _P, _I64, _P, _I64, _P, _P, _P],
    ),
    "kvq_selftest_mfma_f16": (_I, [_P, _P, _P, _P]),
    "kvq_selftest_lds_dma": (_I, [_P, _P, _P]),
    "kvq_selftest_lane_reductions": (_I, [_P, _P, _P]),
    "kvq_int8_decode_workspace_bytes": (_I64, [_I64, _I, _I]),
    "kvq_int8_decode_attn": (
        _I,
        [_P, _I, _I64, _I, _I, _I, _F, _P, _P, _I64, _I, _P, _P, _P, _I64, _P, _P, _I64,
         _P, _P, _P],
    ),
    "kvq_fp8_pth_store": (
        _I,
        [_P, _P, _I, _P, _I, _I64, _I, _I, _P, _P, _P, _P, _I64, _I, _P],
    ),
    "kvq_fp8_pth_gather": (
        _I,
        [_P, _P, _P, _P, _I64, _I, _I, _I, _P, _I, _I64, _P, _I64, _P, _P, _I, _P],
    ),
}

KVQ_ERR_INVALID = -1
KVQ_ERR_GEOMETRY = -2
KVQ_ERR_SCRATCH = -3
KVQ_ERR_CAPACITY = -4
KVQ_PLAN_DEFAULT, KVQ_PLAN_PIECES, KVQ_PLAN_SPLIT, KVQ_PLAN_SPLIT_PAIRED = 0, 1, 2, 3
#: static device scratch of kvq_kivi_decode_attn_noalloc (include/kvq_hip.h)
KVQ_DECODE_SCRATCH_BYTES = 32 << 20


def library_path() -> Path:
    return Path(os.environ.get("KVQ_HIP_LIBRARY", _LIB_PATH))


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"libkvq_hip.so is not built ({path}); run "
                    "`python vllm-ascend-quantized-kv-cache-hust_amd/build_native.py` "
                    "(hipcc, gfx950) before using the quantized-KV kernels"
                )
            handle = ctypes.CDLL(str(path))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _LIB = handle
    return _LIB


_DTYPE_CODES: dict = {}


def dtype_code(dtype) -> int:
    code = _DTYPE_CODES.get(dtype)
    if code is not None:
        return code
    import torch

    codes = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
    if dtype not in codes:
        raise RuntimeError(f"unsupported floating dtype for the HIP kernels: {dtype}")
    _DTYPE_CODES[dtype] = codes[dtype]
    return codes[dtype]


def index_code(dtype) -> int:
    import torch

    if dtype == torch.int32:
        return 0
    if dtype == torch.int64:
        return 1
    raise RuntimeError(f"index tensors must be int32/int64, got {dtype}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu_tensors(what: str, *tensors) -> None:
    """Every tensor must live on a ROCm GPU: the kernels have no CPU path."""
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{what} runs on the MI355X HIP kernels and needs GPU tensors; got a "
                f"tensor on {t.device}. There is no CPU fallback."
            )


def stream_of(t) -> int:
    import torch

    return torch.cuda.current_stream(t.device).cuda_stream


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    if rc == KVQ_ERR_INVALID:
        raise RuntimeError(f"{what}: the HIP kernel rejected its arguments (invalid).")
    if rc == KVQ_ERR_GEOMETRY:
        raise RuntimeError(f"{what}: geometry not supported by the HIP kernels.")
    if rc == KVQ_ERR_CAPACITY:
        raise RuntimeError(f"{what}: the plan does not fit the arrays it was given.")
    if rc == KVQ_ERR_SCRATCH:
        raise RuntimeError(
            f"{what}: the work list needs more than the {KVQ_DECODE_SCRATCH_BYTES >> 20} MiB "
            "static scratch; use the entry point that takes a workspace."
        )
    raise RuntimeError(f"{what}: HIP launch failed with hipError_t {rc}.")


__all__ = [
    "SIGNATURES",
    "check",
    "dtype_code",
    "index_code",
    "lib",
    "library_path",
    "ptr",
    "require_gpu_tensors",
    "stream_of",
]
