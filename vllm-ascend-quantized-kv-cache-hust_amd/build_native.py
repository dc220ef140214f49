# SPDX-License-Identifier: Apache-2.0
"""Build ``libkvq_hip.so`` (the MI355X kernels) in-tree with hipcc.

Usage: ``python build_native.py`` (or ``build()`` from Python).  Each ``.hip``
file compiles to an object for gfx950 in parallel, then they link into
``vllm_ascend_quantized_kv_cache/_lib/libkvq_hip.so``.  hipcc cross-compiles,
so no GPU is needed.

Flags that matter for correctness:
  -ffp-contract=off  every fp32 op rounds once (bit-exact pack / dequant);
  packed-fp32 ops off  hipcc may not emit v_pk_{add,mul,fma}_f32;
HIP's default correctly rounded fp32 division is kept (no fast-math).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
OUT_DIR = HERE / "vllm_ascend_quantized_kv_cache" / "_lib"
LIB_NAME = "libkvq_hip.so"
ARCH = os.environ.get("KVQ_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-file additions.  The pack kernels' group min/max never sees a NaN that
# could change a result the reference defines (a NaN input has no defined
# KIVI code), and without NaN semantics the compiler drops the canonicalizing
# v_max_f32 it otherwise puts in front of every min/max.
# The fp8 store's amax and clamps likewise see only finite activations (a NaN
# has no E4M3 code the reference's clamp could produce).
EXTRA_FLAGS = {
    "kivi_pack.hip": ["-fno-honor-nans"],
    "fp8_kv.hip": ["-fno-honor-nans"],
}


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libkvq_hip.so")


#: host-only sources (planning code with no GPU part), built with the host compiler
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}"]


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        if src.suffix == ".cpp":
            cmd = [shutil.which("g++") or "g++", *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
        else:
            cmd = [hipcc, *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o",
                   str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"compile failed on {src.name}:\n{res.stdout}\n{res.stderr}")
        return obj

    workers = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(compile_one, sources))

    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    final = OUT_DIR / LIB_NAME
    os.replace(tmp, final)
    return final


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
