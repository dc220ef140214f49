# SPDX-License-Identifier: Apache-2.0
"""Test configuration: import paths and the ``gpu`` marker.

``-m "not gpu"`` runs everywhere (oracle, host logic, ABI loading);
``-m gpu`` needs an MI355X and the in-tree ``libkvq_hip.so``.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_ROOT = ROOT / "vllm-ascend-quantized-kv-cache-hust_amd"
for p in (str(PKG_ROOT), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libkvq_hip.so")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")
