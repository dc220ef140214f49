# SPDX-License-Identifier: Apache-2.0
"""Device layer: MI355X HIP kernels behind the plugin's op signatures.

- ``kivi_layout``: validators (pure torch metadata checks).
- ``kivi_pack`` / ``kivi_gather`` / ``kivi_decode`` / ``int8_ops``: the HIP
  kernels of ``libkvq_hip.so`` through ``_native`` (ctypes).  They accept GPU
  tensors only and raise otherwise.
"""

__all__: list[str] = []
