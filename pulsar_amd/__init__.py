"""MI355X-native W4A16 linear-layer path for Pulsar.

Importing the package loads the in-tree native libraries:
  libpulsar_w4a16.so      gfx950 HIP kernels behind the C ABI (include/pulsar_w4a16.h)
  _pulsar_w4a16_torch.so  the reference's at::Tensor operator API and the
                          torch.ops.pulsar.* registrations (gemm_w4a16,
                          gemm_w4a16_split, repack_w4a16, gemm_w4a16_marlin, ...)

There is no fallback: if the libraries are missing the import fails (build
them with `python -m pulsar_amd.build`).  Mirrors the reference loader
pulsar/src/pulsar/core/__init__.py:17-35.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpulsar_w4a16.so")
TORCH_LIB_PATH = os.path.join(_HERE, "_pulsar_w4a16_torch.so")

_loaded = False
_capi = None


def load() -> None:
    global _loaded
    if _loaded:
        return
    for p in (LIB_PATH, TORCH_LIB_PATH):
        if not os.path.isfile(p):
            raise RuntimeError(
                f"native library {os.path.basename(p)} not found in {_HERE}; build it with "
                "`python -m pulsar_amd.build`"
            )
    torch.ops.load_library(TORCH_LIB_PATH)
    _loaded = True


def capi() -> ctypes.CDLL:
    """ctypes handle on the C ABI library (for ABI-level tests and non-torch callers)."""
    global _capi
    if _capi is None:
        if not os.path.isfile(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built; run `python -m pulsar_amd.build`")
        _capi = ctypes.CDLL(LIB_PATH)
    return _capi


load()

from . import ops  # noqa: E402  (registers the fake kernels)

__all__ = ["ops", "load", "capi", "LIB_PATH", "TORCH_LIB_PATH"]
