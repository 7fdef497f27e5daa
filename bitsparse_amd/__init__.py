"""bitsparse_amd — MI355X-native BitSparse activation compression.

Drop-in for the reference package ``lib_sparse`` (module layout and call
signatures mirrored: ``config``, ``bitsparse``, ``fp8``, ``layers``,
``src.functions``, ``src.sparse_matmul``, ``src.triton_operators``), backed by
hand-written HIP kernels for gfx950 in ``libbitsparse_hip.so`` (C ABI in
include/bitsparse_hip.h).  ``install_lib_sparse_alias()`` makes
``import lib_sparse...`` resolve to this package.
"""
from __future__ import annotations

import sys

__version__ = "0.1.0"

_SUBMODULES = ("config", "bitsparse", "fp8", "layers", "src", "src.functions",
               "src.sparse_matmul", "src.triton_operators", "src.hip_operators",
               "src.bitpacking")


def install_lib_sparse_alias() -> None:
    """Register this package under the reference's import name ``lib_sparse``."""
    import importlib
    pkg = sys.modules[__name__]
    sys.modules["lib_sparse"] = pkg
    for name in _SUBMODULES:
        mod = importlib.import_module(f"{__name__}.{name}")
        sys.modules[f"lib_sparse.{name}"] = mod
