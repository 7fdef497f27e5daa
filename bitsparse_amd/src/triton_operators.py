"""Alias of ``hip_operators`` under the reference's module name.

Callers written against reference lib_sparse/src/triton_operators.py
(``unpack_batch_``, ``tile_pack``, ``compact_vals``, ...) keep working; the
kernels behind these names are the HIP ones, there is no Triton.
"""
from .hip_operators import (  # noqa: F401
    compact_vals,
    mask_with_bitmask_,
    relu2_grad_sparse_,
    tile_pack,
    unpack_batch_,
    unpack_relu2_batch_,
)
