"""Host side of the reconstruct-into-LDS MFMA GEMM (C = A @ decode(B)).

Placeholder until the kernel lands: ``supports`` returns False so callers
take the decompress + library GEMM path.
"""
from __future__ import annotations

from torch import Tensor


def supports(A: Tensor, B_sparse, square: bool) -> bool:
    return False


def gemm_compressed_b(A: Tensor, B_sparse, square: bool) -> Tensor:
    raise NotImplementedError("reconstruct-into-LDS GEMM not built")
