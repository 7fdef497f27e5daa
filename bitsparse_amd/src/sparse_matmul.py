"""GEMMs with one operand held as a BitsparseTensor.

Mirrors reference lib_sparse/src/sparse_matmul.py: ``AspB`` (:9-47),
``spAB`` (:50-88), ``AspRelu2B`` (:91-132), same signatures and row_batch
semantics.  For bf16 storage, ``AspB`` / ``AspRelu2B`` with ``row_batch=0``
run the reconstruct-into-LDS MFMA GEMM (the compressed operand is decoded
tile by tile into LDS and never written to HBM); the other cases decompress
to a dense HBM buffer and call the library GEMM, as the reference does.
"""
from __future__ import annotations

import torch
from torch import Tensor

from ..fp8 import matmul
from .hip_operators import unpack_batch_, unpack_relu2_batch_
from ..bitsparse import BitsparseTensor
from . import dw_gemm

# route bf16 AspB / AspRelu2B through the LDS-reconstruct GEMM
USE_LDS_GEMM = True


def AspB(A: Tensor, B_sparse: BitsparseTensor, A_scale: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] @ B[N, K] with B compressed -> out[M, K].

    row_batch > 0 decompresses tile-aligned row batches of B and accumulates
    (lower peak memory).  Reference: sparse_matmul.py:9-47.
    """
    BLOCK_M, BLOCK_N = B_sparse.BLOCK_M, B_sparse.BLOCK_N
    grid_m, grid_n = B_sparse.grid_m, B_sparse.grid_n
    N, K = B_sparse.shape
    M = A.shape[0]

    if row_batch <= 0:
        if USE_LDS_GEMM and dw_gemm.supports(A, B_sparse, square=False):
            return dw_gemm.gemm_compressed_b(A, B_sparse, square=False)
        num_tiles = grid_m * grid_n
        dense = torch.empty(N, K, device=A.device, dtype=B_sparse.dtype)
        unpack_batch_(B_sparse, dense, 0, grid_n, K, N, num_tiles)
        return matmul(A, dense, B_sparse.fp8, A_scale, B_sparse.scale)

    out = torch.zeros(M, K, device=A.device, dtype=A.dtype)
    row_tiles_per_batch = max(1, row_batch // BLOCK_M)
    for first_n_tile in range(0, grid_m, row_tiles_per_batch):
        n_start = first_n_tile * BLOCK_M
        n_end = min(n_start + row_tiles_per_batch * BLOCK_M, N)
        batch_rows = n_end - n_start
        num_row_tiles = (batch_rows + BLOCK_M - 1) // BLOCK_M
        num_tiles_in_batch = num_row_tiles * grid_n
        dense_batch = torch.empty(batch_rows, K, device=A.device, dtype=B_sparse.dtype)
        unpack_batch_(B_sparse, dense_batch, first_n_tile, grid_n, K, batch_rows, num_tiles_in_batch)
        out.addmm_(A[:, n_start:n_end], dense_batch)
    return out


def spAB(A_sparse: BitsparseTensor, B: Tensor, out: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] (compressed) @ B[N, K] -> out[M, K].  Reference: sparse_matmul.py:50-88."""
    BLOCK_M, BLOCK_N = A_sparse.BLOCK_M, A_sparse.BLOCK_N
    grid_m, grid_n = A_sparse.grid_m, A_sparse.grid_n
    M, N = A_sparse.shape
    K = B.shape[1]

    if row_batch <= 0:
        num_tiles = grid_m * grid_n
        dense = torch.empty(M, N, device=B.device, dtype=A_sparse.dtype)
        unpack_batch_(A_sparse, dense, 0, grid_n, N, M, num_tiles)
        return matmul(dense, B, A_sparse.fp8, A_sparse.scale)

    out = torch.zeros(M, K, device=B.device, dtype=B.dtype) if out is None else out
    row_tiles_per_batch = max(1, row_batch // BLOCK_M)
    for first_m_tile in range(0, grid_m, row_tiles_per_batch):
        m_start = first_m_tile * BLOCK_M
        m_end = min(m_start + row_tiles_per_batch * BLOCK_M, M)
        batch_rows = m_end - m_start
        num_row_tiles = (batch_rows + BLOCK_M - 1) // BLOCK_M
        num_tiles_in_batch = num_row_tiles * grid_n
        dense_batch = torch.empty(batch_rows, N, device=B.device, dtype=A_sparse.dtype)
        unpack_batch_(A_sparse, dense_batch, first_m_tile, grid_n, N, batch_rows, num_tiles_in_batch)
        torch.mm(dense_batch, B, out=out[m_start:m_end])
    return out


def AspRelu2B(A: Tensor, B_sparse: BitsparseTensor, A_scale: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] @ (k * B^2) with B = relu(preact) compressed -> out[M, K].

    The square is formed in bf16 (fp8 storage: widened, squared, times
    scale^2), then the GEMM runs in bf16 or fp8 (re-quantized), as the
    reference does.  Reference: sparse_matmul.py:91-132.
    """
    BLOCK_M, BLOCK_N = B_sparse.BLOCK_M, B_sparse.BLOCK_N
    grid_m, grid_n = B_sparse.grid_m, B_sparse.grid_n
    N, K = B_sparse.shape
    M = A.shape[0]

    if row_batch <= 0:
        if USE_LDS_GEMM and dw_gemm.supports(A, B_sparse, square=True):
            return dw_gemm.gemm_compressed_b(A, B_sparse, square=True)
        num_tiles = grid_m * grid_n
        dense = torch.empty(N, K, device=A.device, dtype=torch.bfloat16)
        unpack_relu2_batch_(B_sparse, dense, 0, grid_n, K, N, num_tiles)
        return matmul(A, dense, B_sparse.fp8, A_scale)

    out = torch.zeros(M, K, device=A.device, dtype=A.dtype)
    row_tiles_per_batch = max(1, row_batch // BLOCK_M)
    for first_n_tile in range(0, grid_m, row_tiles_per_batch):
        n_start = first_n_tile * BLOCK_M
        n_end = min(n_start + row_tiles_per_batch * BLOCK_M, N)
        batch_rows = n_end - n_start
        num_row_tiles = (batch_rows + BLOCK_M - 1) // BLOCK_M
        num_tiles_in_batch = num_row_tiles * grid_n
        dense_batch = torch.empty(batch_rows, K, device=A.device, dtype=torch.bfloat16)
        unpack_relu2_batch_(B_sparse, dense_batch, first_n_tile, grid_n, K, batch_rows,
                            num_tiles_in_batch)
        out.addmm_(A[:, n_start:n_end], dense_batch)
    return out
