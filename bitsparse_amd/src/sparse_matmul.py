"""GEMMs with one operand held as a BitsparseTensor.

Public surface of reference lib_sparse/src/sparse_matmul.py: ``AspB``
(:9-47), ``spAB`` (:50-88) and ``AspRelu2B`` (:91-132), same signatures.

Design.  The compressed operand is consumed where it lies:

* B compressed (the MLP backward's dW = dY^T h): the reconstruct-into-LDS
  MFMA GEMM (``dw_gemm``) decodes each 64x64 tile of B into LDS inside the
  GEMM, so no dense B exists in HBM at any point.  bf16 storage multiplies
  in bf16; fp8 storage in fp8, as the reference does (A quantized by
  ``to_fp8`` when it comes in bf16; for AspRelu2B the kernel forms the
  ``to_fp8`` re-quantization of the bf16 k*v^2 from the stored codes).
  ``row_batch``, which in the reference bounds the size of the dense B it
  decompresses, has nothing to bound for bf16 and the product is computed in
  one launch (one fp32 accumulation over all of K instead of one bf16
  rounding per batch).  Packed (pack_sbit) storage goes the same way: a
  pre-pass of each GEMM call unpacks the tensor's value run (15-bit fields
  to bf16; 7-bit codes in the pass that maps fp8 codes), never a dense B.
* Every other case (fp8 row batches -- whose per-batch
  re-quantization is part of their result --, a compressed left operand)
  decodes B to dense -- whole, or ``row_batch`` rows at a time through a
  tile-row view of the compressed tensor (``tile_rows``: bitmask and prefix
  slices over the same values, no copy) -- and multiplies with the library
  GEMM (``fp8.matmul``).
"""
from __future__ import annotations

import torch
from torch import Tensor

from ..bitsparse import BitsparseTensor
from ..config import BLOCK_M
from ..fp8 import Fp8Operand, as_fp8_operand, fp8_gemm, matmul
from . import dw_gemm
from .hip_operators import unpack_batch_, unpack_relu2_batch_

# route AspB / AspRelu2B through the reconstruct-into-LDS GEMM when it applies
USE_LDS_GEMM = True


def tile_rows(sp: BitsparseTensor, first: int, stop: int) -> BitsparseTensor:
    """Tile rows [first, stop) of ``sp`` as a BitsparseTensor over the same
    storage.  Its bitmask and prefix are slices; prefix values stay relative
    to ``vals_offset``, which is how every kernel reads them."""
    gn, tile_bytes = sp.grid_n, sp.BLOCK_M * sp.BLOCK_N // 8
    rows = min(stop * sp.BLOCK_M, sp.shape[0]) - first * sp.BLOCK_M
    return BitsparseTensor(sp.vals, sp.bitmask[first * gn * tile_bytes:stop * gn * tile_bytes],
                           sp.prefix[first * gn:stop * gn + 1], (rows, sp.shape[1]), sp.dtype,
                           stop - first, gn, sp.BLOCK_M, sp.BLOCK_N, scale=sp.scale,
                           vals_offset=sp.vals_offset, pack_sbit=sp.pack_sbit)


def decoded(sp: BitsparseTensor, square: bool) -> Tensor:
    """Dense copy of ``sp``: its stored dtype, or bf16 k*v^2 (times scale^2
    for fp8 storage) when ``square``."""
    rows, cols = sp.shape
    out = torch.empty((rows, cols), device=sp.bitmask.device,
                      dtype=torch.bfloat16 if square else sp.dtype)
    unpack = unpack_relu2_batch_ if square else unpack_batch_
    return unpack(sp, out, 0, sp.grid_n, cols, rows, sp.grid_m * sp.grid_n)


def _row_blocks(sp: BitsparseTensor, row_batch: int):
    """(first row, last row + 1, view) of tile-aligned blocks of at most
    ``row_batch`` rows (at least one tile row)."""
    step = max(1, row_batch // BLOCK_M)
    for first in range(0, sp.grid_m, step):
        view = tile_rows(sp, first, min(first + step, sp.grid_m))
        r0 = first * BLOCK_M
        yield r0, r0 + view.shape[0], view


def _times_compressed(A: Tensor, B_sparse: BitsparseTensor, A_scale: Tensor | None, row_batch: int,
                      square: bool) -> Tensor:
    """A @ op(B) with op = identity or k * (.)^2, B compressed [K, N]."""
    # fp8 values are multiplied in fp8: with their stored scale, or (square)
    # re-quantized from the bf16 square, as the reference does
    fp8 = B_sparse.fp8
    b_scale = None if square else B_sparse.scale
    if fp8 and row_batch <= 0:
        opa = as_fp8_operand(A, A_scale)           # quantized once, whichever GEMM runs
        if USE_LDS_GEMM and dw_gemm.supports_fp8(opa.codes, B_sparse):
            return dw_gemm.gemm_compressed_b_fp8(opa.codes, opa.scale, B_sparse, square)
        return fp8_gemm(opa, as_fp8_operand(decoded(B_sparse, square), b_scale), torch.bfloat16)
    if USE_LDS_GEMM and not fp8 and dw_gemm.supports(A, B_sparse, square=square):
        return dw_gemm.gemm_compressed_b(A, B_sparse, square=square)
    if row_batch <= 0:
        return matmul(A, decoded(B_sparse, square), False)
    M, N = A.shape[0], B_sparse.shape[1]
    if not fp8:
        out = torch.zeros((M, N), device=A.device, dtype=A.dtype)
        for r0, r1, view in _row_blocks(B_sparse, row_batch):
            out.addmm_(A[:, r0:r1], decoded(view, square))
        return out
    # fp8 blocks: each block's fp8 product in fp32, summed, rounded once
    opa = as_fp8_operand(A, A_scale)
    acc = torch.zeros((M, N), device=A.device, dtype=torch.float32)
    for r0, r1, view in _row_blocks(B_sparse, row_batch):
        opb = as_fp8_operand(decoded(view, square), b_scale)
        acc += fp8_gemm(Fp8Operand(opa.codes[:, r0:r1], opa.scale), opb, torch.float32)
    return acc.to(torch.bfloat16)


def AspB(A: Tensor, B_sparse: BitsparseTensor, A_scale: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] @ B[N, K] with B compressed -> out[M, K] (reference
    sparse_matmul.py:9-47).  ``A_scale``: A is fp8 with that scale."""
    return _times_compressed(A, B_sparse, A_scale, row_batch, square=False)


def AspRelu2B(A: Tensor, B_sparse: BitsparseTensor, A_scale: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] @ (k * B^2) with B = relu(preact) compressed -> out[M, K]
    (reference sparse_matmul.py:91-132).  The square is formed in bf16 (fp8
    storage: widened, squared, times scale^2); with fp8 storage the product
    runs in fp8 on the re-quantized square."""
    return _times_compressed(A, B_sparse, A_scale, row_batch, square=True)


def spAB(A_sparse: BitsparseTensor, B: Tensor, out: Tensor | None = None, row_batch: int = 0) -> Tensor:
    """A[M, N] (compressed) @ B[N, K] -> [M, K] (reference
    sparse_matmul.py:50-88).  ``row_batch > 0`` decodes A in tile-row blocks
    and writes each block's rows of ``out`` (allocated when None); with
    ``row_batch <= 0`` the whole product is returned and ``out`` is not
    used, as in the reference."""
    fp8 = A_sparse.fp8
    if row_batch <= 0:
        return matmul(decoded(A_sparse, False), B, fp8, a_scale=A_sparse.scale)
    M, K = A_sparse.shape[0], B.shape[1]
    if out is None:
        out = torch.zeros((M, K), device=B.device, dtype=B.dtype)
    for r0, r1, view in _row_blocks(A_sparse, row_batch):
        block = decoded(view, False)
        if fp8:
            out[r0:r1] = matmul(block, B, True, a_scale=A_sparse.scale)
        else:
            torch.mm(block, B, out=out[r0:r1])
    return out
