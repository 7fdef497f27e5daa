"""Host side of the reconstruct-into-LDS MFMA GEMM (``bs_gemm_compressed_b``).

``gemm_compressed_b(A, B_sparse, square)`` computes ``A @ B`` (or
``A @ (k * B^2)``) with B a BitsparseTensor decoded tile by tile into LDS by
the kernel; it replaces the decompress-to-HBM + GEMM of reference
lib_sparse/src/sparse_matmul.py:24-28 / :109-113.  Packed (pack_sbit) values
go to the ``*_packed`` entry points, which unpack the tensor's value run (not
a dense B) in a pre-pass that the GEMM then stages from (reference
bitpacking.py:37-55 ahead of the same GEMMs).
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from .._lib import check, ptr, stream_handle
from ..config import RELU2_SCALE


def _stored(B_sparse) -> torch.dtype:
    """The stored value type (a packed stream's logical dtype)."""
    return B_sparse.dtype if B_sparse.pack_sbit else B_sparse.vals.dtype


def _vals_aligned(B_sparse) -> bool:
    # raw runs are read as aligned 16-byte slots, packed streams as dwords
    return B_sparse.vals.data_ptr() % (4 if B_sparse.pack_sbit else 16) == 0


def supports(A: Tensor, B_sparse, square: bool) -> bool:
    """Shapes / dtypes the kernel handles: bf16 A on the GPU; B stored as
    bf16 (raw or packed), or raw fp8 when the operand is the ReLU^2 square."""
    if not A.is_cuda or A.dim() != 2 or A.dtype != torch.bfloat16:
        return False
    if A.shape[1] != B_sparse.shape[0] or not _vals_aligned(B_sparse):
        return False
    vdt = _stored(B_sparse)
    if B_sparse.pack_sbit:
        return vdt == torch.bfloat16
    if vdt == torch.bfloat16:
        return True
    return square and vdt in (torch.float8_e4m3fn, torch.float8_e5m2)


def supports_fp8(A: Tensor, B_sparse) -> bool:
    """The fp8-operand kernel: e4m3fn A on the GPU (2-D, any strides) and B
    stored as e4m3fn / e5m2 values, raw or packed."""
    if not A.is_cuda or A.dim() != 2 or A.dtype != torch.float8_e4m3fn:
        return False
    if A.shape[1] != B_sparse.shape[0] or not _vals_aligned(B_sparse):
        return False
    return _stored(B_sparse) in (torch.float8_e4m3fn, torch.float8_e5m2)


def gemm_compressed_b_fp8(A: Tensor, A_scale: Tensor, B_sparse, square: bool,
                          b_scale_out: Tensor | None = None) -> Tensor:
    """bf16(A_scale * sB * (A @ Bq)) with A in e4m3fn and B compressed fp8:
    square=False multiplies the stored codes with their scale (AspB);
    square=True the to_fp8 re-quantization of the bf16 k*v^2 (times
    bf16(scale^2)) that AspRelu2B unpacks, formed from the codes in the
    kernel.  ``b_scale_out`` (fp32 0-d) receives sB."""
    from .hip_operators import dtype_code
    if not supports_fp8(A, B_sparse):
        raise ValueError("gemm_compressed_b_fp8: unsupported operand combination")
    if A_scale is None or not A_scale.is_cuda or A_scale.dtype != torch.float32:
        raise TypeError("gemm_compressed_b_fp8: A_scale must be an fp32 GPU tensor")
    K, N = B_sparse.shape
    M = A.shape[0]
    if A.stride(1) == 1 and A.stride(0) >= max(K, 1):
        a_layout, a_src, lda = 1, A, A.stride(0)
    elif A.stride(0) == 1 and A.stride(1) >= max(M, 1):
        a_layout, a_src, lda = 0, A.t(), A.stride(1)      # At [K, M] is m-contiguous
    else:
        a_layout, a_src, lda = 1, A.contiguous(), K
    stored_scale = B_sparse.scale
    if not square and stored_scale is None:
        raise ValueError("gemm_compressed_b_fp8: fp8 values without their scale")
    L = _lib.load()
    C = torch.empty((M, N), device=A.device, dtype=torch.bfloat16)
    packed = B_sparse.pack_sbit
    # a packed stream is unpacked into the room square=1 maps its codes into
    need = L.bs_gemm_compressed_b_fp8_workspace_bytes(M, N, K, a_layout, int(square or packed))
    ws = torch.empty(need, device=A.device, dtype=torch.uint8)
    fn = L.bs_gemm_compressed_b_fp8_packed if packed else L.bs_gemm_compressed_b_fp8
    check(fn(
        a_src.data_ptr(), A_scale.data_ptr(), M, K, lda, a_layout, B_sparse.vals.data_ptr(),
        dtype_code(_stored(B_sparse)), B_sparse.vals.numel(), B_sparse.bitmask.data_ptr(),
        B_sparse.prefix.data_ptr(), B_sparse.vals_offset.data_ptr(), N, int(square), float(RELU2_SCALE),
        ptr(stored_scale), C.data_ptr(), ptr(b_scale_out), ws.data_ptr(), need, stream_handle(A.device)),
        "bs_gemm_compressed_b_fp8")
    return C


def gemm_compressed_b(A: Tensor, B_sparse, square: bool) -> Tensor:
    from .hip_operators import dtype_code
    if not supports(A, B_sparse, square):
        raise ValueError("gemm_compressed_b: unsupported operand combination")
    K, N = B_sparse.shape
    M = A.shape[0]
    if A.stride(1) == 1 and A.stride(0) % 8 == 0 and A.data_ptr() % 16 == 0 and K % 8 == 0:
        a_layout, a_src, lda = 1, A, A.stride(0)          # k contiguous: read in place
    else:
        # the kernel transposes A^T [K, M] (m contiguous; for A = dY.T this
        # is dY itself) into its workspace; rows padded to a multiple of 8
        At = A.t()
        if At.stride(1) != 1 or At.stride(0) % 8 != 0 or At.data_ptr() % 16 != 0:
            ld = (M + 7) // 8 * 8
            pad = torch.zeros((K, ld), device=A.device, dtype=A.dtype)
            pad[:, :M] = At
            At = pad
        a_layout, a_src, lda = 0, At, At.stride(0)
    L = _lib.load()
    C = torch.empty((M, N), device=A.device, dtype=torch.bfloat16)
    wsfn = (L.bs_gemm_compressed_b_packed_workspace_bytes if B_sparse.pack_sbit
            else L.bs_gemm_compressed_b_workspace_bytes)
    need = wsfn(M, N, K, a_layout)
    ws = torch.empty(max(need, 0), device=A.device, dtype=torch.uint8) if need > 0 else None
    scale = B_sparse.scale if (square and B_sparse.scale is not None) else None
    fn = L.bs_gemm_compressed_b_packed if B_sparse.pack_sbit else L.bs_gemm_compressed_b
    check(fn(
        a_src.data_ptr(), M, K, lda, a_layout, B_sparse.vals.data_ptr(), dtype_code(_stored(B_sparse)),
        B_sparse.vals.numel(), B_sparse.bitmask.data_ptr(), B_sparse.prefix.data_ptr(),
        B_sparse.vals_offset.data_ptr(), N, int(square), float(RELU2_SCALE), ptr(scale),
        C.data_ptr(), ptr(ws), need, stream_handle(A.device)), "bs_gemm_compressed_b")
    return C
