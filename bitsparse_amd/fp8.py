"""FP8 storage and GEMM helpers.

Mirrors reference lib_sparse/fp8.py: ``is_fp8`` (:20-22), ``_scaled_mm``
(:25-49), ``MatmulFp8`` (:52-115), ``matmul`` (:118-120) and ``to_fp8``
(:123-129).  ``to_fp8`` runs two HIP kernels (amax, quantize) instead of an
Inductor graph; its rule is fixed as

    scale = max(fp32(amax|x|) / 448, 1e-9),  q = e4m3fn_RNE(fp32(x) / scale)

(one correctly rounded fp32 division, no saturation).  The fp8 GEMMs go to
hipBLASLt through torch's ``scaled_mm`` with per-tensor scales.
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function
from torch.nn import functional as F

from .config import CACHE_FP8_MATMUl

_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
_FP8_DTYPE = torch.float8_e4m3fn
_FP8_MAX = torch.finfo(_FP8_DTYPE).max


def is_fp8(dtype) -> bool:
    """True for the supported 8-bit float storage dtypes (e4m3fn, e5m2)."""
    return dtype in _FP8_DTYPES


def _scaled_mm(a: Tensor, b: Tensor, a_scale: Tensor, b_scale: Tensor, output_dtype: torch.dtype) -> Tensor:
    """Per-tensor-scaled fp8 GEMM.  hipBLASLt takes A row-major and B
    column-major, so B is re-laid out when it is not (reference fp8.py:25-49
    does the same for Ada)."""
    if a.stride(1) != 1:
        a = a.contiguous()
    if b.stride(0) != 1:
        b = b.T.contiguous().T
    return F.scaled_mm(
        mat_a=a, mat_b=b,
        scale_a=a_scale, scale_b=b_scale, output_dtype=output_dtype,
        scale_recipe_a=F.ScalingType.TensorWise, scale_recipe_b=F.ScalingType.TensorWise,
    )


class MatmulFp8(Function):
    """a @ b with fp8 operands (bf16 inputs are quantized with to_fp8).
    Reference: lib_sparse/fp8.py:52-115."""

    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor, a_scale: Tensor | None = None, b_scale: Tensor | None = None) -> Tensor:
        if not CACHE_FP8_MATMUl:
            ctx.save_for_backward(a, b)
            ctx.a_scale, ctx.b_scale = a_scale, b_scale

        if a.dtype == torch.bfloat16:
            assert a_scale is None
            a_fp8, a_scale = to_fp8(a)
        else:
            assert a_scale is not None
            a_fp8 = a
        if b.dtype == torch.bfloat16:
            assert b_scale is None
            b_fp8, b_scale = to_fp8(b)
        else:
            assert b_scale is not None
            b_fp8 = b

        if CACHE_FP8_MATMUl:
            ctx.save_for_backward(a_fp8, b_fp8, a_scale, b_scale)

        return _scaled_mm(a_fp8.contiguous(), b_fp8, a_scale, b_scale, output_dtype=torch.bfloat16)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        if CACHE_FP8_MATMUl:
            a_fp8, b_fp8, a_scale, b_scale = ctx.saved_tensors
        else:
            a, b = ctx.saved_tensors
            a_scale, b_scale = ctx.a_scale, ctx.b_scale
            if a.dtype == torch.bfloat16:
                assert a_scale is None
                a_fp8, a_scale = to_fp8(a)
            else:
                assert a_scale is not None
                a_fp8 = a
            if b.dtype == torch.bfloat16:
                assert b_scale is None
                b_fp8, b_scale = to_fp8(b)
            else:
                assert b_scale is not None
                b_fp8 = b

        grad_out_fp8, grad_out_scale = to_fp8(grad_output)
        grad_a, grad_b = None, None
        if ctx.needs_input_grad[0]:
            grad_a = _scaled_mm(grad_out_fp8, b_fp8.T, grad_out_scale, b_scale,
                                output_dtype=torch.bfloat16)
        if ctx.needs_input_grad[1]:
            grad_b = _scaled_mm(a_fp8.T.contiguous(), grad_out_fp8, a_scale, grad_out_scale,
                                output_dtype=torch.bfloat16)
        return grad_a, grad_b, None, None


def matmul(a: Tensor, b: Tensor, fp8: bool, a_scale: Tensor | None = None, b_scale: Tensor | None = None) -> Tensor:
    """a @ b; fp8 operands through MatmulFp8.  Reference: lib_sparse/fp8.py:118-120."""
    return MatmulFp8.apply(a, b, a_scale, b_scale) if fp8 else a @ b


@torch.no_grad()
def to_fp8(x: Tensor) -> tuple[Tensor, Tensor]:
    """(e4m3fn copy of x, fp32 0-d scale) — HIP amax + quantize kernels.
    Reference: lib_sparse/fp8.py:123-129."""
    from .src import hip_operators as ops
    ops.require_device(x, "to_fp8")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"to_fp8 expects a bfloat16 tensor, got {x.dtype}")
    x = x.detach()
    if x.dim() == 2 and not x.is_contiguous() and x.t().is_contiguous():
        # a transposed view (e.g. W.T): quantize the storage, keep the layout
        q, scale = to_fp8(x.t())
        return q.t(), scale
    x = x.contiguous()
    epoch = ops.amax_into_workspace(x)
    return ops.quantize_e4m3fn(x, epoch)
