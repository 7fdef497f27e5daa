"""FP8 value storage and the per-tensor-scaled fp8 GEMM of the BitSparse path.

Public surface of reference lib_sparse/fp8.py: ``is_fp8`` (:20-22),
``MatmulFp8`` (:52-115), ``matmul`` (:118-120) and ``to_fp8`` (:123-129);
``_scaled_mm`` (:25-49) is kept under its name for callers that used it.

Design.  An fp8 GEMM operand is a pair (codes, fp32 scale) -- ``Fp8Operand``.
A bf16 tensor becomes one through ``to_fp8`` (two HIP kernels: amax, then the
exact e4m3fn quantizer), an fp8 tensor is taken with the scale the caller
passes.  ``fp8_gemm`` multiplies two operands on hipBLASLt (torch's
``scaled_mm`` with tensor-wise scales; hipBLASLt wants A row-major and B
column-major, so an operand in the other layout is re-laid out).

``to_fp8`` follows one fixed rule (the reference's is whatever Inductor makes
of its graph):

    scale = max(fp32(amax|x|) / 448, 1e-9),  q = e4m3fn_RNE(fp32(x) / scale)

with one correctly rounded fp32 division and no saturation (|x/scale| past
464 gives NaN, as torch's own fp32 -> e4m3fn cast does).

Gradients of ``MatmulFp8`` come back in the fp8 dtype of the operand they
belong to, as in the reference (lib_sparse/fp8.py:107,112: ``output_dtype=
a_fp8.dtype`` / ``b_fp8.dtype``); autograd then widens them to the input's
bf16.  hipBLASLt rounds its fp32 result to e4m3fn with round-to-nearest-even
and saturation at +-448 (checked bit for bit against a saturating cast of its
own fp32 output on MI355X).  ``config.FP8_GRAD_DTYPE = torch.bfloat16`` asks
for bf16 gradients instead (more precise; not the reference's numbers).
"""
from __future__ import annotations

from typing import NamedTuple

import torch
from torch import Tensor
from torch.autograd import Function
from torch.nn import functional as F

from . import config

_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)


def is_fp8(dtype) -> bool:
    """True for the supported 8-bit float storage dtypes (e4m3fn, e5m2)."""
    return dtype in _FP8_DTYPES


class Fp8Operand(NamedTuple):
    """fp8 codes and the fp32 0-d scale they are multiplied by."""
    codes: Tensor
    scale: Tensor

    @property
    def T(self) -> "Fp8Operand":
        return Fp8Operand(self.codes.t(), self.scale)


def as_fp8_operand(x: Tensor, scale: Tensor | None) -> Fp8Operand:
    """A GEMM operand in fp8: a bf16 tensor is quantized with ``to_fp8`` and
    must come without a scale; an fp8 tensor must come with its scale
    (reference fp8.py:60-71 asserts the same pairing)."""
    if x.dtype == torch.bfloat16:
        if scale is not None:
            raise AssertionError("a bf16 operand is quantized here and takes no scale")
        return Fp8Operand(*to_fp8(x))
    if scale is None:
        raise AssertionError(f"an operand already in {x.dtype} needs its scale")
    return Fp8Operand(x, scale)


def fp8_gemm(a: Fp8Operand, b: Fp8Operand, out_dtype: torch.dtype) -> Tensor:
    """(a.codes * a.scale) @ (b.codes * b.scale) on hipBLASLt, fp32
    accumulation, rounded once to ``out_dtype`` (bf16, fp32 or an fp8 dtype,
    which saturates).  hipBLASLt's fp8 path takes A row-major and B
    column-major (both k-contiguous); an operand in the other layout is
    transposed by the HIP byte-transpose kernel (reference fp8.py:36-43)."""
    from .src import hip_operators as ops
    qa = ops.row_major_bytes(a.codes)
    qb = b.codes if b.codes.stride(0) == 1 else ops.row_major_bytes(b.codes.t()).t()
    return F.scaled_mm(mat_a=qa, mat_b=qb, scale_a=a.scale, scale_b=b.scale, output_dtype=out_dtype,
                       scale_recipe_a=F.ScalingType.TensorWise, scale_recipe_b=F.ScalingType.TensorWise)


def _scaled_mm(a: Tensor, b: Tensor, a_scale: Tensor, b_scale: Tensor, output_dtype: torch.dtype) -> Tensor:
    """fp8 codes a, b with their scales -> a @ b (reference fp8.py:25-49)."""
    return fp8_gemm(Fp8Operand(a, a_scale), Fp8Operand(b, b_scale), output_dtype)


def _grad_dtype(operand_dtype: torch.dtype) -> torch.dtype:
    wanted = getattr(config, "FP8_GRAD_DTYPE", None)
    return operand_dtype if wanted is None else wanted


class MatmulFp8(Function):
    """a @ b with both operands in fp8 (a bf16 operand is quantized with
    ``to_fp8``; an fp8 one needs its scale).  The output is bf16.

    Saved for the backward: the inputs as given (re-quantized there), or with
    ``config.CACHE_FP8_MATMUl`` the fp8 operands themselves (reference
    fp8.py:55-57, :73-74, :84-86).  The flag is read at each forward."""

    @staticmethod
    def forward(ctx, a: Tensor, b: Tensor, a_scale: Tensor | None = None,
                b_scale: Tensor | None = None) -> Tensor:
        opa, opb = as_fp8_operand(a, a_scale), as_fp8_operand(b, b_scale)
        ctx.cached = bool(config.CACHE_FP8_MATMUl)
        if ctx.cached:
            ctx.save_for_backward(opa.codes, opa.scale, opb.codes, opb.scale)
        else:
            ctx.save_for_backward(a, b)
            ctx.given_scales = (a_scale, b_scale)
        ctx.grad_dtypes = (opa.codes.dtype, opb.codes.dtype)
        ctx.in_dtypes = (a.dtype, b.dtype)
        # b given as a transposed view of row-major storage (W.T): its
        # gradient is formed in that storage's layout, so that autograd hands
        # it to W without a layout copy
        ctx.b_transposed = b.dim() == 2 and not b.is_contiguous() and b.t().is_contiguous()
        return fp8_gemm(opa, opb, torch.bfloat16)

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        if ctx.cached:
            qa, sa, qb, sb = ctx.saved_tensors
            opa, opb = Fp8Operand(qa, sa), Fp8Operand(qb, sb)
        else:
            a, b = ctx.saved_tensors
            opa = as_fp8_operand(a, ctx.given_scales[0])
            opb = as_fp8_operand(b, ctx.given_scales[1])
        g = Fp8Operand(*to_fp8(grad_output))
        need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grad_a = grad_b = None
        if need_a:
            grad_a = _as_input_dtype(fp8_gemm(g, opb.T, _grad_dtype(ctx.grad_dtypes[0])), ctx.in_dtypes[0])
        if need_b:
            if ctx.b_transposed:
                # (a^T g)^T = g^T a, delivered as a transposed view
                grad_b = _as_input_dtype(fp8_gemm(g.T, opa, _grad_dtype(ctx.grad_dtypes[1])), ctx.in_dtypes[1]).t()
            else:
                grad_b = _as_input_dtype(fp8_gemm(opa.T, g, _grad_dtype(ctx.grad_dtypes[1])), ctx.in_dtypes[1])
        return grad_a, grad_b, None, None


def _as_input_dtype(grad: Tensor, in_dtype: torch.dtype) -> Tensor:
    """An e4m3fn gradient of a bf16 input widened to bf16 by the HIP kernel
    (exact; the cast autograd would otherwise make with torch's float8 copy)."""
    if grad.dtype == torch.float8_e4m3fn and in_dtype == torch.bfloat16:
        from .src import hip_operators as ops
        return ops.widen_e4m3fn(grad)
    return grad


def matmul(a: Tensor, b: Tensor, fp8: bool, a_scale: Tensor | None = None,
           b_scale: Tensor | None = None) -> Tensor:
    """a @ b; with ``fp8`` through ``MatmulFp8`` (reference fp8.py:118-120)."""
    if not fp8:
        return a @ b
    return MatmulFp8.apply(a, b, a_scale, b_scale)


@torch.no_grad()
def to_fp8(x: Tensor) -> tuple[Tensor, Tensor]:
    """(e4m3fn copy of x, fp32 0-d scale) from the HIP amax and quantize
    kernels (reference fp8.py:123-129; rule in the module docstring)."""
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
