"""Autograd MLP layers whose ReLU / ReLU^2 activation is saved compressed.

Mirrors reference lib_sparse/layers.py: ``ReluLinear`` (:20-66), ``FFNRelu``
(:69-94), ``Relu2Linear`` (:100-151), ``FFNRelu2`` (:154-177) — same
signatures, including the reference's ``dtype`` (FFNRelu) vs
``storage_dtype`` (FFNRelu2) keyword names.  Forward: GEMM -> ReLU (in
place) -> [fp8 quantize] -> compress (HIP) -> GEMM.  Backward: dW from the
compressed activation (reconstruct-into-LDS GEMM for bf16), dZ from the
bitmask (HIP mask / ReLU^2-gradient kernels).
"""
from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd import Function

from .bitsparse import BitsparseTensor, TensorBuffer
from .config import RELU2_SCALE
from .fp8 import is_fp8, matmul, to_fp8
from .src.functions import (fused_linear_relu_ok, linear_relu_and_compress, relu2_and_compress,
                            relu2_fused_ok, relu2_quantize_and_compress, relu_and_compress,
                            relu_quantize_and_compress)
from .src.hip_operators import mask_with_bitmask_, quantize_e4m3fn, relu2_grad_sparse_, relu2_square_amax_
from .src.sparse_matmul import AspB, AspRelu2B

# FFNRelu / FFNRelu2 with bf16 storage into a TensorBuffer run the up-projection
# GEMM, ReLU and compress as one kernel (bs_linear_relu_compress) when the
# operands qualify; False keeps the library GEMM + bias add + compress path.
USE_FUSED_UP = False


# ------------------------------------------------------------
# ReLU layers
# ------------------------------------------------------------
class ReluLinear(Function):
    """y = relu(z) @ W.T with relu(z) saved compressed."""

    @staticmethod
    def forward(ctx, z, W, sparse_data: TensorBuffer | None = None, pack_sbit: bool = False,
                dtype: torch.dtype = torch.bfloat16):
        ctx.dtype = dtype
        ctx.save_for_backward(W)
        # h = z.relu_() fused into the compress pass (z is still updated in place)
        if is_fp8(dtype):
            # any fp8 dtype stores e4m3fn codes + scale: the reference quantizes
            # with to_fp8, whose output is e4m3fn for e5m2 too (fp8.py:123-129)
            h, scale, h_sparse = relu_quantize_and_compress(z, sparse_data, pack_sbit)
        else:
            scale = None
            h, h_sparse = relu_and_compress(z, sparse_data, pack_sbit)

        ctx.h_sparse = h_sparse
        y = matmul(h, W.T, is_fp8(dtype), a_scale=scale)
        return y

    @staticmethod
    @torch.compiler.disable
    def backward(ctx, grad_output: Tensor):
        W = ctx.saved_tensors[0]
        needs_z = ctx.needs_input_grad[0]
        h: BitsparseTensor = ctx.h_sparse
        ctx.h_sparse = None

        fp8 = is_fp8(ctx.dtype)
        if fp8:
            grad_output, scale = to_fp8(grad_output)
        else:
            grad_output, scale = grad_output, None

        grad_W2 = AspB(grad_output.T, h, A_scale=scale)

        if needs_z:
            grad_h = matmul(grad_output, W, fp8=fp8, a_scale=scale)
            grad_z = mask_with_bitmask_(grad_h, h)
        else:
            grad_z = None
        return grad_z, grad_W2, None, None, None


class FFNRelu:
    """FFN block with ReLU activation: y = relu(x @ W1.T + b1) @ W2.T + b2."""

    @staticmethod
    def apply(x, W1, W2, b1=None, b2=None, *,
              sparse_data: TensorBuffer | None = None, pack_sbit: bool = False,
              dtype: torch.dtype = torch.bfloat16):
        """x [*bs, d_in], W1 [d_ff, d_in], W2 [d_out, d_ff], b1 [d_ff], b2 [d_out]
        -> [*bs, d_out]."""
        bs_dims = x.shape[:-1]
        x = x.reshape(-1, x.shape[-1])

        if not is_fp8(dtype) and not pack_sbit and USE_FUSED_UP and fused_linear_relu_ok(x, W1, b1, sparse_data):
            y = _UpReluLinear.apply(x, W1, b1, W2, sparse_data, False)
        else:
            z = matmul(x, W1.T, is_fp8(dtype))
            if b1 is not None:
                z = z + b1
            y = ReluLinear.apply(z, W2, sparse_data, pack_sbit, dtype)

        y = y.reshape(*bs_dims, y.shape[-1])
        if b2 is not None:
            y = y + b2
        return y


# ------------------------------------------------------------
# ReLU^2 layers
# ------------------------------------------------------------
class Relu2Linear(Function):
    """y = (k * relu(z)^2) @ W.T with r = relu(z) saved compressed."""

    @staticmethod
    def forward(ctx, z, W, sparse_data: TensorBuffer | None, pack_sbit: bool = False,
                storage_dtype: torch.dtype = torch.bfloat16):
        ctx.dtype = storage_dtype
        ctx.save_for_backward(W)
        # h = z.relu_() fused into the compress pass (z is still updated in place)
        fused_sq = relu2_fused_ok(z, sparse_data, pack_sbit, RELU2_SCALE)
        if is_fp8(storage_dtype):
            # e4m3fn codes for every fp8 storage dtype, as to_fp8 makes them;
            # the forward multiplies the bf16 square, so no dense e4m3fn copy
            if fused_sq:
                # the compress also writes h = k r^2 into z; amax|h| follows
                # from the amax of r
                _, h_sparse, epoch = relu2_quantize_and_compress(z, sparse_data, RELU2_SCALE)
            else:
                _, _, h_sparse = relu_quantize_and_compress(z, sparse_data, pack_sbit, dense_out=False)
                # h.square_(); h.mul_(k) and the amax of to_fp8(h) in one pass
                epoch = relu2_square_amax_(z, RELU2_SCALE)
            ctx.h_sparse = h_sparse
            # h ends up in z, as the reference's in-place ops leave it
            h8, h_scale = quantize_e4m3fn(z, epoch)
            return matmul(h8, W.T, True, a_scale=h_scale)
        if fused_sq:
            h_sparse = relu2_and_compress(z, sparse_data, RELU2_SCALE)
            h = z
        else:
            h, h_sparse = relu_and_compress(z, sparse_data, pack_sbit)
            if h.is_contiguous():
                # h.square_(); h.mul_(k) in one pass, bit for bit (its amax goes unused)
                relu2_square_amax_(h, RELU2_SCALE)
            else:
                h.square_()
                h.mul_(RELU2_SCALE)
        ctx.h_sparse = h_sparse
        return matmul(h, W.T, False)

    @staticmethod
    @torch.compiler.disable
    def backward(ctx, grad_output: Tensor):
        W = ctx.saved_tensors[0]
        needs_z = ctx.needs_input_grad[0]
        h: BitsparseTensor = ctx.h_sparse
        ctx.h_sparse = None

        fp8 = is_fp8(ctx.dtype)
        if fp8:
            grad_output, scale = to_fp8(grad_output)
        else:
            grad_output, scale = grad_output, None

        grad_W2 = AspRelu2B(grad_output.T, h, A_scale=scale)

        if needs_z:
            grad_h = matmul(grad_output, W, fp8=fp8, a_scale=scale)
            grad_z = relu2_grad_sparse_(grad_h, h)
        else:
            grad_z = None
        return grad_z, grad_W2, None, None, None


class FFNRelu2:
    """FFN block with ReLU^2 activation: y = k*relu(x @ W1.T + b1)^2 @ W2.T + b2."""

    @staticmethod
    def apply(x, W1, W2, b1=None, b2=None, *,
              sparse_data: TensorBuffer | None = None, pack_sbit: bool = False,
              storage_dtype: torch.dtype = torch.bfloat16):
        bs_dims = x.shape[:-1]
        x = x.reshape(-1, x.shape[-1])
        if (not is_fp8(storage_dtype) and not pack_sbit and USE_FUSED_UP
                and fused_linear_relu_ok(x, W1, b1, sparse_data)):
            y = _UpReluLinear.apply(x, W1, b1, W2, sparse_data, True)
        else:
            z = matmul(x, W1.T, is_fp8(storage_dtype))
            if b1 is not None:
                z = z + b1
            y = Relu2Linear.apply(z, W2, sparse_data, pack_sbit, storage_dtype)
        y = y.reshape(*bs_dims, y.shape[-1])
        if b2 is not None:
            y = y + b2
        return y


# ------------------------------------------------------------
# fused up-projection (bf16 storage into a TensorBuffer)
# ------------------------------------------------------------
class _UpReluLinear(Function):
    """The autograd node of ``z = x @ W1.T + b1`` followed by ReluLinear
    (square=False) or Relu2Linear (square=True), with z, relu(z) and its
    compressed form produced by one kernel.  Backward repeats the calls of the
    two-node graph: the same dz from the bitmask (or the ReLU^2 gradient), then
    autograd's own products for x, W1 and b1."""

    @staticmethod
    def forward(ctx, x, W1, b1, W2, sparse_data: TensorBuffer, square: bool):
        h, h_sparse = linear_relu_and_compress(x, W1, b1, sparse_data)
        ctx.h_sparse = h_sparse
        ctx.square = square
        ctx.has_b1 = b1 is not None
        ctx.save_for_backward(x, W1, W2)
        if square:
            h.square_()
            h.mul_(RELU2_SCALE)
        return matmul(h, W2.T, False)

    @staticmethod
    @torch.compiler.disable
    def backward(ctx, grad_output: Tensor):
        x, W1, W2 = ctx.saved_tensors
        h: BitsparseTensor = ctx.h_sparse
        ctx.h_sparse = None
        if ctx.square:
            grad_W2 = AspRelu2B(grad_output.T, h)
        else:
            grad_W2 = AspB(grad_output.T, h)
        grad_x = grad_W1 = grad_b1 = None
        if any(ctx.needs_input_grad[:3]):
            grad_h = matmul(grad_output, W2, fp8=False)
            grad_z = relu2_grad_sparse_(grad_h, h) if ctx.square else mask_with_bitmask_(grad_h, h)
            # the products autograd forms for z = x @ W1.T + b1
            if ctx.needs_input_grad[0]:
                grad_x = grad_z.mm(W1)
            if ctx.needs_input_grad[1]:
                grad_W1 = grad_z.t().mm(x)          # W1's own layout, as autograd forms it for x @ W1.T
            if ctx.has_b1 and ctx.needs_input_grad[2]:
                grad_b1 = grad_z.sum(0)
        # the forward kernel's look-back must not have given up: checked once
        # this node's kernels are queued (the check waits for that forward
        # kernel, so checking first would leave the GPU idle while the host
        # queues them); gradients from a misplaced value run are never returned
        h.lookback_check.raise_if_timed_out()
        return grad_x, grad_W1, grad_b1, grad_W2, None, None
