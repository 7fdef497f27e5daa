"""Dense-activation comparators: the MLP blocks that save their activation
uncompressed.  They define the denominator of "compressed backward within
1.2x of dense backward" and the dense side of the gradient parity tests.

Semantics of reference experiments/experiment.py:242-306 (``FFN``: saves
relu(z) and masks with threshold_backward) and :322-384 (``FFNRelu2_2``:
saves r = relu(z), rebuilds k*r^2 in backward).  ``DenseFFNReluFp8`` and
``DenseFFNRelu2Fp8`` are their fp8 modes (the same functions with an fp8
DTYPE): fp8 GEMMs, the activation cached as e4m3fn + scale, k*r^2 rebuilt
in bf16.

``apply_ckpt`` / ``forward_ckpt`` are the reference's activation-checkpointing
comparator (experiment.py:300-306, :378-384): the block saves only its inputs
and recomputes the activation in backward.
"""
from __future__ import annotations

import torch
import torch.utils.checkpoint
from torch.autograd import Function

from .config import RELU2_SCALE
from .fp8 import matmul, to_fp8


class DenseFFNRelu(Function):
    """y = relu(x @ W1.T) @ W2.T saving the dense activation (bf16)."""

    @staticmethod
    def forward(ctx, x, W1, W2):
        z = x @ W1.T
        z.relu_()
        out = z @ W2.T
        ctx.save_for_backward(x, W1, W2, z)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        x, W1, W2, z = ctx.saved_tensors
        grad_z = grad_output @ W2
        grad_W2 = grad_output.T @ z
        grad_pre = torch.ops.aten.threshold_backward.grad_input(grad_z, z, 0, grad_input=grad_z)
        grad_x = grad_pre @ W1 if ctx.needs_input_grad[0] else None
        grad_W1 = grad_pre.T @ x
        return grad_x, grad_W1, grad_W2

    @staticmethod
    def forward_ckpt(x, W1, W2):
        """The block as plain autograd ops (recomputed in backward)."""
        return (x @ W1.T).relu_() @ W2.T

    @staticmethod
    def apply_ckpt(x, W1, W2):
        return torch.utils.checkpoint.checkpoint(DenseFFNRelu.forward_ckpt, x, W1, W2, use_reentrant=False)


class DenseFFNReluFp8(Function):
    """fp8 mode of DenseFFNRelu (reference experiment.py:242-306 with an fp8
    DTYPE): fp8 GEMMs, relu(z) saved as e4m3fn + scale, the ReLU mask taken
    from the saved codes (q > 0); optional first-layer bias b1 (no gradient),
    added before the activation."""

    @staticmethod
    def forward(ctx, x, W1, W2, b1=None):
        z = matmul(x, W1.T, True)
        if b1 is not None:
            z = z + b1
        z.relu_()
        z8, z_scale = to_fp8(z)
        ctx.save_for_backward(x, W1, W2, z8)
        ctx.z_scale = z_scale
        return matmul(z8, W2.T, True, a_scale=z_scale)

    @staticmethod
    def backward(ctx, grad_output):
        x, W1, W2, z8 = ctx.saved_tensors
        g8, gs = to_fp8(grad_output)
        grad_z = matmul(g8, W2, True, a_scale=gs)
        grad_W2 = matmul(g8.T, z8, True, a_scale=gs, b_scale=ctx.z_scale)
        grad_pre = grad_z * (z8.to(torch.bfloat16) > 0)
        del grad_z
        p8, ps = to_fp8(grad_pre)
        grad_x = matmul(p8, W1, True, a_scale=ps) if ctx.needs_input_grad[0] else None
        grad_W1 = matmul(p8.T, x, True, a_scale=ps)
        return grad_x, grad_W1, grad_W2, None


class DenseFFNRelu2(Function):
    """y = (k * relu(x @ W1.T)^2) @ W2.T saving r = relu(z) (bf16)."""

    @staticmethod
    def forward(ctx, x, W1, W2):
        z = x @ W1.T
        r = z.relu_()
        h = r.square()
        h.mul_(RELU2_SCALE)
        ctx.save_for_backward(x, W1, W2, r)
        return h @ W2.T

    @staticmethod
    def backward(ctx, grad_output):
        x, W1, W2, r = ctx.saved_tensors
        h = r.square().mul_(RELU2_SCALE)
        grad_W2 = grad_output.T @ h
        del h
        grad_z = grad_output @ W2
        grad_pre = grad_z * (2.0 * RELU2_SCALE * r)
        grad_x = grad_pre @ W1 if ctx.needs_input_grad[0] else None
        grad_W1 = grad_pre.T @ x
        return grad_x, grad_W1, grad_W2

    @staticmethod
    def forward_ckpt(x, W1, W2):
        r = (x @ W1.T).relu_()
        return r.square().mul_(RELU2_SCALE) @ W2.T

    @staticmethod
    def apply_ckpt(x, W1, W2):
        return torch.utils.checkpoint.checkpoint(DenseFFNRelu2.forward_ckpt, x, W1, W2, use_reentrant=False)


class DenseFFNRelu2Fp8(Function):
    """fp8 mode of DenseFFNRelu2: every GEMM per-tensor fp8, r = relu(z)
    saved as e4m3fn + scale (reference experiment.py:330-384); optional
    first-layer bias b1 (no gradient), added before the activation.

    ``WIDEN_WITH_HIP``: the reference dequantizes the saved codes with torch's
    float8 -> bf16 cast (``r_fp8.to(bfloat16)``, experiment.py:362), an
    elementwise copy that runs at a fraction of HBM speed on ROCm; set True,
    the comparator widens them with the library's exact e4m3fn -> bf16
    kernel instead (same bits), so the compressed path is timed against a
    comparator with the same fp8 plumbing."""
    WIDEN_WITH_HIP = False

    @staticmethod
    def forward(ctx, x, W1, W2, b1=None):
        z = matmul(x, W1.T, True)
        if b1 is not None:
            z = z + b1
        r = z.relu_()
        r_fp8, r_scale = to_fp8(r)
        h = r.square()
        h.mul_(RELU2_SCALE)
        ctx.save_for_backward(x, W1, W2, r_fp8)
        ctx.r_scale = r_scale
        return matmul(h, W2.T, True)

    @staticmethod
    def backward(ctx, grad_output):
        x, W1, W2, r_fp8 = ctx.saved_tensors
        g8, gs = to_fp8(grad_output)
        if DenseFFNRelu2Fp8.WIDEN_WITH_HIP:
            from .src.hip_operators import widen_e4m3fn
            r = widen_e4m3fn(r_fp8) * ctx.r_scale
        else:
            r = r_fp8.to(torch.bfloat16) * ctx.r_scale
        h = r.square().mul_(RELU2_SCALE)
        grad_W2 = matmul(g8.T, h, True, a_scale=gs)
        del h
        grad_z = matmul(g8, W2, True, a_scale=gs)
        grad_pre = grad_z * (2.0 * RELU2_SCALE * r)
        del grad_z, r
        p8, ps = to_fp8(grad_pre)
        grad_x = matmul(p8, W1, True, a_scale=ps) if ctx.needs_input_grad[0] else None
        grad_W1 = matmul(p8.T, x, True, a_scale=ps)
        return grad_x, grad_W1, grad_W2, None
