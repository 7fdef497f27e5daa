"""Dense-activation comparators: the MLP blocks that save their activation
uncompressed.  They define the denominator of "compressed backward within
1.2x of dense backward" and the dense side of the gradient parity tests.

Semantics of reference experiments/experiment.py:242-306 (``FFN``: saves
relu(z) and masks with threshold_backward) and :322-384 (``FFNRelu2_2``:
saves r = relu(z), rebuilds k*r^2 in backward), bf16 path.
"""
from __future__ import annotations

import torch
from torch.autograd import Function

from .config import RELU2_SCALE


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
