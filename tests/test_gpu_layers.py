"""Autograd layers with compressed activations against the dense-activation
comparators (experiments/experiment.py:242-384 semantics) on the same inputs.

Reference tolerance: experiment.py:24,160-164 compares loss and x.grad.std()
at 3e-6 for bf16.  Here every gradient tensor is compared: the forward output
and dx are bit-identical paths up to GEMM ordering, and dW2 comes from a
different GEMM (the reconstruct-into-LDS kernel vs hipBLASLt), so gradients
are compared to an fp32 CPU computation of the same math at bf16 tolerance
(2^-6 relative to the tensor's max)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _mlp_inputs(B, D, H, seed, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, D), generator=g).to(torch.bfloat16)
    W1 = (0.05 * torch.randn((H, D), generator=g) + shift).to(torch.bfloat16)
    W2 = (0.05 * torch.randn((D, H), generator=g)).to(torch.bfloat16)
    dY = torch.randn((B, D), generator=g).to(torch.bfloat16)
    return x, W1, W2, dY


def _close(a, b, name):
    scale = b.abs().max().item() + 1e-6
    err = (a.float().cpu() - b.float().cpu()).abs().max().item() / scale
    assert err < 2 ** -6, f"{name}: max error {err:.3e} of max |ref|"


@pytest.mark.parametrize("use_buffer", [False, True])
def test_ffn_relu_matches_dense(dev, use_buffer):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.dense import DenseFFNRelu
    from bitsparse_amd.layers import FFNRelu
    x, W1, W2, dY = _mlp_inputs(512, 256, 1024, seed=1)
    buf = TensorBuffer(2 * 512 * 1024, device=dev) if use_buffer else None
    xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    y = FFNRelu.apply(xs, W1s, W2s, sparse_data=buf)
    y.backward(dY.to(dev))
    xd, W1d, W2d = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    yd = DenseFFNRelu.apply(xd, W1d, W2d)
    yd.backward(dY.to(dev))
    assert torch.equal(y, yd)                         # same forward ops
    assert torch.equal(xs.grad, xd.grad)              # mask kernel == threshold_backward
    assert torch.equal(W1s.grad, W1d.grad)
    xf, W1f, W2f = (t.float().requires_grad_() for t in (x, W1, W2))
    (torch.relu(xf @ W1f.T) @ W2f.T).backward(dY.float())
    _close(W2s.grad, W2f.grad, "dW2")
    if buf is not None:
        assert not buf.overflowed()


def test_ffn_relu2_matches_dense(dev):
    from bitsparse_amd.dense import DenseFFNRelu2
    from bitsparse_amd.layers import FFNRelu2
    x, W1, W2, dY = _mlp_inputs(512, 256, 768, seed=2)
    xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    FFNRelu2.apply(xs, W1s, W2s).backward(dY.to(dev))
    xd, W1d, W2d = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    DenseFFNRelu2.apply(xd, W1d, W2d).backward(dY.to(dev))
    assert torch.equal(xs.grad, xd.grad)              # relu2 grad == grad_z * (2 k r)
    assert torch.equal(W1s.grad, W1d.grad)
    xf, W1f, W2f = (t.float().requires_grad_() for t in (x, W1, W2))
    (torch.relu(xf @ W1f.T).square() @ W2f.T).backward(dY.float())
    _close(W2s.grad, W2f.grad, "dW2")


def test_ffn_relu_leading_batch_dims_and_bias(dev):
    from bitsparse_amd.layers import FFNRelu
    g = torch.Generator().manual_seed(3)
    x = torch.randn((4, 64, 128), generator=g).to(torch.bfloat16).to(dev).requires_grad_()
    W1 = (0.05 * torch.randn((384, 128), generator=g)).to(torch.bfloat16).to(dev).requires_grad_()
    W2 = (0.05 * torch.randn((128, 384), generator=g)).to(torch.bfloat16).to(dev).requires_grad_()
    b1 = torch.zeros(384, dtype=torch.bfloat16, device=dev, requires_grad=True)
    b2 = torch.zeros(128, dtype=torch.bfloat16, device=dev, requires_grad=True)
    y = FFNRelu.apply(x, W1, W2, b1, b2)
    assert y.shape == (4, 64, 128)
    y.sum().backward()
    assert x.grad.shape == x.shape and b1.grad is not None and b2.grad is not None


def test_ffn_relu2_fp8_storage_matches_fp8_dense(dev):
    """fp8 (e4m3fn) activation storage against the reference's fp8 dense
    comparator (experiment.py:330-384 with an fp8 DTYPE).  Both run every GEMM
    in per-tensor fp8; they differ only in bf16 rounding order of the ReLU^2
    reconstruction, which can move an fp8 re-quantization by one step, so the
    bound is fp8-sized: 2^-3 of each tensor's max."""
    from bitsparse_amd.dense import DenseFFNRelu2Fp8
    from bitsparse_amd.layers import FFNRelu2
    x, W1, W2, dY = _mlp_inputs(256, 256, 512, seed=4)
    xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    ys = FFNRelu2.apply(xs, W1s, W2s, storage_dtype=torch.float8_e4m3fn)
    ys.backward(dY.to(dev))
    xd, W1d, W2d = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    yd = DenseFFNRelu2Fp8.apply(xd, W1d, W2d)
    yd.backward(dY.to(dev))
    for name, a, b in (("y", ys, yd), ("dx", xs.grad, xd.grad), ("dW1", W1s.grad, W1d.grad),
                       ("dW2", W2s.grad, W2d.grad)):
        scale = b.abs().max().item() + 1e-6
        err = (a.float() - b.float()).abs().max().item() / scale
        assert err < 2 ** -3, f"{name}: {err:.3e}"
