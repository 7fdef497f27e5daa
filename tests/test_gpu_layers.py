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


@pytest.mark.parametrize("k", [1.0, 0.5, 3.0])
@pytest.mark.parametrize("case", ["finite", "inf", "nan"])
def test_relu2_square_amax_matches_torch_ops(dev, k, case):
    """The fused pass of the fp8 ReLU^2 forward (reference layers.py:103-120:
    h.square_(); h.mul_(k); to_fp8(h)) against torch's own ops on the same GPU:
    h bit for bit (-0, subnormals, negatives; with Inf, or NaN of both signs,
    or values whose square overflows), then the amax it leaves gives the same
    codes and the same scale bits as to_fp8(h)."""
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import hip_operators as H
    from tests.helpers import special_bf16
    xb = special_bf16((257, 136), seed=31).view(torch.int16).clone()
    mag = xb.view(torch.int16).to(torch.int32) & 0x7fff
    xb[mag >= 0x7f80] = 0x3f80                           # no Inf / NaN unless asked for
    xb[mag == 0x7f7f] = 0x4100
    if case == "inf":
        xb.view(-1)[:3] = torch.tensor([0x7f80, -0x80, 0x5f80], dtype=torch.int16)   # +-Inf, 2^64 (square -> Inf)
    if case == "nan":
        xb.view(-1)[:2] = torch.tensor([0x7fc0, -0x40], dtype=torch.int16)           # +-NaN
    x = xb.to(dev).view(torch.bfloat16)
    want = x.clone()
    want.square_()
    want.mul_(k)
    h = x.clone()
    epoch = H.relu2_square_amax_(h, k)
    assert torch.equal(h.view(torch.int16), want.view(torch.int16))
    q, s = H.quantize_e4m3fn(h, epoch)
    qt, st = to_fp8(want)
    assert torch.equal(q.view(torch.uint8), qt.view(torch.uint8))
    assert torch.equal(s.view(torch.int32), st.view(torch.int32))
    if case == "finite":
        assert 0 < int((q.view(torch.uint8) & 0x7f).max().item()) < 0x7f   # real codes, not NaN


def test_ffn_relu2_fp8_forward_bit_identical_to_dense(dev):
    """With the fused square / scale / amax pass the compressed fp8 layer's y
    is bit-identical to the fp8 dense comparator's (the same h8, scale and
    GEMM), and z ends up holding k * relu(z)^2 as the in-place ops leave it."""
    from bitsparse_amd.dense import DenseFFNRelu2Fp8
    from bitsparse_amd.fp8 import matmul
    from bitsparse_amd.layers import FFNRelu2, Relu2Linear
    from bitsparse_amd.config import RELU2_SCALE
    x, W1, W2, _ = _mlp_inputs(256, 256, 512, seed=9)
    xs, W1s, W2s = (t.to(dev) for t in (x, W1, W2))
    ys = FFNRelu2.apply(xs, W1s, W2s, storage_dtype=torch.float8_e4m3fn)
    yd = DenseFFNRelu2Fp8.apply(xs, W1s, W2s)
    assert torch.equal(ys.view(torch.int16), yd.view(torch.int16))
    z = matmul(xs, W1s.T, True)
    want = z.clone().relu_()
    want.square_()
    want.mul_(RELU2_SCALE)
    Relu2Linear.apply(z, W2s, None, False, torch.float8_e4m3fn)
    assert torch.equal(z.view(torch.int16), want.view(torch.int16))
