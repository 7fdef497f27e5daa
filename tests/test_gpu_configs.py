"""BASELINE configs at their own sizes on the GPU.

* one GPT-2-small MLP training step (8192 x 768 -> 3072 -> 768,
  W ~ N(0, 0.02), x, dY ~ N(0, 1), CPU generator seed 0): the layer's
  compressed activation bit-exact against the oracle; y, dx, dW1
  bit-identical to the dense-activation comparator; dW2 (reconstruct-into-LDS
  GEMM) within 2^-6 of an fp32 product.
* the 8B-class ReLU^2 step (4096 rows, 4096 -> 16384 -> 4096,
  bias for ~90% zeros, e4m3fn storage): the layer's quantized + compressed
  activation bit-exact against the oracle's to_fp8 + compress; gradients
  against the reference's fp8 dense comparator at fp8 tolerance.
* 12 residual blocks x <- x + FFNRelu(rms_norm(x)) (the
  reference's harness, experiments/run_relu.py:22-28): loss and x.grad
  bit-identical to the dense-activation stack, dW1 bit-identical, dW2 within
  bf16 tolerance, and a lower peak memory; with the library GEMM for dW2 the
  whole tracking vector of experiment.py:56-66 matches at the reference's
  3e-6 (experiment.py:24, :160-164).
* every sweep point, bit-exact against the oracle, lives in
  tests/test_gpu_configs2.py.
* the reference's benchmark matrix (experiments/benchmark.py:12, :121-146):
  shapes (1000, 4096), (4000, 4096), (15000, 4096) x sparsity 0.5 / 0.8 x
  pack_sbit, exact round trip and the vram_size() storage ratio.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits

pytestmark = pytest.mark.gpu


def _layer_ctx(y):
    """The autograd node of the compressed layer (it holds h_sparse until
    the backward runs)."""
    node, seen = y.grad_fn, 0
    while not hasattr(node, "h_sparse"):
        node = node.next_functions[0][0]
        seen += 1
        assert seen < 8, "compressed layer node not found"
    return node


def _check_vs_oracle(sp, q_bits, code):
    bm, pf, v = O.compress(q_bits, code)
    assert (bits(sp.bitmask) == bm).all(), "bitmask"
    assert (bits(sp.prefix) == pf).all(), "prefix"
    off = int(sp.vals_offset.reshape(-1)[0].item())
    assert (bits(sp.vals)[off:off + v.size] == v).all(), "vals"
    return v.size


def _rel_err(a, b):
    return ((a.float() - b.float()).abs().max() / (b.float().abs().max() + 1e-6)).item()


def test_configs1_gpt2_mlp_step(dev):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.dense import DenseFFNRelu
    from bitsparse_amd.layers import FFNRelu
    g = torch.Generator().manual_seed(0)
    B, D, H = 8192, 768, 3072
    x = torch.randn((8, 1024, D), generator=g).to(torch.bfloat16)
    W1 = (0.02 * torch.randn((H, D), generator=g)).to(torch.bfloat16)
    W2 = (0.02 * torch.randn((D, H), generator=g)).to(torch.bfloat16)
    dY = torch.randn((8, 1024, D), generator=g).to(torch.bfloat16).to(dev)
    buf = TensorBuffer(2 * B * H, device=dev)
    xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    y = FFNRelu.apply(xs, W1s, W2s, sparse_data=buf)
    sp = _layer_ctx(y).h_sparse
    with torch.no_grad():
        h = (xs.detach().reshape(-1, D) @ W1s.detach().T).relu_()
    nnz = _check_vs_oracle(sp, bits(h), O.BF16)
    assert 0.45 < 1 - nnz / h.numel() < 0.55
    assert sp.vram_size() < 0.6 * h.numel() * 2
    y.backward(dY)
    xd, W1d, W2d = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    yd = DenseFFNRelu.apply(xd.reshape(-1, D), W1d, W2d).reshape(8, 1024, D)
    yd.backward(dY)
    assert torch.equal(y, yd)
    assert torch.equal(xs.grad, xd.grad)
    assert torch.equal(W1s.grad, W1d.grad)
    ref = dY.reshape(-1, D).float().T @ h.float()
    assert _rel_err(W2s.grad, ref) < 2 ** -6
    assert not buf.overflowed()


def test_configs3_relu2_fp8_mlp_step(dev):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.dense import DenseFFNRelu2Fp8
    from bitsparse_amd.fp8 import matmul, to_fp8
    from bitsparse_amd.layers import FFNRelu2
    from bitsparse_amd.src.sparse_matmul import decoded
    g = torch.Generator().manual_seed(0)
    B, D, H = 4096, 4096, 16384
    x = torch.randn((B, D), generator=g).to(torch.bfloat16).to(dev)
    W1 = (0.02 * torch.randn((H, D), generator=g)).to(torch.bfloat16).to(dev)
    W2 = (0.02 * torch.randn((D, H), generator=g)).to(torch.bfloat16).to(dev)
    dY = torch.randn((B, D), generator=g).to(torch.bfloat16).to(dev)
    b1 = torch.full((H,), -1.2816 * 0.02 * D ** 0.5, dtype=torch.bfloat16, device=dev)
    buf = TensorBuffer(B * H, device=dev, dtype=torch.float8_e4m3fn)
    xs, W1s, W2s = (t.clone().requires_grad_() for t in (x, W1, W2))
    y = FFNRelu2.apply(xs, W1s, W2s, b1, sparse_data=buf, storage_dtype=torch.float8_e4m3fn)
    sp = _layer_ctx(y).h_sparse
    with torch.no_grad():
        r = (matmul(x, W1.T, True) + b1).relu_()
    q, s = O.to_fp8(bits(r))
    assert float(sp.scale.item()) == s
    nnz = _check_vs_oracle(sp, q, O.E4M3FN)
    assert 0.85 < 1 - nnz / r.numel() < 0.95
    # dW2 of the compressed path: the fp8 product of to_fp8(dY)^T with the
    # re-quantized k r^2 s^2 (reference sparse_matmul.py:109-113)
    k_r2 = decoded(sp, True)
    y.backward(dY)
    xd, W1d, W2d = (t.clone().requires_grad_() for t in (x, W1, W2))
    DenseFFNRelu2Fp8.apply(xd, W1d, W2d, b1).backward(dY)
    for name, a, b in (("dx", xs.grad, xd.grad), ("dW1", W1s.grad, W1d.grad),
                       ("dW2", W2s.grad, W2d.grad)):
        assert torch.isfinite(a).all(), name
        assert _rel_err(a, b) < 2 ** -3, name
    # exact operands: to_fp8(dY) and to_fp8(k r^2 s^2) with their scales, an
    # fp32 product scaled once; the kernel differs only in its fp32 summation
    # order and the final bf16 rounding (one fp8 step in either operand's
    # scale or rounding would be far outside this bound)
    qd, sd = to_fp8(dY)
    qb, sb = to_fp8(k_r2)
    ref = (qd.float().T @ qb.float()) * (sd * sb)
    torch.testing.assert_close(W2s.grad.float(), ref, rtol=2 ** -7, atol=2 ** -7 * ref.abs().max().item() * 1e-2)
    assert not buf.overflowed()


def _stack(x0, Ws, compressed, buf):
    from bitsparse_amd.dense import DenseFFNRelu
    from bitsparse_amd.layers import FFNRelu
    import torch.nn.functional as F
    if buf is not None:
        buf.reset_buffer()
    x = x0
    for W1, W2 in Ws:
        xi = F.rms_norm(x, x.shape[1:])
        if compressed:
            x = x + FFNRelu.apply(xi, W1, W2, sparse_data=buf)
        else:
            x = x + DenseFFNRelu.apply(xi, W1, W2)
    return (x - x0).abs().mean()


@pytest.mark.parametrize("lds_gemm", [True, False])
def test_configs4_twelve_block_stack(dev, lds_gemm, monkeypatch):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src import sparse_matmul
    monkeypatch.setattr(sparse_matmul, "USE_LDS_GEMM", lds_gemm)
    g = torch.Generator().manual_seed(0)
    L, B, D, H = 12, 8192, 768, 3072
    Ws = [((0.02 * torch.randn((H, D), generator=g)).to(torch.bfloat16).to(dev),
           (0.02 * torch.randn((D, H), generator=g)).to(torch.bfloat16).to(dev)) for _ in range(L)]
    x = torch.randn((B, D), generator=g).to(torch.bfloat16).to(dev)
    res = {}
    buf = None
    for compressed in (False, True):
        params = [(W1.clone().requires_grad_(), W2.clone().requires_grad_()) for W1, W2 in Ws]
        x0 = x.clone().requires_grad_()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        if compressed:       # counted in the compressed peak: values of ~50% of 12 activations
            buf = TensorBuffer(2 * L * B * H * 55 // 100, device=dev)
        loss = _stack(x0, params, compressed, buf)
        loss.backward()
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        res[compressed] = (loss.detach(), x0.grad, [p[0].grad for p in params],
                           [p[1].grad for p in params], peak)
    ld, gxd, dW1d, dW2d, peak_d = res[False]
    lc, gxc, dW1c, dW2c, peak_c = res[True]
    assert torch.equal(lc, ld)
    assert torch.equal(gxc, gxd)
    for a, b in zip(dW1c, dW1d):
        assert torch.equal(a, b)
    for a, b in zip(dW2c, dW2d):
        if lds_gemm:
            assert _rel_err(a, b) < 2 ** -6
        else:
            assert torch.equal(a, b)
    assert not buf.overflowed()
    assert peak_c < 0.9 * peak_d, (peak_c, peak_d)
    if not lds_gemm:
        # the reference's own check (experiment.py:56-66, :160-164)
        def tracking(loss, gx, dW1, dW2):
            t = [loss, gx.std()] + [w.std() for pair in zip(dW1, dW2) for w in pair]
            return torch.stack([v.float() for v in t]) * 1e3
        torch.testing.assert_close(tracking(lc, gxc, dW1c, dW2c), tracking(ld, gxd, dW1d, dW2d),
                                   atol=3e-6, rtol=3e-6)


@pytest.mark.parametrize("pack_sbit", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_reference_benchmark_matrix(dev, pack_sbit, dtype):
    """experiments/benchmark.py's matrix (8 tensors per shape, data from its
    generate_data: |N(0,1)| with a uniform zero mask): exact round trip and
    the storage ratio vram_size() / dense bytes from the format's sizes."""
    from bitsparse_amd.bitsparse import bits_per_value
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from tests.test_gpu_codec import decompress
    gen = torch.Generator(device=dev).manual_seed(0)
    for sparsity in (0.5, 0.8):
        for shape in ((1000, 4096), (4000, 4096), (15000, 4096)):
            ratios = []
            for _ in range(8):
                data = torch.randn(shape, generator=gen, dtype=torch.bfloat16, device=dev).abs_()
                data.masked_fill_(torch.rand(shape, generator=gen, device=dev) < sparsity, 0)
                data = data.to(dtype)
                scale = torch.ones((), device=dev) if dtype != torch.bfloat16 else None
                sp = dense_to_tilesparse(data, scale, pack_sbit=pack_sbit)
                out = decompress(sp) if not pack_sbit else _decompress_packed(sp)
                assert torch.equal(out.view(torch.uint8), data.view(torch.uint8)), (shape, sparsity)
                M, N = shape
                T = ((M + 63) // 64) * ((N + 63) // 64)
                nnz = int((data.float() > 0).sum().item())
                vb = data.element_size()
                val_bytes = (nnz * bits_per_value(dtype) + 7) // 8 if pack_sbit else nnz * vb
                stored = val_bytes + 512 * T + 4 * (T + 1)
                assert sp.vram_size() == stored
                ratios.append(stored / (M * N * vb))
            ratio = sum(ratios) / len(ratios)
            expect = (1 - sparsity) * (bits_per_value(dtype) / 8 / vb if pack_sbit else 1) + 1 / (8 * vb)
            assert abs(ratio - expect) < 0.01, (shape, sparsity, ratio, expect)


def _decompress_packed(sp):
    from bitsparse_amd.src.hip_operators import unpack_batch_
    M, N = sp.shape
    out = torch.empty((M, N), device=sp.vals.device, dtype=sp.dtype)
    return unpack_batch_(sp, out, 0, sp.grid_n, N, M, sp.grid_m * sp.grid_n)
