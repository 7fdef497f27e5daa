"""The fp8 GEMM facade (``bitsparse_amd.fp8``: MatmulFp8 / matmul) against an
fp64 CPU computation on the same quantized operands, and the fp8 ReLU layer
against the reference's fp8 dense comparator.

Semantics pinned (reference lib_sparse/fp8.py:52-120):
  * forward: bf16(acc * sa * sb), acc = sum of exact fp8 x fp8 products in fp32;
  * gradients: the same product of to_fp8(grad) with the other operand,
    delivered in the operand's fp8 dtype (output_dtype=a_fp8.dtype /
    b_fp8.dtype, fp8.py:107,112), i.e. rounded to e4m3fn with saturation at
    +-448, then widened to bf16 by autograd.

Tolerance: the library accumulates in fp32 in an order (and with MFMA-internal
roundings) it does not document, so the GPU value must lie between the
target-format roundings of p - t and p + t, where p is the exact (fp64)
product and t = 4 (K + 6) 2^-24 * sum|a_i b_i|: four times the error bound of
fp32 summation in any order plus the scale products.  Away from rounding
boundaries this leaves exactly one admissible code; the tests also require
that most outputs are decided that way (fp8 outputs; bf16's grid is finer
than the accumulation error where terms cancel), so a wrong rule cannot
pass.  The rounding rule itself is pinned exactly: an fp8 result is the
saturating round-to-nearest-even of the same product delivered in fp32."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _codes_f64(q: torch.Tensor) -> np.ndarray:
    return q.detach().cpu().float().double().numpy()


def _round_e4m3_sat(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(x.astype(np.float32)).clamp(-448.0, 448.0)
    return t.to(torch.float8_e4m3fn).float().double().numpy()


def _round_bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).double().numpy()


def _check_rounded(got: torch.Tensor, qa, sa, qb, sb, rounder, min_decided=0.9, what=""):
    """got ~ rounder(qa*sa @ qb*sb) within the fp32-summation interval."""
    a, b = _codes_f64(qa), _codes_f64(qb)
    s = float(sa) * float(sb)
    p = (a @ b) * s
    K = a.shape[1]
    t = 4 * (K + 6) * 2.0 ** -24 * (np.abs(a) @ np.abs(b)) * s
    lo, hi = rounder(p - t), rounder(p + t)
    g = got.detach().cpu().double().numpy()
    bad = ~((g >= lo) & (g <= hi))
    assert not bad.any(), f"{what}: {int(bad.sum())} values outside the rounding interval"
    decided = float((lo == hi).mean())
    assert decided >= min_decided, f"{what}: only {decided:.3f} of the outputs are decided"


def _operands(M, K, N, seed, gmul=1.0):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((M, K), generator=g).to(torch.bfloat16)
    b = (0.05 * torch.randn((K, N), generator=g)).to(torch.bfloat16)
    dy = (gmul * torch.randn((M, N), generator=g)).to(torch.bfloat16)
    return a, b, dy


@pytest.mark.parametrize("gmul", [1.0, 3000.0])      # 3000: gradients past +-448 saturate
def test_matmul_fp8_forward_and_grads_vs_fp64(dev, gmul):
    from bitsparse_amd.fp8 import matmul, to_fp8
    M, K, N = 256, 512, 384
    a, b, dy = _operands(M, K, N, seed=1, gmul=gmul)
    ad, bd = a.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    y = matmul(ad, bd, True)
    y.backward(dy.to(dev))
    qa, sa = to_fp8(a.to(dev))
    qb, sb = to_fp8(b.to(dev))
    qg, sg = to_fp8(dy.to(dev))
    assert y.dtype == torch.bfloat16
    _check_rounded(y, qa, sa, qb, sb, _round_bf16, min_decided=0.1, what="y")
    # gradients in e4m3fn (saturating), widened to bf16
    assert ad.grad.dtype == torch.bfloat16 and bd.grad.dtype == torch.bfloat16
    for gr in (ad.grad, bd.grad):
        assert torch.equal(gr.float(), gr.to(torch.float8_e4m3fn).float()), "not e4m3fn values"
    _check_rounded(ad.grad, qg, sg, qb.t(), sb, _round_e4m3_sat, what="da")
    _check_rounded(bd.grad, qa.t(), sa, qg, sg, _round_e4m3_sat, what="db")
    # exactly: the saturating RNE of the library's fp32 result of the same product
    from bitsparse_amd.fp8 import Fp8Operand, fp8_gemm
    da32 = fp8_gemm(Fp8Operand(qg, sg), Fp8Operand(qb.t(), sb), torch.float32)
    assert torch.equal(ad.grad.float(), da32.clamp(-448, 448).to(torch.float8_e4m3fn).float())
    y32 = fp8_gemm(Fp8Operand(qa, sa), Fp8Operand(qb, sb), torch.float32)
    assert torch.equal(y, y32.to(torch.bfloat16))
    if gmul > 1.0:
        assert ad.grad.abs().max().item() == 448.0, "saturation at 448 expected"
        assert not torch.isnan(ad.grad).any()


def test_matmul_fp8_operand_given_with_scale(dev):
    """An fp8 operand with its scale is used as given (fp8.py:60-71)."""
    from bitsparse_amd.fp8 import matmul, to_fp8
    a, b, dy = _operands(128, 256, 192, seed=2)
    qa, sa = to_fp8(a.to(dev))
    bd = b.to(dev).requires_grad_()
    y = matmul(qa, bd, True, a_scale=sa)
    qb, sb = to_fp8(b.to(dev))
    _check_rounded(y, qa, sa, qb, sb, _round_bf16, min_decided=0.1, what="y")
    y.backward(dy.to(dev))
    qg, sg = to_fp8(dy.to(dev))
    _check_rounded(bd.grad, qa.t(), sa, qg, sg, _round_e4m3_sat, what="db")
    with pytest.raises(AssertionError):
        matmul(qa, bd, True)                          # fp8 operand without its scale
    with pytest.raises(AssertionError):
        matmul(a.to(dev), bd, True, a_scale=sa)       # bf16 operand with a scale


def test_cache_fp8_matmul_gives_identical_gradients(dev, monkeypatch):
    """CACHE_FP8_MATMUl=True saves the fp8 operands instead of re-quantizing
    them in the backward (fp8.py:55-57, :73-74, :84-86); quantization is
    deterministic, so every gradient is bit-identical."""
    from bitsparse_amd import config
    from bitsparse_amd.fp8 import matmul
    a, b, dy = _operands(256, 384, 256, seed=3)
    grads = {}
    for cached in (False, True):
        monkeypatch.setattr(config, "CACHE_FP8_MATMUl", cached)
        ad, bd = a.to(dev).requires_grad_(), b.to(dev).requires_grad_()
        y = matmul(ad, bd, True)
        y.backward(dy.to(dev))
        grads[cached] = (y.detach(), ad.grad, bd.grad)
    for x0, x1 in zip(grads[False], grads[True]):
        assert torch.equal(x0, x1)


def test_fp8_grad_dtype_knob(dev, monkeypatch):
    """config.FP8_GRAD_DTYPE = bf16: the same products rounded to bf16."""
    from bitsparse_amd import config
    from bitsparse_amd.fp8 import matmul, to_fp8
    a, b, dy = _operands(256, 256, 128, seed=4)
    monkeypatch.setattr(config, "FP8_GRAD_DTYPE", torch.bfloat16)
    ad, bd = a.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    matmul(ad, bd, True).backward(dy.to(dev))
    qb, sb = to_fp8(b.to(dev))
    qg, sg = to_fp8(dy.to(dev))
    _check_rounded(ad.grad, qg, sg, qb.t(), sb, _round_bf16, min_decided=0.1, what="da")
    assert not torch.equal(ad.grad.float(), ad.grad.to(torch.float8_e4m3fn).float())


def _mlp(B, D, H, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, D), generator=g).to(torch.bfloat16)
    W1 = (0.05 * torch.randn((H, D), generator=g)).to(torch.bfloat16)
    W2 = (0.05 * torch.randn((D, H), generator=g)).to(torch.bfloat16)
    dY = torch.randn((B, D), generator=g).to(torch.bfloat16)
    return x, W1, W2, dY


@pytest.mark.parametrize("use_buffer", [False, True])
def test_ffn_relu_fp8_storage_matches_fp8_dense(dev, use_buffer, monkeypatch):
    """FFNRelu(dtype=float8_e4m3fn) (reference layers.py:32-35, :52-58)
    against the reference's fp8 dense comparator (experiment.py:242-306 with
    an fp8 DTYPE): the same quantized activation, the same fp8 GEMMs.

    y and dW2 are bit-identical; with bf16 gradients requested, dx is too
    (value-equal: the sparse mask writes +0 where the dense product gives
    -0).  With the reference's e4m3fn gradients, dx and dW1 are the e4m3fn
    rounding of those bf16 values, up to one bf16 rounding step."""
    from bitsparse_amd import config
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.dense import DenseFFNReluFp8
    from bitsparse_amd.layers import FFNRelu
    B, D, H = 512, 256, 1024
    x, W1, W2, dY = _mlp(B, D, H, seed=5)
    res = {}
    for mode in (torch.bfloat16, None):
        monkeypatch.setattr(config, "FP8_GRAD_DTYPE", mode)
        buf = TensorBuffer(B * H, device=dev, dtype=torch.float8_e4m3fn) if use_buffer else None
        xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
        y = FFNRelu.apply(xs, W1s, W2s, sparse_data=buf, dtype=torch.float8_e4m3fn)
        y.backward(dY.to(dev))
        res[mode] = (y.detach(), xs.grad, W1s.grad, W2s.grad)
        if buf is not None:
            assert not buf.overflowed()
    xd, W1d, W2d = (t.to(dev).requires_grad_() for t in (x, W1, W2))
    yd = DenseFFNReluFp8.apply(xd, W1d, W2d)
    yd.backward(dY.to(dev))
    y16, dx16, dW1_16, dW2_16 = res[torch.bfloat16]
    assert torch.equal(y16, yd)
    assert torch.equal(dW2_16, W2d.grad)
    assert torch.equal(dx16, xd.grad)
    y8, dx8, dW1_8, dW2_8 = res[None]
    assert torch.equal(y8, yd) and torch.equal(dW2_8, W2d.grad)
    for name, g8, g16 in (("dx", dx8, dx16), ("dW1", dW1_8, dW1_16)):
        assert torch.equal(g8.float(), g8.to(torch.float8_e4m3fn).float()), f"{name}: not e4m3fn"
        f = g16.double()
        lo = f * (1 - 2.0 ** -8)
        hi = f * (1 + 2.0 ** -8)
        lo_r = torch.minimum(lo, hi).float().clamp(-448, 448).to(torch.float8_e4m3fn).double()
        hi_r = torch.maximum(lo, hi).float().clamp(-448, 448).to(torch.float8_e4m3fn).double()
        g = g8.double()
        assert bool(((g >= lo_r) & (g <= hi_r)).all()), f"{name}: not the e4m3fn rounding of the bf16 gradient"


# ---------------------------------------------------------------------------
# operand layout change: bs_transpose_u8 (the fp8 GEMM's row-major /
# column-major copies, reference fp8.py:36-43, :111)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(4, 16), (16, 16), (128, 128), (300, 208), (132, 400), (4096, 1024),
                                   (1028, 4112)])
def test_transpose_u8_bit_exact(dev, shape):
    """Every byte lands at its transposed place: whole and partial 128 x 128
    tiles, rows not a multiple of 128 or 16, padded leading dimensions."""
    from bitsparse_amd.src import hip_operators as H
    R, C = shape
    a = np.random.default_rng(R * 131 + C).integers(0, 256, size=(R, C), dtype=np.uint8)
    x = torch.from_numpy(a).to(dev)
    assert (H.transpose_u8(x).cpu().numpy() == a.T).all()
    # strided input (row stride C + 32) into a strided output (row stride R + 4)
    big = torch.zeros((R, C + 32), dtype=torch.uint8, device=dev)
    big[:, :C] = x
    obig = torch.full((C, R + 4), 7, dtype=torch.uint8, device=dev)
    H.transpose_u8(big[:, :C], out=obig[:, :R])
    ob = obig.cpu().numpy()
    assert (ob[:, :R] == a.T).all() and (ob[:, R:] == 7).all()


def test_transpose_u8_fp8_view_and_row_major_bytes(dev):
    """fp8 codes keep their bits; row_major_bytes copies a transposed view
    through the kernel and returns a row-major tensor unchanged."""
    from bitsparse_amd.src import hip_operators as H
    a = np.random.default_rng(9).integers(0, 256, size=(256, 512), dtype=np.uint8)
    q = torch.from_numpy(a).to(dev).view(torch.float8_e4m3fn)
    assert H.row_major_bytes(q) is q
    r = H.row_major_bytes(q.t())
    assert r.is_contiguous() and r.dtype == torch.float8_e4m3fn
    assert (r.view(torch.uint8).cpu().numpy() == a.T).all()


def test_transpose_u8_refuses_unsupported_shapes(dev):
    """Invalid arguments come back as ValueError (BS_ERR_INVALID)."""
    from bitsparse_amd.src import hip_operators as H
    x = torch.zeros((8, 24), dtype=torch.uint8, device=dev)          # C % 16 != 0
    assert not H.transpose_u8_supported(x)
    with pytest.raises(ValueError, match="C must be a multiple of 16 and R of 4"):
        H.transpose_u8(x)
    y = torch.zeros((6, 32), dtype=torch.uint8, device=dev)          # R % 4 != 0
    assert not H.transpose_u8_supported(y)
    with pytest.raises(ValueError, match="C must be a multiple of 16 and R of 4"):
        H.transpose_u8(y)
    z = torch.zeros((6, 24), dtype=torch.uint8, device=dev)          # falls back to torch's copy
    assert torch.equal(H.row_major_bytes(z.t()), z.t().contiguous())


# ---------------------------------------------------------------------------
# gradient delivery: e4m3fn gradients of bf16 inputs widened by
# bs_widen_e4m3fn, and a W.T operand's gradient formed in W's own layout
# ---------------------------------------------------------------------------
def test_widen_e4m3fn_every_code(dev):
    """All 256 codes (NaN, +-0, subnormals, +-448), a length that is not a
    multiple of 16, and a transposed view: bit-identical to torch's cast on
    the GPU and on the CPU."""
    from bitsparse_amd.src import hip_operators as H
    codes = torch.arange(256, dtype=torch.uint8).repeat(5)[:1000]
    q = codes.view(torch.float8_e4m3fn)
    want_cpu = q.to(torch.bfloat16).view(torch.int16)
    got = H.widen_e4m3fn(q.to(dev))
    assert torch.equal(got.view(torch.int16).cpu(), want_cpu)
    assert torch.equal(got.view(torch.int16), q.to(dev).to(torch.bfloat16).view(torch.int16))
    m = q[:992].reshape(31, 32).to(dev)
    gt = H.widen_e4m3fn(m.t())
    assert gt.shape == (32, 31) and gt.t().is_contiguous()
    assert torch.equal(gt.view(torch.int16), m.t().to(torch.bfloat16).view(torch.int16))


def test_transposed_weight_operand_gradient(dev):
    """matmul(x, W.T): W.grad arrives in W's row-major layout (formed as
    g^T x), the same saturating e4m3fn rounding of the same product as the
    gradient of an untransposed operand, and x.grad is bit-identical."""
    from bitsparse_amd.fp8 import matmul, to_fp8
    a, b, dy = _operands(256, 384, 320, seed=6)
    W = b.t().contiguous()                            # [N, K]: the layer's weight layout
    ad, Wd = a.to(dev).requires_grad_(), W.to(dev).requires_grad_()
    matmul(ad, Wd.T, True).backward(dy.to(dev))
    assert Wd.grad.is_contiguous() and Wd.grad.dtype == torch.bfloat16
    qa, sa = to_fp8(a.to(dev))
    qg, sg = to_fp8(dy.to(dev))
    _check_rounded(Wd.grad.t(), qa.t(), sa, qg, sg, _round_e4m3_sat, what="dW")
    a2, b2 = a.to(dev).requires_grad_(), b.to(dev).requires_grad_()
    matmul(a2, b2, True).backward(dy.to(dev))
    assert torch.equal(ad.grad, a2.grad)
