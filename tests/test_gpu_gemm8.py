"""fp8-operand reconstruct-into-LDS GEMM (bs_gemm_compressed_b_fp8).

The reference multiplies fp8 storage in fp8 on a dense operand it
decompresses (lib_sparse/src/sparse_matmul.py:24-28, :109-113): AspB takes
the stored codes with their scale, AspRelu2B re-quantizes the bf16 k*v^2
(times bf16(scale^2)) with to_fp8 (lib_sparse/fp8.py:123-129).  The kernel
forms that operand from the stored codes inside the GEMM.

Pinned two ways:
* exactly: with A = I (e4m3fn 1.0, scale 1) every output is one product
  1.0 * Bq[k, n] scaled once by sB, so C must equal bf16(Bq * sB) of the
  reference's own operand -- to_fp8(unpack_relu2_batch_(B)) for AspRelu2B,
  the decompressed codes with their scale for AspB -- bit for bit, and the
  kernel's sB must equal to_fp8's scale exactly;
* numerically: random A against the fp32 product of the same quantized
  operands, within 2^-7 of max |C| (fp32 accumulation order, one bf16
  rounding).
"""
import pytest
import torch

from tests.helpers import preact_input, relu_input

pytestmark = pytest.mark.gpu


def _identity_fp8(n, dev):
    eye = torch.zeros((n, n), dtype=torch.uint8, device=dev)
    eye.fill_diagonal_(0x38)                      # e4m3fn 1.0
    return eye.view(torch.float8_e4m3fn), torch.ones((), device=dev)


def _relu2_operand(sp):
    """The reference's fp8 operand of AspRelu2B: to_fp8 of the bf16 unpack."""
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src.sparse_matmul import decoded
    return to_fp8(decoded(sp, True))


def _compressed_e4m3(K, N, mu, seed, dev):
    from bitsparse_amd.src.functions import quantize_and_compress
    z = (preact_input((K, N), mu=mu, seed=seed)).to(dev)
    _, _, sp = quantize_and_compress(z.relu(), None)
    return sp


def _compressed_e5m2(K, N, seed, dev):
    from bitsparse_amd.src.functions import dense_to_tilesparse
    x = relu_input((K, N), 0.6, seed=seed).to(torch.float8_e5m2).to(dev)
    return dense_to_tilesparse(x, torch.tensor(0.37, device=dev))


# (K = M, N): 256-row and 512-row workgroups, partial tiles in K and N, and a
# split-K grid (few output tiles, 32 K-steps)
SHAPES = [(256, 200), (512, 320), (320, 128), (2048, 64), (100, 70)]


@pytest.mark.parametrize("KN", SHAPES)
@pytest.mark.parametrize("storage", ["e4m3fn", "e5m2"])
def test_relu2_operand_bit_exact_with_identity(dev, KN, storage):
    from bitsparse_amd.src import dw_gemm
    K, N = KN
    sp = _compressed_e4m3(K, N, -0.8, 5, dev) if storage == "e4m3fn" else _compressed_e5m2(K, N, 6, dev)
    q, s = _relu2_operand(sp)
    A, sa = _identity_fp8(K, dev)
    sb_out = torch.empty((), device=dev)
    C = dw_gemm.gemm_compressed_b_fp8(A, sa, sp, square=True, b_scale_out=sb_out)
    assert torch.equal(sb_out.view(torch.int32), s.view(torch.int32)), (sb_out.item(), s.item())
    want = (q.float() * s).to(torch.bfloat16)
    assert torch.equal(C.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("KN", SHAPES)
@pytest.mark.parametrize("storage", ["e4m3fn", "e5m2"])
def test_stored_codes_bit_exact_with_identity(dev, KN, storage):
    """AspB on fp8 storage: the stored codes times their scale."""
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.sparse_matmul import decoded
    K, N = KN
    sp = _compressed_e4m3(K, N, 0.0, 7, dev) if storage == "e4m3fn" else _compressed_e5m2(K, N, 8, dev)
    codes = decoded(sp, False)
    A, sa = _identity_fp8(K, dev)
    C = dw_gemm.gemm_compressed_b_fp8(A, sa, sp, square=False)
    want = (codes.float() * sp.scale).to(torch.bfloat16)
    assert torch.equal(C.view(torch.int16), want.view(torch.int16))


def _trimmed(sp, lead):
    """sp with its values alone in a buffer of exactly lead + nnz bytes, at
    vals_offset = lead: the last run ends at the buffer's end."""
    from bitsparse_amd.bitsparse import BitsparseTensor
    p = sp.prefix.cpu().to(torch.int64)
    vo = int(sp.vals_offset.item())
    nnz = int(p[-1] - p[0])
    buf = torch.zeros(lead + nnz, dtype=torch.uint8, device=sp.vals.device)
    buf[lead:] = sp.vals.view(torch.uint8)[vo + int(p[0]):vo + int(p[0]) + nnz]
    prefix = (p - p[0]).to(torch.int32).view(torch.uint32).to(sp.prefix.device)
    return BitsparseTensor(buf.view(sp.vals.dtype), sp.bitmask, prefix, sp.shape, sp.dtype, sp.grid_m, sp.grid_n,
                           sp.BLOCK_M, sp.BLOCK_N, scale=sp.scale,
                           vals_offset=torch.full((), lead, dtype=torch.int64, device=sp.vals.device))


@pytest.mark.parametrize("lead", [0, 5, 16])
@pytest.mark.parametrize("square", [True, False])
def test_vals_ending_inside_a_run_unit(dev, lead, square):
    """Values in a buffer that ends mid 16-byte unit (and starts off a unit
    boundary when lead % 16 != 0): the unit crossing the end must carry the
    last bytes, as from the full-size buffer."""
    from bitsparse_amd.src import dw_gemm
    K, N = 512, 320
    for seed in range(20, 40):
        sp = _compressed_e4m3(K, N, -0.8, seed, dev)
        p = sp.prefix.cpu().to(torch.int64)
        if (lead + int(p[-1] - p[0])) % 16:
            break
    spt = _trimmed(sp, lead)
    assert spt.vals.numel() % 16 != 0
    A, sa = _identity_fp8(K, dev)
    want = dw_gemm.gemm_compressed_b_fp8(A, sa, sp, square=square)
    got = dw_gemm.gemm_compressed_b_fp8(A, sa, spt, square=square)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("lead", [0, 5])
def test_relu2_largest_code_in_the_last_partial_unit(dev, lead):
    """sB comes from the largest stored code, and the value run is mapped
    through the code table before the GEMM: with the one largest code as the
    last byte of a buffer that ends mid 16-byte unit (and a run that starts
    off a dword boundary for lead = 5), the unit crossing the end must still
    be read in full, by the code maximum and by the mapping."""
    from bitsparse_amd.src import dw_gemm
    K, N = 512, 320
    for seed in range(20, 40):
        sp = _compressed_e4m3(K, N, -0.8, seed, dev)
        p = sp.prefix.cpu().to(torch.int64)
        if (lead + int(p[-1] - p[0])) % 16:
            break
    spt = _trimmed(sp, lead)
    raw = spt.vals.view(torch.uint8)
    assert raw.numel() % 16 != 0
    raw[lead:].clamp_(max=0x40)               # stored codes stay positive, all below the last
    raw[-1] = 0x7e                            # e4m3fn 448, the only code above 0x40
    q, s = _relu2_operand(spt)
    A, sa = _identity_fp8(K, dev)
    sb_out = torch.empty((), device=dev)
    C = dw_gemm.gemm_compressed_b_fp8(A, sa, spt, square=True, b_scale_out=sb_out)
    assert torch.equal(sb_out.view(torch.int32), s.view(torch.int32)), (sb_out.item(), s.item())
    want = (q.float() * s).to(torch.bfloat16)
    assert torch.equal(C.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("M,K,N", [(256, 256, 256), (512, 1024, 384), (192, 640, 200), (64, 4096, 64),
                                   (1000, 512, 700)])
@pytest.mark.parametrize("square", [True, False])
@pytest.mark.parametrize("a_transposed", [True, False])
def test_random_a_against_fp32(dev, M, K, N, square, a_transposed):
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.sparse_matmul import decoded
    sp = _compressed_e4m3(K, N, -0.5, 9, dev)
    if a_transposed:                               # A = dY^T, the MLP backward's call shape
        dY = preact_input((K, M), seed=10).to(dev)
        qd, sa = to_fp8(dY)
        A = qd.T
    else:
        qa, sa = to_fp8(preact_input((M, K), seed=11).to(dev))
        A = qa
    if square:
        qb, sb = _relu2_operand(sp)
    else:
        qb, sb = decoded(sp, False), sp.scale
    C = dw_gemm.gemm_compressed_b_fp8(A, sa, sp, square=square)
    ref = (A.float() @ qb.float()) * (sa * sb)
    tol = 2 ** -7 * (ref.abs().max().item() + 1e-30)
    torch.testing.assert_close(C.float(), ref, rtol=2 ** -7, atol=tol)


def test_aspb_and_asprelu2b_route_fp8_storage_through_the_kernel(dev, monkeypatch):
    """AspB / AspRelu2B with fp8 storage and fp8 (or bf16, quantized) A run
    the LDS kernel and agree with the decompress + hipBLASLt path within the
    fp8 GEMMs' own accumulation-order differences."""
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import dw_gemm, sparse_matmul
    calls = []
    real = dw_gemm.gemm_compressed_b_fp8
    monkeypatch.setattr(dw_gemm, "gemm_compressed_b_fp8", lambda *a, **k: calls.append(1) or real(*a, **k))
    K, N, M = 512, 384, 256
    sp = _compressed_e4m3(K, N, -1.0, 12, dev)
    dY = preact_input((K, M), seed=13).to(dev)
    qd, sd = to_fp8(dY)
    for fn in (sparse_matmul.AspB, sparse_matmul.AspRelu2B):
        got = fn(qd.T, sp, A_scale=sd)
        got_bf16_a = fn(dY.T, sp)                  # bf16 A: quantized by to_fp8 first, as the reference does
        monkeypatch.setattr(sparse_matmul, "USE_LDS_GEMM", False)
        lib = fn(qd.T, sp, A_scale=sd)
        monkeypatch.setattr(sparse_matmul, "USE_LDS_GEMM", True)
        tol = 2 ** -7 * lib.float().abs().max().item()
        torch.testing.assert_close(got.float(), lib.float(), rtol=2 ** -7, atol=tol)
        torch.testing.assert_close(got_bf16_a.float(), lib.float(), rtol=2 ** -7, atol=tol)
    assert len(calls) == 4


def test_nan_scale_propagates(dev):
    """A NaN stored scale makes every element of the reference's dense operand
    NaN (0 * NaN for the cleared ones), so to_fp8's scale and every output is
    NaN; the kernel's table reproduces that."""
    from bitsparse_amd.bitsparse import BitsparseTensor
    from bitsparse_amd.src import dw_gemm
    K, N = 256, 128
    sp = _compressed_e4m3(K, N, -0.5, 14, dev)
    spn = BitsparseTensor(sp.vals, sp.bitmask, sp.prefix, sp.shape, sp.dtype, sp.grid_m, sp.grid_n,
                          sp.BLOCK_M, sp.BLOCK_N, scale=torch.tensor(float("nan"), device=dev),
                          vals_offset=sp.vals_offset)
    q, s = _relu2_operand(spn)
    assert torch.isnan(s)
    A, sa = _identity_fp8(K, dev)
    C = dw_gemm.gemm_compressed_b_fp8(A, sa, spn, square=True)
    assert torch.isnan(C.float()).all()
