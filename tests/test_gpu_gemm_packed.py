"""Reconstruct-into-LDS GEMMs on packed (pack_sbit) storage:
bs_gemm_compressed_b_packed (bf16 values: the run's 15-bit fields unpacked to
bf16 by a pre-pass the GEMM stages from) and bs_gemm_compressed_b_fp8_packed
(7-bit fp8 codes, unpacked by the pass that maps them).

The packed and the raw storage of one activation hold the same values, and
both GEMMs run the same kernels over them (same workgroup shape, split and
accumulation order), so the packed call must reproduce the raw call bit for
bit; with A = I it must also reproduce the packed decompress (which the
oracle pins) exactly.  Streams that end inside the last unit's dwords (the
payload alone, exactly ceil(bits / 8) bytes, written by the oracle's packer
at a value offset) exercise the byte-wise tail reads.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, preact_input, relu_input

pytestmark = pytest.mark.gpu


def _pair_bf16(K, N, sparsity, seed, dev):
    from bitsparse_amd.src.functions import dense_to_tilesparse
    h = relu_input((K, N), sparsity, seed=seed).to(dev)
    return dense_to_tilesparse(h, None), dense_to_tilesparse(h, None, pack_sbit=True)


def _pair_fp8(K, N, storage, seed, dev):
    from bitsparse_amd.src.functions import dense_to_tilesparse, quantize_and_compress
    if storage == "e4m3fn":
        r = preact_input((K, N), mu=-0.6, seed=seed).relu().to(dev)
        _, _, raw = quantize_and_compress(r, None)
        _, _, pk = quantize_and_compress(r, None, pack_sbit=True)
        return raw, pk
    x = relu_input((K, N), 0.6, seed=seed).to(torch.float8_e5m2).to(dev)
    s = torch.tensor(0.37, device=dev)
    return dense_to_tilesparse(x, s), dense_to_tilesparse(x, s, pack_sbit=True)


def _identity_fp8(n, dev):
    eye = torch.zeros((n, n), dtype=torch.uint8, device=dev)
    eye.fill_diagonal_(0x38)                      # e4m3fn 1.0
    return eye.view(torch.float8_e4m3fn), torch.ones((), device=dev)


def _same(a, b):
    assert a.shape == b.shape
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _exact_stream(sp_raw, lead, code):
    """The packed form of sp_raw's value run alone: stream value `lead` on,
    in a buffer of exactly ceil((lead + nnz) * PB / 8) bytes (so the last
    value's byte is the buffer's last byte), prefix made relative to it."""
    from bitsparse_amd.bitsparse import BitsparseTensor
    p = sp_raw.prefix.cpu().to(torch.int64)
    vo = int(sp_raw.vals_offset.item())
    nnz = int(p[-1] - p[0])
    run = bits(sp_raw.vals[vo + int(p[0]):vo + int(p[0]) + nnz])
    nbytes = ((lead + nnz) * O.bits_per_value(code) + 7) // 8
    stream = np.zeros(nbytes, np.uint8)
    O.pack_bits(run, code, stream, lead)
    dev = sp_raw.vals.device
    prefix = (p - p[0]).to(torch.int32).view(torch.uint32).to(dev)
    return BitsparseTensor(torch.from_numpy(stream).to(dev), sp_raw.bitmask, prefix, sp_raw.shape, sp_raw.dtype,
                           sp_raw.grid_m, sp_raw.grid_n, sp_raw.BLOCK_M, sp_raw.BLOCK_N, scale=sp_raw.scale,
                           vals_offset=torch.full((), lead, dtype=torch.int64, device=dev), pack_sbit=True)


# ---------------------------------------------------------------------------
# bf16 storage
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("K", [320, 1024])           # 256- and 512-row workgroups (M = K)
@pytest.mark.parametrize("square", [False, True])
def test_bf16_packed_identity_reproduces_packed_decompress(dev, K, square):
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.sparse_matmul import decoded
    N = 448
    _, pk = _pair_bf16(K, N, 0.55, 31, dev)
    assert dw_gemm.supports(torch.eye(K, dtype=torch.bfloat16, device=dev), pk, square=square)
    C = dw_gemm.gemm_compressed_b(torch.eye(K, dtype=torch.bfloat16, device=dev), pk, square=square)
    _same(C, decoded(pk, square))


@pytest.mark.parametrize("M,K,N", [(256, 384, 448), (768, 2048, 640), (1000, 512, 700), (64, 4096, 130),
                                   (33, 64, 1)])
@pytest.mark.parametrize("square", [False, True])
@pytest.mark.parametrize("sparsity", [0.0, 0.5, 0.95])
def test_bf16_packed_equals_raw(dev, M, K, N, square, sparsity):
    from bitsparse_amd.src import dw_gemm
    raw, pk = _pair_bf16(K, N, sparsity, 32, dev)
    dY = preact_input((K, M), seed=33).to(dev)
    for A in (dY.T, preact_input((M, K), seed=34).to(dev)):      # transposed (AspB's call) and row-major
        _same(dw_gemm.gemm_compressed_b(A, pk, square=square), dw_gemm.gemm_compressed_b(A, raw, square=square))


@pytest.mark.parametrize("lead", [0, 3, 13])
@pytest.mark.parametrize("square", [False, True])
def test_bf16_packed_stream_ending_inside_the_last_unit(dev, lead, square):
    from bitsparse_amd.src import dw_gemm
    K, N, M = 512, 320, 256
    raw, _ = _pair_bf16(K, N, 0.6, 35, dev)
    spt = _exact_stream(raw, lead, O.BF16)
    A = preact_input((M, K), seed=36).to(dev)
    _same(dw_gemm.gemm_compressed_b(A, spt, square=square), dw_gemm.gemm_compressed_b(A, raw, square=square))


# ---------------------------------------------------------------------------
# fp8 storage
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("KN", [(256, 200), (512, 320), (2048, 64), (100, 70)])
@pytest.mark.parametrize("storage", ["e4m3fn", "e5m2"])
@pytest.mark.parametrize("square", [False, True])
def test_fp8_packed_equals_raw_with_identity(dev, KN, storage, square):
    from bitsparse_amd.src import dw_gemm
    K, N = KN
    raw, pk = _pair_fp8(K, N, storage, 37, dev)
    assert dw_gemm.supports_fp8(_identity_fp8(K, dev)[0], pk)
    A, sa = _identity_fp8(K, dev)
    sb_raw, sb_pk = torch.empty((), device=dev), torch.empty((), device=dev)
    want = dw_gemm.gemm_compressed_b_fp8(A, sa, raw, square=square, b_scale_out=sb_raw)
    got = dw_gemm.gemm_compressed_b_fp8(A, sa, pk, square=square, b_scale_out=sb_pk)
    assert torch.equal(sb_pk.view(torch.int32), sb_raw.view(torch.int32))
    _same(got, want)


@pytest.mark.parametrize("M,K,N", [(256, 256, 256), (512, 1024, 384), (64, 4096, 64)])
@pytest.mark.parametrize("square", [False, True])
def test_fp8_packed_equals_raw_random_a(dev, M, K, N, square):
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import dw_gemm
    raw, pk = _pair_fp8(K, N, "e4m3fn", 38, dev)
    qd, sa = to_fp8(preact_input((K, M), seed=39).to(dev))
    _same(dw_gemm.gemm_compressed_b_fp8(qd.T, sa, pk, square=square),
          dw_gemm.gemm_compressed_b_fp8(qd.T, sa, raw, square=square))


@pytest.mark.parametrize("lead", [0, 5, 9])
@pytest.mark.parametrize("square", [False, True])
def test_fp8_packed_stream_ending_inside_the_last_window(dev, lead, square):
    """The stream's payload alone, with the largest code as its last value:
    the code maximum (sB) and the unpacking must both read the final, partial
    dword byte by byte."""
    from bitsparse_amd.src import dw_gemm
    K, N = 512, 320
    raw, _ = _pair_fp8(K, N, "e4m3fn", 40, dev)
    p = raw.prefix.cpu().to(torch.int64)
    vo = int(raw.vals_offset.item())
    run = raw.vals.view(torch.uint8)[vo + int(p[0]):vo + int(p[-1])]
    run.clamp_(max=0x40)                       # every stored code below the last one
    run[-1] = 0x7e                             # e4m3fn 448
    spt = _exact_stream(raw, lead, O.E4M3FN)
    A, sa = _identity_fp8(K, dev)
    sb_raw, sb_pk = torch.empty((), device=dev), torch.empty((), device=dev)
    want = dw_gemm.gemm_compressed_b_fp8(A, sa, raw, square=square, b_scale_out=sb_raw)
    got = dw_gemm.gemm_compressed_b_fp8(A, sa, spt, square=square, b_scale_out=sb_pk)
    assert torch.equal(sb_pk.view(torch.int32), sb_raw.view(torch.int32))
    _same(got, want)


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------
def test_aspb_and_asprelu2b_route_packed_storage_through_the_lds_gemms(dev, monkeypatch):
    """pack_sbit operands of AspB / AspRelu2B go to the LDS GEMMs (no dense B)
    and agree with the decompress + library GEMM path."""
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import dw_gemm, sparse_matmul
    calls = []
    for name in ("gemm_compressed_b", "gemm_compressed_b_fp8"):
        real = getattr(dw_gemm, name)
        monkeypatch.setattr(dw_gemm, name, lambda *a, _r=real, _n=name, **k: calls.append(_n) or _r(*a, **k))
    K, N, M = 512, 384, 256
    dY = preact_input((K, M), seed=41).to(dev)
    _, pk16 = _pair_bf16(K, N, 0.5, 42, dev)
    _, pk8 = _pair_fp8(K, N, "e4m3fn", 43, dev)
    qd, sd = to_fp8(dY)
    for fn in (sparse_matmul.AspB, sparse_matmul.AspRelu2B):
        for sp, kw, A in ((pk16, {}, dY.T), (pk8, {"A_scale": sd}, qd.T)):
            got = fn(A, sp, **kw)
            monkeypatch.setattr(sparse_matmul, "USE_LDS_GEMM", False)
            lib = fn(A, sp, **kw)
            monkeypatch.setattr(sparse_matmul, "USE_LDS_GEMM", True)
            tol = 2 ** -7 * lib.float().abs().max().item()
            torch.testing.assert_close(got.float(), lib.float(), rtol=2 ** -7, atol=tol)
    assert calls == ["gemm_compressed_b", "gemm_compressed_b_fp8"] * 2
