"""GEMMs with a compressed operand (``src.sparse_matmul``: AspB, AspRelu2B,
spAB, reference lib_sparse/src/sparse_matmul.py:9-132), including the
``row_batch`` variants and the tile-row view they run on.

Where the product goes through the decompress kernel and a library GEMM, it
is the reference's computation on a bit-exact decompressed operand, so it is
compared bit for bit with the same library call on the original dense
matrix.  Where it goes through the reconstruct-into-LDS GEMM (bf16 storage),
it is compared with an fp32 product (2^-7 relative, as in test_gpu_gemm)."""
import pytest
import torch

from tests.helpers import preact_input, relu_input

pytestmark = pytest.mark.gpu


def _close(C, ref):
    scale = ref.abs().max().item() + 1e-6
    torch.testing.assert_close(C.float(), ref.float(), rtol=2 ** -7, atol=2 ** -7 * scale * 1e-2)


def _compress(h, dev, pack_sbit=False, dtype=None):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import dense_to_tilesparse
    dt = dtype or h.dtype
    buf = TensorBuffer(h.numel() * h.element_size() + 4096, device=dev, dtype=dt, pack_sbit=pack_sbit)
    # a first tensor in the buffer puts the operand at a nonzero value offset
    dense_to_tilesparse(relu_input((64, 64), 0.5, seed=99, dtype=dt).to(dev), None, buf, pack_sbit)
    scale = torch.ones((), device=dev) if dt != torch.bfloat16 else None
    return dense_to_tilesparse(h.to(dev), scale, buf, pack_sbit)


@pytest.mark.parametrize("rows", [64, 200, 320])
def test_tile_rows_view_decompresses_to_the_rows(dev, rows):
    from bitsparse_amd.src.sparse_matmul import decoded, tile_rows
    h = relu_input((rows, 192), 0.6, seed=1)
    sp = _compress(h, dev)
    full = decoded(sp, False)
    assert torch.equal(full.cpu(), h)
    for first, stop in ((0, 1), (1, sp.grid_m), (0, sp.grid_m)):
        if first >= stop:
            continue
        v = tile_rows(sp, first, stop)
        r0, r1 = 64 * first, min(64 * stop, rows)
        assert tuple(v.shape) == (r1 - r0, 192)
        assert torch.equal(decoded(v, False), full[r0:r1])
        assert torch.equal(decoded(v, True), decoded(sp, True)[r0:r1])


@pytest.mark.parametrize("row_batch", [0, 64, 100, 256, 10000])
def test_aspb_bf16_row_batch_runs_the_lds_gemm(dev, row_batch):
    """bf16 storage: every row_batch is the one LDS-GEMM launch (no dense B)."""
    from bitsparse_amd.src.sparse_matmul import AspB, AspRelu2B, decoded
    K, N, M = 448, 320, 256
    h = relu_input((K, N), 0.5, seed=2)
    dY = preact_input((K, M), seed=3).to(dev)
    sp = _compress(h, dev)
    C = AspB(dY.T, sp, row_batch=row_batch)
    _close(C, dY.T.float() @ h.to(dev).float())
    assert torch.equal(C, AspB(dY.T, sp, row_batch=0))
    C2 = AspRelu2B(dY.T, sp, row_batch=row_batch)
    _close(C2, dY.T.float() @ decoded(sp, True).float())     # the operand k*v^2 rounded to bf16


@pytest.mark.parametrize("row_batch", [0, 128, 200])
def test_aspb_packed_runs_the_lds_gemm_as_raw_storage(dev, row_batch):
    """Packed (pack_sbit) bf16 storage takes the LDS GEMM like raw storage:
    every row_batch is its one launch (no dense B), bit-identical to the
    raw-storage product of the same activation."""
    from bitsparse_amd.src.sparse_matmul import AspB, AspRelu2B, decoded
    K, N, M = 320, 256, 128
    h = relu_input((K, N), 0.5, seed=4)
    dY = preact_input((K, M), seed=5).to(dev)
    sp = _compress(h, dev, pack_sbit=True)
    raw = _compress(h, dev)
    for fn in (AspB, AspRelu2B):
        got = fn(dY.T, sp, row_batch=row_batch)
        assert torch.equal(got, fn(dY.T, raw, row_batch=row_batch))
        assert torch.equal(got, fn(dY.T, sp, row_batch=0))
    _close(AspB(dY.T, sp, row_batch=row_batch), dY.T.float() @ h.to(dev).float())
    _close(AspRelu2B(dY.T, sp, row_batch=row_batch), dY.T.float() @ decoded(sp, True).float())


@pytest.mark.parametrize("row_batch", [0, 128])
def test_aspb_fp8_storage(dev, row_batch):
    """fp8 (e4m3fn) storage with fp8 A: the product runs in fp8 with both
    scales (reference sparse_matmul.py:24-28 through MatmulFp8)."""
    from bitsparse_amd.fp8 import matmul, to_fp8
    from bitsparse_amd.src.functions import quantize_and_compress
    from bitsparse_amd.src.sparse_matmul import AspB
    K, N, M = 384, 256, 128
    h = relu_input((K, N), 0.5, seed=6).to(dev)
    dY = preact_input((K, M), seed=7).to(dev)
    q, s, sp = quantize_and_compress(h)
    g8, gs = to_fp8(dY)
    got = AspB(g8.T, sp, A_scale=gs, row_batch=row_batch)
    ref = matmul(g8.T, q, True, a_scale=gs, b_scale=s)
    if row_batch <= 0:
        assert torch.equal(got, ref)
    else:
        _close(got, ref)


@pytest.mark.parametrize("row_batch", [0, 64, 200])
@pytest.mark.parametrize("give_out", [False, True])
def test_spab_bf16(dev, row_batch, give_out):
    from bitsparse_amd.src.sparse_matmul import spAB
    M, N, K = 300, 256, 192
    a = relu_input((M, N), 0.7, seed=8)
    B = preact_input((N, K), seed=9).to(dev)
    sp = _compress(a, dev)
    out = torch.full((M, K), 7.0, device=dev, dtype=torch.bfloat16) if give_out else None
    got = spAB(sp, B, out=out, row_batch=row_batch)
    ad = a.to(dev)
    if row_batch <= 0:
        assert torch.equal(got, ad @ B)
        if give_out:
            assert bool((out == 7.0).all())       # reference ignores out here
    else:
        ref = torch.empty((M, K), device=dev, dtype=torch.bfloat16)
        step = max(1, row_batch // 64) * 64
        for r0 in range(0, M, step):
            torch.mm(ad[r0:r0 + step], B, out=ref[r0:r0 + step])
        assert torch.equal(got, ref)
        if give_out:
            assert got is out


def test_spab_fp8_storage(dev):
    from bitsparse_amd.fp8 import matmul
    from bitsparse_amd.src.functions import quantize_and_compress
    from bitsparse_amd.src.sparse_matmul import spAB
    M, N, K = 256, 192, 128
    a = relu_input((M, N), 0.5, seed=10).to(dev)
    B = (0.1 * preact_input((N, K), seed=11)).to(dev)
    q, s, sp = quantize_and_compress(a)
    assert torch.equal(spAB(sp, B), matmul(q, B, True, a_scale=s))
    got = spAB(sp, B, row_batch=64)
    ref = torch.cat([matmul(q[r0:r0 + 64], B, True, a_scale=s) for r0 in range(0, M, 64)])
    assert torch.equal(got, ref)
