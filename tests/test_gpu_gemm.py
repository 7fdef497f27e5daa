"""Reconstruct-into-LDS MFMA GEMM (bs_gemm_compressed_b) against an fp32
reference on the decompressed operand.  Tolerance: the kernel accumulates in
fp32 and rounds once to bf16, so results agree with the fp32 product to about
one bf16 ulp (2^-8 relative); the bound below is 2^-7 relative plus a small
absolute term for near-cancelling sums."""
import pytest
import torch

from tests.helpers import preact_input, relu_input

pytestmark = pytest.mark.gpu


def _ref(A, B_dense):
    return A.float() @ B_dense.float()


def _check(C, ref):
    assert C.dtype == torch.bfloat16 and C.shape == ref.shape
    scale = ref.abs().max().item() + 1e-6
    torch.testing.assert_close(C.float(), ref, rtol=2 ** -7, atol=2 ** -7 * scale * 1e-2)


@pytest.mark.parametrize("M,K,N", [(256, 64, 64), (300, 200, 130), (64, 100, 64), (768, 8192, 3072),
                                   (1000, 512, 700), (33, 64, 1), (255, 4096, 130), (600, 1000, 200),
                                   (513, 64, 65)])
def test_gemm_bf16(dev, M, K, N):
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse
    h = relu_input((K, N), 0.5, seed=1).to(dev)
    A = preact_input((M, K), seed=2).to(dev)
    sp = dense_to_tilesparse(h, None)
    assert dw_gemm.supports(A, sp, square=False)
    C = dw_gemm.gemm_compressed_b(A, sp, square=False)
    _check(C, _ref(A, h))


@pytest.mark.parametrize("d_out", [192, 1024, 768])   # 256-, 512- and 768-row workgroups
def test_gemm_transposed_a_and_buffer_offset(dev, d_out):
    """AspB's call shape: A = dY.T (a transposed view), h in a shared buffer."""
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from bitsparse_amd.src.sparse_matmul import AspB
    dY = preact_input((512, d_out), seed=3).to(dev)
    h1 = relu_input((512, 320), 0.7, seed=4).to(dev)
    h2 = relu_input((512, 320), 0.3, seed=5).to(dev)
    buf = TensorBuffer(2 * 2 * 512 * 320, device=dev)
    sp1 = dense_to_tilesparse(h1, None, buf)
    sp2 = dense_to_tilesparse(h2, None, buf)
    assert int(sp2.vals_offset.item()) > 0
    for h, sp in ((h1, sp1), (h2, sp2)):
        _check(AspB(dY.T, sp), _ref(dY.T, h))


@pytest.mark.parametrize("M", [320, 1024, 700])  # 256-, 512- and 768-row workgroups
@pytest.mark.parametrize("storage", ["bf16", "e4m3fn"])
def test_gemm_relu2_square(dev, storage, M):
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse, quantize_and_compress
    from bitsparse_amd.src.hip_operators import unpack_relu2_batch_
    K, N = 384, 448
    r = preact_input((K, N), seed=6).relu().to(dev)
    A = preact_input((M, K), seed=7).to(dev)
    if storage == "bf16":
        sp = dense_to_tilesparse(r, None)
    else:
        _, _, sp = quantize_and_compress(r, None)
    sq = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
    unpack_relu2_batch_(sp, sq, 0, sp.grid_n, N, K, sp.grid_m * sp.grid_n)
    assert dw_gemm.supports(A, sp, square=True)
    C = dw_gemm.gemm_compressed_b(A, sp, square=True)
    _check(C, _ref(A, sq))


def test_gemm_all_zero_and_dense_operands(dev):
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse
    A = preact_input((256, 128), seed=8).to(dev)
    for sparsity in (1.0, 0.0):
        h = relu_input((128, 192), sparsity, seed=9).to(dev)
        C = dw_gemm.gemm_compressed_b(A, dense_to_tilesparse(h, None), square=False)
        _check(C, _ref(A, h))


@pytest.mark.parametrize("K", [320, 1024, 768])  # 256-, 512- and 768-row workgroups
@pytest.mark.parametrize("storage,square", [("bf16", False), ("bf16", True), ("e4m3fn", True)])
def test_gemm_identity_reproduces_decoded_operand(dev, storage, square, K):
    """With A = I (K = M) every output is 1.0 * b accumulated in fp32, so C
    must equal the decompressed operand bit for bit: this pins the GEMM's
    in-LDS decode (ranks, byte permutes, hardware bf16 / fp8 conversions,
    ReLU^2 square and scale^2) to the decompress kernel, which the oracle
    pins."""
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse, quantize_and_compress
    from bitsparse_amd.src.hip_operators import unpack_batch_, unpack_relu2_batch_
    N = 448
    r = preact_input((K, N), seed=11).relu().to(dev)
    if storage == "bf16":
        sp = dense_to_tilesparse(r, None)
    else:
        _, _, sp = quantize_and_compress(r, None)
    ref = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
    if square:
        unpack_relu2_batch_(sp, ref, 0, sp.grid_n, N, K, sp.grid_m * sp.grid_n)
    else:
        unpack_batch_(sp, ref, 0, sp.grid_n, N, K, sp.grid_m * sp.grid_n)
    A = torch.eye(K, dtype=torch.bfloat16, device=dev)
    C = dw_gemm.gemm_compressed_b(A, sp, square=square)
    assert torch.equal(C.view(torch.int16), ref.view(torch.int16))


def test_gemm_relu2_nonfinite_scale_matches_decompress(dev):
    """ReLU^2 with fp8 storage and an infinite scale: every decoded element is
    bf16(k v^2 * bf16(scale^2)), so cleared elements are 0 * inf = NaN, as
    the decompress kernel (and the reference's unpack-then-scale,
    lib_sparse/src/triton_operators.py:160-161) produces them.  The LDS GEMM's
    cleared-element fix-up must give the same NaN / non-NaN pattern as
    decompress + an fp32 product."""
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import quantize_and_compress
    from bitsparse_amd.src.hip_operators import unpack_relu2_batch_
    K, N, M = 192, 320, 256
    # ~38% of the columns hold no stored value: without the fix-up they
    # would come out 0 instead of NaN
    r = relu_input((K, N), 0.995, seed=12).to(dev)
    A = preact_input((M, K), seed=13).to(dev)
    _, _, sp = quantize_and_compress(r, None)
    sp.scale = torch.full_like(sp.scale, float("inf"))
    dense = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
    unpack_relu2_batch_(sp, dense, 0, sp.grid_n, N, K, sp.grid_m * sp.grid_n)
    assert torch.isnan(dense).any() and (~torch.isnan(dense)).any()
    ref = A.float() @ dense.float()
    C = dw_gemm.gemm_compressed_b(A, sp, square=True)
    assert torch.equal(torch.isnan(C), torch.isnan(ref))
    assert torch.equal(torch.isinf(C), torch.isinf(ref))


def test_gemm_empty_k_under_graph_capture(dev):
    """K = 0 (an empty compressed operand): C = 0, written by a kernel, so
    the call captures into a HIP graph; every replay rewrites the zeros."""
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse
    M, N = 96, 130
    sp = dense_to_tilesparse(torch.zeros((0, N), dtype=torch.bfloat16, device=dev), None)
    A = torch.empty((M, 0), dtype=torch.bfloat16, device=dev)
    C = dw_gemm.gemm_compressed_b(A, sp, square=False)
    assert C.shape == (M, N) and bool((C == 0).all())
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dw_gemm.gemm_compressed_b(A, sp, square=False)          # warm-up off the graph
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        out = dw_gemm.gemm_compressed_b(A, sp, square=False)
    for _ in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bool((out == 0).all())
