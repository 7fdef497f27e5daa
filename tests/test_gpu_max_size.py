"""Inputs past 2^31 elements: the codec and the dW GEMM index HBM with 64-bit
offsets and a uint32 prefix.  These shapes check that every element offset
and every prefix value above 2^31 is carried without wrapping.

Regression: compress once broadcast the unit's exclusive prefix (a uint32)
through __builtin_amdgcn_readfirstlane, whose int result was widened to
int64 with sign extension, so every unit whose prefix had passed 2^31 stored
its values up to 8 GiB before the value buffer and faulted the GPU.  The
broadcast now widens the unsigned value (uniform_u32).  The oracle is far too
slow at this size, so the checks are size-independent properties computed
with torch ops on the GPU: the exact round trip, the bitmask and prefix
rebuilt from the dense input, the tile-major value order, and the GEMM
against an fp32 product on the decompressed operand.

Shape 32768 x 65600 = 2,149,580,800 elements (2^31 + 2,097,152); at mean +4
about 99.997% of the elements are positive, so the last prefix values (and the
value-stream offsets) also pass 2^31.
"""
import pytest
import torch

from tests.test_gpu_codec import _torch_tile_bitmask, decompress

pytestmark = pytest.mark.gpu

M_BIG, N_BIG = 32768, 65600


@pytest.fixture(scope="module")
def big_dev(dev):
    free, _ = torch.cuda.mem_get_info(dev)
    if free < 64 * 2 ** 30:
        pytest.skip("needs 64 GiB of free device memory")
    return dev


def test_codec_round_trip_past_2_31_elements(big_dev):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import dense_to_tilesparse
    M, N = M_BIG, N_BIG
    assert M * N > 2 ** 31
    g = torch.Generator(device=big_dev).manual_seed(11)
    x = torch.empty((M, N), dtype=torch.bfloat16, device=big_dev)
    for r in range(0, M, 4096):          # fp32 normal draws in slices, kept as bf16
        x[r:r + 4096] = torch.randn((4096, N), device=big_dev, generator=g) + 4.0
    x.relu_()
    buf = TensorBuffer(2 * M * N, device=big_dev)
    sp = dense_to_tilesparse(x, None, buf)
    torch.cuda.synchronize()
    counts = (x > 0).reshape(M // 64, 64, N // 64, 64).sum((1, 3), dtype=torch.int64).reshape(-1)
    pref = torch.zeros(counts.numel() + 1, dtype=torch.int64, device=big_dev)
    pref[1:] = counts.cumsum(0)
    nnz = int(pref[-1].item())
    assert nnz > 2 ** 31
    assert torch.equal(sp.prefix.to(torch.int64), pref)
    assert int(buf.offset.item()) == nnz
    assert torch.equal(sp.bitmask, _torch_tile_bitmask(x))
    del counts, pref
    # values in tile-major order, compared in row-block slices to bound memory
    done = 0
    for tm0 in range(0, M // 64, 64):
        blk = x[tm0 * 64:(tm0 + 64) * 64].reshape(64, 64, N // 64, 64).permute(0, 2, 1, 3).reshape(-1)
        blk = blk[blk > 0]
        assert torch.equal(sp.vals[done:done + blk.numel()], blk), f"values of tile rows {tm0}.."
        done += blk.numel()
        del blk
    assert done == nnz
    d = decompress(sp)
    assert torch.equal(d, x)


def test_gemm_compressed_operand_past_2_31_elements(big_dev):
    """K*N > 2^31 for the compressed operand of the dW GEMM (512-row shape)."""
    from bitsparse_amd.src import dw_gemm
    from bitsparse_amd.src.functions import dense_to_tilesparse
    K, N, M = M_BIG, N_BIG, 512
    g = torch.Generator(device=big_dev).manual_seed(12)
    h = torch.empty((K, N), dtype=torch.bfloat16, device=big_dev)
    for r in range(0, K, 4096):
        h[r:r + 4096] = torch.randn((4096, N), device=big_dev, generator=g)
    h.relu_()
    A = torch.randn((M, K), device=big_dev, generator=g).to(torch.bfloat16)
    sp = dense_to_tilesparse(h, None)
    assert dw_gemm.supports(A, sp, square=False)
    C = dw_gemm.gemm_compressed_b(A, sp, square=False)
    torch.cuda.synchronize()
    Af = A.float()
    for c0 in range(0, N, 8192):         # fp32 reference in column slices
        ref = Af @ h[:, c0:c0 + 8192].float()
        got = C[:, c0:c0 + 8192].float()
        scale = ref.abs().max().item() + 1e-6
        torch.testing.assert_close(got, ref, rtol=2 ** -7, atol=2 ** -7 * scale * 1e-2)
