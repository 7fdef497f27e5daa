"""Fused ReLU + compress (bs_compress_relu / bs_amax_relu) against the
unfused reference sequence h = z.relu_(); compress(h) (lib_sparse/layers.py:29,37
and :107,117).

Bar: bit-exact.  relu(z) written back into z equals torch.relu(z) on the GPU bit
for bit (x <= 0 -> +0, -0 included; NaN payloads kept), and every compress
output (bitmask, prefix, values or packed stream, fp8 scale and quantized
copy) equals the unfused path on the same inputs, which test_gpu_codec pins
against the oracle; inputs are salted with +-0, +-denormals, +-Inf and NaNs.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, from_bits, preact_input, special_bf16

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (64, 64), (129, 131), (200, 70), (320, 1024)]


def _same(a, b):
    return np.array_equal(bits(a), bits(b))


def _z(shape, seed):
    z = preact_input(shape, -0.3, seed)
    s = special_bf16(shape, seed + 100)
    keep = torch.rand(shape, generator=torch.Generator().manual_seed(seed)) < 0.7
    return torch.where(keep, z, s)


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("mode", ["standalone", "buffer", "packed"])
def test_relu_and_compress_equals_relu_then_compress(dev, shape, mode):
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.bitsparse import TensorBuffer
    z = _z(shape, 1).to(dev)
    pack = mode == "packed"

    def buf():
        return None if mode == "standalone" else TensorBuffer(4 * shape[0] * shape[1] + 64, device=dev,
                                                              pack_sbit=pack)
    h_ref = torch.relu(z.clone())
    sp_ref = F.dense_to_tilesparse(h_ref, None, buf(), pack_sbit=pack)
    zf = z.clone()
    h, sp = F.relu_and_compress(zf, buf(), pack_sbit=pack)
    assert h.data_ptr() == zf.data_ptr()                 # in place, like z.relu_()
    assert _same(zf, h_ref)
    assert _same(sp.bitmask, sp_ref.bitmask) and _same(sp.prefix, sp_ref.prefix)
    nnz = int(sp.prefix[-1].item())
    if pack:
        nb = (nnz * 15 + 7) // 8
        assert _same(sp.vals[:nb], sp_ref.vals[:nb])
    else:
        o1, o2 = int(sp.vals_offset.reshape(-1)[0]), int(sp_ref.vals_offset.reshape(-1)[0])
        assert _same(sp.vals[o1:o1 + nnz], sp_ref.vals[o2:o2 + nnz])
    # and against the oracle on relu(z) computed by torch on the CPU
    bm, pf, v = O.compress(bits(torch.relu(z.cpu())), O.BF16)
    assert (bits(sp.bitmask) == bm).all() and (bits(sp.prefix) == pf).all()


@pytest.mark.parametrize("shape", [(64, 64), (129, 131), (256, 1024)])
@pytest.mark.parametrize("use_buffer", [False, True])
def test_relu_quantize_and_compress_equals_unfused(dev, shape, use_buffer):
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.bitsparse import TensorBuffer
    z = preact_input(shape, -0.5, 2).to(dev)             # finite inputs: a NaN would make the scale NaN

    def buf():
        return TensorBuffer(shape[0] * shape[1], device=dev, dtype=torch.float8_e4m3fn) if use_buffer else None
    q_ref, s_ref, sp_ref = F.quantize_and_compress(torch.relu(z.clone()), buf())
    zf = z.clone()
    q, s, sp = F.relu_quantize_and_compress(zf, buf())
    assert _same(zf, torch.relu(z))
    assert _same(s, s_ref) and _same(q, q_ref)
    assert _same(sp.bitmask, sp_ref.bitmask) and _same(sp.prefix, sp_ref.prefix)
    nnz = int(sp.prefix[-1].item())
    o1, o2 = int(sp.vals_offset.reshape(-1)[0]), int(sp_ref.vals_offset.reshape(-1)[0])
    assert _same(sp.vals[o1:o1 + nnz], sp_ref.vals[o2:o2 + nnz])


def test_amax_relu(dev):
    """scale of relu(z) from the fused amax == scale of torch.relu(z): the
    largest magnitude of z is negative, so plain amax(|z|) would differ."""
    import bitsparse_amd.src.hip_operators as H
    z = preact_input((300, 500), 0.0, 3)
    z[7, 11] = -100.0
    z = z.to(dev)
    e1 = H.amax_into_workspace(torch.relu(z))
    _, s1 = H.quantize_e4m3fn(torch.relu(z), e1)
    e2 = H.amax_into_workspace(z, relu=True)
    _, s2 = H.quantize_e4m3fn(torch.relu(z), e2)
    assert _same(s1, s2)
    e3 = H.amax_into_workspace(z)
    _, s3 = H.quantize_e4m3fn(z, e3)
    assert not _same(s1, s3)


@pytest.mark.parametrize("code", [O.E4M3FN, O.E5M2])
def test_relu_and_compress_fp8_input(dev, code):
    """fp8 pre-activations (torch has no fp8 relu on the GPU): the bf16 rule on
    fp8 bit patterns, x <= 0 -> +0 (e4m3fn 0x80..0xfe, e5m2 0x80..0xfc), NaN
    and positives keep their bits."""
    import bitsparse_amd.src.functions as F
    dt = torch.float8_e4m3fn if code == O.E4M3FN else torch.float8_e5m2
    raw = np.random.default_rng(code).integers(0, 256, (129, 200)).astype(np.uint8)
    last = 0xFE if code == O.E4M3FN else 0xFC
    want = np.where((raw >= 0x80) & (raw <= last), 0, raw).astype(np.uint8)
    z = from_bits(raw, dt).to(dev)
    h, sp = F.relu_and_compress(z)
    assert (bits(h) == want).all()
    bm, pf, v = O.compress(want, code)
    assert (bits(sp.bitmask) == bm).all() and (bits(sp.prefix) == pf).all()
    assert (bits(sp.vals) == v).all()
