"""Reference behaviours a drop-in caller relies on.

* fp8 activation storage given as float8_e5m2: the reference layers quantize
  with to_fp8, which always yields e4m3fn codes + scale
  (lib_sparse/layers.py:32-35, :112-115; fp8.py:123-129), so dtype=e5m2
  (ReluLinear / FFNRelu) and storage_dtype=e5m2 (Relu2Linear / FFNRelu2)
  behave exactly as e4m3fn: same outputs and gradients bit for bit.
* the TensorBuffer cursor advanced in place (lib_sparse/src/functions.py:80-94:
  the compress snapshots ``offset.clone()`` and ends with ``offset.copy_``),
  offered by TensorBuffer(..., inplace_offset=True): ``buf.offset`` keeps its
  identity across compresses, each BitsparseTensor keeps its own snapshot,
  and every result equals the default (rebinding) buffer's.
"""
import pytest
import torch

from tests.helpers import relu_input

pytestmark = pytest.mark.gpu


def _inputs(dev, B=256, D=128, H=512, seed=3, shift=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, D), generator=g).to(torch.bfloat16)
    W1 = (0.05 * torch.randn((H, D), generator=g) + shift).to(torch.bfloat16)
    W2 = (0.05 * torch.randn((D, H), generator=g)).to(torch.bfloat16)
    dY = torch.randn((B, D), generator=g).to(torch.bfloat16)
    return [t.to(dev) for t in (x, W1, W2, dY)]


def _step(fn, x, W1, W2, dY, **kw):
    xs, W1s, W2s = (t.clone().requires_grad_() for t in (x, W1, W2))
    y = fn(xs, W1s, W2s, **kw)
    y.backward(dY)
    return [t.view(torch.int16) for t in (y.detach(), xs.grad, W1s.grad, W2s.grad)]


@pytest.mark.parametrize("use_buffer", [False, True])
@pytest.mark.parametrize("relu2", [False, True])
def test_e5m2_storage_dtype_stores_e4m3fn(dev, use_buffer, relu2):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.layers import FFNRelu, FFNRelu2
    x, W1, W2, dY = _inputs(dev, shift=0.01 if relu2 else 0.0)
    key = "storage_dtype" if relu2 else "dtype"
    fn = FFNRelu2.apply if relu2 else FFNRelu.apply
    outs = []
    for dt in (torch.float8_e4m3fn, torch.float8_e5m2):
        buf = TensorBuffer(256 * 512, device=dev, dtype=torch.float8_e4m3fn) if use_buffer else None
        outs.append(_step(fn, x, W1, W2, dY, sparse_data=buf, **{key: dt}))
        if buf is not None:
            assert not buf.overflowed()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_e5m2_layer_saves_e4m3fn_codes(dev):
    """The compressed activation a dtype=e5m2 ReluLinear keeps is the e4m3fn
    to_fp8 form of relu(z)."""
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.layers import ReluLinear
    from bitsparse_amd.src.hip_operators import unpack_batch_
    x, W1, W2, _ = _inputs(dev)
    z = x @ W1.T
    h8, s = to_fp8(z.relu())
    captured = {}
    orig = ReluLinear.forward

    def spy(ctx, *a, **k):
        y = orig(ctx, *a, **k)
        captured["sp"] = ctx.h_sparse
        return y
    ReluLinear.forward = staticmethod(spy)
    try:
        ReluLinear.apply(z.clone().requires_grad_(), W2, None, False, torch.float8_e5m2)
    finally:
        ReluLinear.forward = staticmethod(orig)
    sp = captured["sp"]
    assert sp.dtype == torch.float8_e4m3fn and torch.equal(sp.scale, s)
    M, N = z.shape
    out = torch.empty((M, N), device=dev, dtype=torch.float8_e4m3fn)
    unpack_batch_(sp, out, 0, sp.grid_n, N, M, sp.grid_m * sp.grid_n)
    assert torch.equal(out.view(torch.uint8), h8.view(torch.uint8))


def _compress_seq(dev, buf, xs, kind):
    from bitsparse_amd.src.functions import dense_to_tilesparse, quantize_and_compress
    sps = []
    for x in xs:
        if kind == "e4m3fn":
            sps.append(quantize_and_compress(x.to(dev), buf, pack_sbit=buf.pack_sbit)[2])
        else:
            sps.append(dense_to_tilesparse(x.to(dev), None, buf, pack_sbit=buf.pack_sbit))
    return sps


@pytest.mark.parametrize("kind,pack", [("bf16", False), ("bf16", True), ("e4m3fn", False), ("e4m3fn", True)])
def test_inplace_offset_matches_rebinding_cursor(dev, kind, pack):
    from bitsparse_amd.bitsparse import TensorBuffer
    dt = torch.float8_e4m3fn if kind == "e4m3fn" else torch.bfloat16
    xs = [relu_input(s, 0.6, seed=20 + i) for i, s in enumerate([(129, 131), (64, 200), (300, 77)])]
    size = 300_000
    ref_buf = TensorBuffer(size, device=dev, dtype=dt, pack_sbit=pack)
    ref = _compress_seq(dev, ref_buf, xs, kind)
    buf = TensorBuffer(size, device=dev, dtype=dt, pack_sbit=pack, inplace_offset=True)
    held = buf.offset                                   # the tensor a caller holds
    got = _compress_seq(dev, buf, xs, kind)
    assert buf.offset is held
    assert int(held.item()) == int(ref_buf.offset.item())
    for a, b in zip(ref, got):
        assert int(a.vals_offset.item()) == int(b.vals_offset.item())   # each keeps its own snapshot
        assert b.vals_offset.data_ptr() != held.data_ptr()
        assert torch.equal(a.bitmask, b.bitmask) and torch.equal(a.prefix, b.prefix)
    assert torch.equal(ref_buf.vals.view(torch.uint8), buf.vals.view(torch.uint8))
    buf.reset_buffer()
    assert buf.offset is held and int(held.item()) == 0


@pytest.mark.parametrize("fused_up", [False, True])
def test_inplace_offset_in_layers(dev, monkeypatch, fused_up):
    """A layer step into an in-place buffer (library GEMM + compress, or the
    fused up-projection): same outputs and gradients as the default buffer,
    and the held cursor tensor ends at the activation's nonzeros."""
    from bitsparse_amd import layers
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.layers import FFNRelu
    monkeypatch.setattr(layers, "USE_FUSED_UP", fused_up)
    x, W1, W2, dY = _inputs(dev)
    ref_buf = TensorBuffer(2 * 256 * 512, device=dev)
    ref = _step(FFNRelu.apply, x, W1, W2, dY, sparse_data=ref_buf)
    buf = TensorBuffer(2 * 256 * 512, device=dev, inplace_offset=True)
    held = buf.offset
    got = _step(FFNRelu.apply, x, W1, W2, dY, sparse_data=buf)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)
    assert buf.offset is held and int(held.item()) == int(ref_buf.offset.item())
    if not fused_up:       # the fused GEMM's z may differ from the library's in the last bit
        assert int(held.item()) == int(((x @ W1.T) > 0).sum().item())
