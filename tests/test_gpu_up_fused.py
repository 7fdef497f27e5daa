"""Up-projection GEMM with the ReLU and the compress in its epilogue
(bs_linear_relu_compress), the fused form of reference lib_sparse/layers.py:86-89
(z = x @ W1^T; z = z + b1), :29 (h = z.relu_()) and :37 (dense_to_tilesparse).

Pinned two ways:
* the compressed form is bit-exact against the oracle's compress of the h the
  kernel wrote (same bitmask, prefix and values), at every shape, with NaN /
  Inf / -0 in the products, and at configs[1]'s full 8192 x 768 -> 3072;
* h against an fp32 product rounded as the reference rounds
  (relu(bf16(bf16(x @ W^T) + b))): the kernel's fp32 accumulation order is its
  own, so each element is within rtol 2^-7 (two bf16 roundings of a slightly
  different sum) plus atol 2^-8 * max|h| (sums that cancel to near zero).
"""
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, preact_input, special_bf16

pytestmark = pytest.mark.gpu


def _ops():
    import bitsparse_amd.src.hip_operators as H
    return H


def _operands(M, N, K, seed, dev, bias=True, scale=None):
    x = preact_input((M, K), seed=seed).to(dev)
    s = scale if scale is not None else K ** -0.5
    W = (preact_input((N, K), seed=seed + 1).float() * s).to(torch.bfloat16).to(dev)
    b = preact_input((N,), mu=-0.3, seed=seed + 2).to(dev) if bias else None
    return x, W, b


def _run(x, W, b, cap=None, offset=0):
    H = _ops()
    M, N = x.shape[0], W.shape[0]
    T = ((M + 63) // 64) * ((N + 63) // 64)
    dev = x.device
    h = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    bm = torch.empty(T * 512, device=dev, dtype=torch.uint8)
    pf = torch.empty(T + 1, device=dev, dtype=torch.uint32)
    vals = torch.zeros(cap if cap is not None else offset + M * N, device=dev, dtype=torch.bfloat16)
    off_in = torch.full((1,), offset, device=dev, dtype=torch.int64)
    off_out = torch.empty(1, device=dev, dtype=torch.int64)
    err = torch.zeros(1, device=dev, dtype=torch.int32)
    H.linear_relu_compress_into(x, W, b, h, bm, pf, vals, off_in, off_out, err)
    return h, bm, pf, vals, off_out, err


def _reference_h(x, W, b):
    z = (x.float() @ W.float().T).to(torch.bfloat16)
    if b is not None:
        z = (z.float() + b.float()).to(torch.bfloat16)
    return torch.relu(z)


def _check_compressed(h, bm, pf, vals, off_out, offset=0):
    obm, opf, ov = O.compress(bits(h), O.BF16)
    assert (bits(bm) == obm).all(), "bitmask"
    assert (bits(pf) == opf).all(), "prefix"
    got = bits(vals)[offset:offset + ov.size]
    assert (got == ov).all(), "vals"
    assert int(off_out.item()) == offset + ov.size


def _check_h(h, x, W, b):
    ref = _reference_h(x, W, b).float()
    fin = ref[torch.isfinite(ref)]
    atol = 2 ** -8 * ((fin.abs().max().item() if fin.numel() else 0.0) + 1e-30)
    torch.testing.assert_close(h.float(), ref, rtol=2 ** -7, atol=atol, equal_nan=True)


# (M, N, K): whole and partial 128 x 192 workgroup tiles, partial 64 x 64
# format tiles, K not a multiple of the 64-deep step, one-tile matrices, and
# right-edge units of one, two (N = 320, 128) or three format tiles (each
# unit's rounds split between two waves)
SHAPES = [(256, 192, 64), (300, 200, 72), (64, 8, 8), (1000, 768, 256), (513, 392, 40), (40, 1000, 128),
          (2048, 3072, 96), (200, 320, 48), (130, 128, 64)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("bias", [True, False])
def test_compressed_form_is_that_of_h(dev, shape, bias):
    M, N, K = shape
    x, W, b = _operands(M, N, K, 3, dev, bias)
    h, bm, pf, vals, off_out, err = _run(x, W, b)
    assert int(err.item()) == 0
    _check_compressed(h, bm, pf, vals, off_out)
    _check_h(h, x, W, b)


def test_special_values(dev):
    """NaN / Inf / -0 / denormals in x: torch's relu keeps NaN in h, the
    bitmask excludes it; -0 and negatives become +0."""
    M, N, K = 320, 384, 64
    x = special_bf16((M, K), seed=4).to(dev)
    _, W, b = _operands(M, N, K, 5, dev)
    h, bm, pf, vals, off_out, err = _run(x, W, b)
    _check_compressed(h, bm, pf, vals, off_out)
    _check_h(h, x, W, b)
    hb = bits(h)
    assert not ((hb >= 0x8000) & (hb <= 0xff80)).any(), "relu leaves no negative or -0 bits"


def test_cursor_capacity_and_offset(dev):
    """Values land at the cursor; the next cursor is start + nnz; values past
    the capacity are not written and flag bit 0."""
    M, N, K = 512, 384, 64
    x, W, b = _operands(M, N, K, 6, dev)
    h, bm, pf, vals, off_out, err = _run(x, W, b, offset=37)
    _check_compressed(h, bm, pf, vals, off_out, offset=37)
    assert (bits(vals)[:37] == 0).all()
    nnz = int(off_out.item()) - 37
    cap = 37 + nnz // 2
    h2, bm2, pf2, vals2, off2, err2 = _run(x, W, b, cap=cap, offset=37)
    assert int(err2.item()) & 1
    assert int(off2.item()) == 37 + nnz
    _, _, ov = O.compress(bits(h2), O.BF16)
    assert (bits(vals2)[37:cap] == ov[:cap - 37]).all()


def test_shared_buffer_two_activations(dev):
    """Two fused compresses into one TensorBuffer, then both decompress."""
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src import functions as F
    H = _ops()
    buf = TensorBuffer(2 * 320 * 392, device=dev)
    outs = []
    for seed in (7, 9):
        x, W, b = _operands(320, 392, 64, seed, dev)
        h, sp = F.linear_relu_and_compress(x, W, b, buf)
        outs.append((h.clone(), sp))
    assert not buf.overflowed()
    for h, sp in outs:
        d = torch.empty_like(h)
        H.unpack_batch_(sp, d, 0, sp.grid_n, h.shape[1], h.shape[0], sp.grid_m * sp.grid_n)
        assert torch.equal(d.view(torch.int16), torch.where(h > 0, h, torch.zeros_like(h)).view(torch.int16))


def test_configs1_full_size(dev):
    """configs[1]'s up-projection: x 8192 x 768, W1 3072 x 768 N(0, 0.02), b1."""
    M, N, K = 8192, 3072, 768
    x, W, b = _operands(M, N, K, 11, dev, scale=0.02)
    h, bm, pf, vals, off_out, err = _run(x, W, b)
    assert int(err.item()) == 0
    _check_compressed(h, bm, pf, vals, off_out)
    _check_h(h, x, W, b)
    zeros = 1.0 - int(off_out.item()) / (M * N)
    assert 0.3 < zeros < 0.7


@pytest.mark.parametrize("square", [False, True])
def test_layers_take_the_fused_path(dev, monkeypatch, square):
    """FFNRelu / FFNRelu2 (bf16, TensorBuffer) run the fused kernel and agree
    with the library-GEMM path: y and the gradients within bf16 tolerance
    (z differs in the last bit of some elements, so a few bitmask bits near
    zero may too)."""
    from bitsparse_amd import layers
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src import functions as F
    calls = []
    real = F.linear_relu_and_compress
    monkeypatch.setattr(layers, "linear_relu_and_compress", lambda *a: calls.append(1) or real(*a))
    M, D, FF = 512, 256, 768
    x0 = preact_input((M, D), seed=12).to(dev)
    W1 = (preact_input((FF, D), seed=13).float() * 0.05).to(torch.bfloat16).to(dev)
    W2 = (preact_input((D, FF), seed=14).float() * 0.05).to(torch.bfloat16).to(dev)
    b1 = (preact_input((FF,), seed=15).float() * 0.1).to(torch.bfloat16).to(dev)
    dy = preact_input((M, D), seed=16).to(dev)
    fn = layers.FFNRelu2 if square else layers.FFNRelu
    res = []
    for fused in (True, False):
        monkeypatch.setattr(layers, "USE_FUSED_UP", fused)
        x = x0.clone().requires_grad_(True)
        p = [t.clone().requires_grad_(True) for t in (W1, W2, b1)]
        buf = TensorBuffer(M * FF, device=dev)
        y = fn.apply(x, p[0], p[1], p[2], sparse_data=buf)
        y.backward(dy)
        res.append([y.detach(), x.grad, p[0].grad, p[1].grad, p[2].grad])
    assert len(calls) == 1
    for got, want in zip(*res):
        tol = 2 ** -6 * want.float().abs().max().item()
        torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -6, atol=tol)


def test_unsupported_operands_are_refused(dev):
    """K or N not a multiple of 8 is refused by the entry point (the layers
    then keep the library path)."""
    H = _ops()
    x, W, b = _operands(64, 100, 12, 17, dev)
    assert not H.linear_relu_compress_supported(x, W, b)
    with pytest.raises(ValueError, match="multiples of 8"):
        _run(x, W, b)


def test_forced_lookback_timeout_sets_its_own_flag(dev, monkeypatch):
    """Patience 0 makes every unit but the first give up without waiting (the
    host forces the time-out; every wave still ends normally): the time-out
    word is set and the capacity flags stay clear."""
    H = _ops()
    monkeypatch.setattr(H, "UP_LOOKBACK_PATIENCE_TICKS", 0)
    x, W, b = _operands(512, 768, 64, 21, dev)          # 4 strips x 4 workgroups x 2 units
    M, N = x.shape[0], W.shape[0]
    T = (M // 64) * (N // 64)
    h = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    bm = torch.empty(T * 512, device=dev, dtype=torch.uint8)
    pf = torch.empty(T + 1, device=dev, dtype=torch.uint32)
    vals = torch.zeros(M * N, device=dev, dtype=torch.bfloat16)
    off_in = torch.zeros(1, device=dev, dtype=torch.int64)
    off_out = torch.empty(1, device=dev, dtype=torch.int64)
    err = torch.zeros(1, device=dev, dtype=torch.int32)
    timeout = torch.zeros(1, device=dev, dtype=torch.int32)
    H.linear_relu_compress_into(x, W, b, h, bm, pf, vals, off_in, off_out, err, timeout)
    torch.cuda.synchronize()
    assert int(timeout.item()) == 1
    assert int(err.item()) == 0
    # the default patience on the same operands: no time-out, exact result
    monkeypatch.setattr(H, "UP_LOOKBACK_PATIENCE_TICKS", -1)
    timeout.zero_()
    off_out.zero_()
    H.linear_relu_compress_into(x, W, b, h, bm, pf, vals, off_in, off_out, err, timeout)
    torch.cuda.synchronize()
    assert int(timeout.item()) == 0 and int(err.item()) == 0
    _check_compressed(h, bm, pf, vals, off_out)


@pytest.mark.parametrize("relu2", [False, True])
def test_layer_raises_on_lookback_timeout(dev, monkeypatch, relu2):
    """FFNRelu / FFNRelu2 through the fused up-projection refuse to use an
    activation whose look-back gave up: backward raises LookbackTimeout
    instead of computing gradients from a misplaced value run."""
    from bitsparse_amd import layers
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import LookbackTimeout
    H = _ops()
    monkeypatch.setattr(layers, "USE_FUSED_UP", True)
    monkeypatch.setattr(H, "UP_LOOKBACK_PATIENCE_TICKS", 0)
    x, W1, b1 = _operands(512, 768, 128, 22, dev)
    W2 = (0.05 * preact_input((128, 768), seed=23).float()).to(torch.bfloat16).to(dev).requires_grad_()
    W1 = W1.clone().requires_grad_()
    buf = TensorBuffer(2 * 512 * 768, device=dev)
    fn = layers.FFNRelu2 if relu2 else layers.FFNRelu
    y = fn.apply(x, W1, W2, b1, sparse_data=buf)
    with pytest.raises(LookbackTimeout):
        y.backward(torch.ones_like(y))
    assert not buf.overflowed()


def test_flag_ring_keeps_a_timeout_across_slot_reuse(dev, monkeypatch):
    """The layers' time-out flags are slots of a pinned host ring that the
    kernel stores into through its device address (no copy on the stream).
    A slot is reused after SLOTS launches: a check taken before that still
    reports its own launch's (forced) time-out, and the later launches'
    checks report none."""
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src import functions as F
    H = _ops()
    x, W, _ = _operands(256, 192, 64, 24, dev, bias=False)   # 4 units: every unit but the first gives up
    buf = TensorBuffer(2 * 256 * 192 + 64, device=dev)
    monkeypatch.setattr(H, "UP_LOOKBACK_PATIENCE_TICKS", 0)
    buf.reset_buffer()
    _, sp0 = F.linear_relu_and_compress(x, W, None, buf)
    monkeypatch.setattr(H, "UP_LOOKBACK_PATIENCE_TICKS", -1)
    checks = []
    for _ in range(F._FlagRing.SLOTS + 3):
        buf.reset_buffer()
        h, sp = F.linear_relu_and_compress(x, W, None, buf)
        checks.append(sp.lookback_check)
    assert sp0.lookback_check.timed_out()
    assert not any(c.timed_out() for c in checks)
    _check_compressed(h, sp.bitmask, sp.prefix, buf.vals, buf.offset)


def test_width_bound_from_occupancy(dev):
    """The widest N the fused kernel takes comes from the occupancy API (half
    of the workgroups the device holds, 192 columns each); wider is refused by
    the entry point and routed to the library path by the layers."""
    H = _ops()
    from bitsparse_amd import _lib
    from bitsparse_amd.src.functions import fused_linear_relu_ok
    from bitsparse_amd.bitsparse import TensorBuffer
    max_n = H.linear_relu_compress_max_n(dev)
    props = torch.cuda.get_device_properties(dev)
    assert max_n > 0 and max_n % 192 == 0
    assert max_n <= 192 * props.multi_processor_count      # half of two workgroups per CU
    assert int(_lib.load().bs_linear_relu_compress_max_n(dev.index or 0)) == max_n
    x, W, b = _operands(64, max_n + 192, 16, 24, dev, bias=False)
    assert not H.linear_relu_compress_supported(x, W, b)
    assert not fused_linear_relu_ok(x, W, b, TensorBuffer(2 * 64 * (max_n + 192), device=dev))
    with pytest.raises(ValueError, match="at most"):
        _run(x, W, b)
