"""GPU parity of the packed value stream (pack_sbit storage) against the CPU
oracle.

Bar: bit-exact.  Stream bytes equal the oracle's packing (``oracle.pack_bits``,
pinned in tests/test_oracle.py against hand-worked streams, a bit-by-bit
packer and the numpy formulation) of the oracle's compacted values, with the
bytes around a run untouched; decompressed tiles, the ReLU^2 unpack and the
ReLU^2 gradient from a packed stream equal the raw-storage results (pinned
against the oracle in tests/test_gpu_codec.py), since packing drops only the
sign bit, which is 0 for every stored (positive) value.  Reference behaviour
followed: lib_sparse/src/bitpacking.py, functions.py:76-92 (8-value aligned
cursor), triton_operators.py:36-115.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, from_bits, relu_input

pytestmark = pytest.mark.gpu

TORCH_DT = {O.BF16: torch.bfloat16, O.E4M3FN: torch.float8_e4m3fn, O.E5M2: torch.float8_e5m2}


def _np_dt(code):
    return np.uint16 if code == O.BF16 else np.uint8


def _call_pack(dev, raw_np, code, stream_np, start, count_dev=None, count_max=None, nbytes=None):
    from bitsparse_amd import _lib
    L = _lib.load()
    raw = from_bits(raw_np, TORCH_DT[code]).to(dev)
    stream = torch.from_numpy(stream_np.copy()).to(dev)
    start_t = torch.tensor([start], dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    n = raw_np.size if count_max is None else count_max
    rc = L.bs_pack_bits(raw.data_ptr(), code, count_dev.data_ptr() if count_dev is not None else None,
                        n, stream.data_ptr(), stream.numel() if nbytes is None else nbytes,
                        start_t.data_ptr(), err.data_ptr(), _lib.stream_handle(dev))
    assert rc == 0, L.bs_last_error()
    torch.cuda.synchronize()
    return stream.cpu().numpy(), int(err.item())


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN, O.E5M2])
@pytest.mark.parametrize("start", [0, 1, 5, 8, 31, 1000])
@pytest.mark.parametrize("n", [1, 7, 100, 5000])
def test_pack_bits_kernel_matches_oracle(dev, code, start, n):
    rng = np.random.default_rng(start * 7 + n + code)
    dt = _np_dt(code)
    raw = rng.integers(0, np.iinfo(dt).max + 1, n).astype(dt)      # sign bits set too
    b = O.bits_per_value(code)
    nbytes = (((start + n) * b + 7) // 8 + 11) // 4 * 4
    init = rng.integers(0, 256, nbytes).astype(np.uint8)
    got, err = _call_pack(dev, raw, code, init, start)
    want = O.pack_bits(raw, code, init.copy(), start)
    assert err == 0
    assert (got == want).all()


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
@pytest.mark.parametrize("start", [0, 8, 16 * 1024 + 8])
def test_pack_bits_aligned_large(dev, code, start):
    """8-aligned starts take the staged-group path: several workgroups and
    grid-stride iterations, partial last group, stale bytes around the run."""
    rng = np.random.default_rng(start + code)
    dt = _np_dt(code)
    b = O.bits_per_value(code)
    for n in (8 * 256 * 3 + 5, 100_003):
        raw = rng.integers(0, np.iinfo(dt).max + 1, n).astype(dt)
        nbytes = (((start + n) * b + 7) // 8 + 11) // 4 * 4
        init = rng.integers(0, 256, nbytes).astype(np.uint8)
        got, err = _call_pack(dev, raw, code, init, start)
        assert err == 0
        assert (got == O.pack_bits(raw, code, init.copy(), start)).all()


def test_pack_bits_unaligned_raw(dev):
    """Raw values not aligned for 16-byte loads take the per-dword path."""
    from bitsparse_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(21)
    raw = rng.integers(0, 1 << 16, 5001).astype(np.uint16)
    t = from_bits(raw, torch.bfloat16).to(dev)
    init = rng.integers(0, 256, 4 * ((5000 * 15 // 8 + 16) // 4)).astype(np.uint8)
    stream = torch.from_numpy(init.copy()).to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = L.bs_pack_bits(t.data_ptr() + 2, O.BF16, None, 5000, stream.data_ptr(), stream.numel(), None,
                        err.data_ptr(), _lib.stream_handle(dev))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert (stream.cpu().numpy() == O.pack_bits(raw[1:], O.BF16, init.copy(), 0)).all()


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
def test_pack_bits_device_count_and_capacity(dev, code):
    rng = np.random.default_rng(3)
    dt = _np_dt(code)
    b = O.bits_per_value(code)
    raw = rng.integers(0, np.iinfo(dt).max + 1, 300).astype(dt)
    init = rng.integers(0, 256, 1024).astype(np.uint8)
    # the count comes from a device uint32 below the launch bound
    cnt = torch.tensor([123], dtype=torch.int32, device=dev).view(torch.uint32)
    got, err = _call_pack(dev, raw, code, init, 3, count_dev=cnt, count_max=300)
    assert err == 0
    assert (got == O.pack_bits(raw[:123], code, init.copy(), 3)).all()
    # storage of 64 bytes (16 words): words past it are neither written nor read
    got, err = _call_pack(dev, raw, code, init, 0, nbytes=64)
    assert err & 1
    assert (got[64:] == init[64:]).all()
    full = O.pack_bits(raw, code, init.copy(), 0)
    assert (got[:64] == full[:64]).all()


def _dense(sp):
    import bitsparse_amd.src.hip_operators as H
    M, N = sp.shape
    out = torch.empty((M, N), device=sp.vals.device, dtype=sp.dtype)
    return H.unpack_batch_(sp, out, 0, sp.grid_n, N, M, sp.grid_m * sp.grid_n)


@pytest.mark.parametrize("shape", [(1, 1), (64, 64), (129, 131), (200, 70), (320, 1024)])
@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN, O.E5M2])
def test_compress_packed_standalone(dev, shape, code):
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.src.bitpacking import packed_storage_nbytes
    x = relu_input(shape, 0.5, seed=4, dtype=TORCH_DT[code])
    sp = F.dense_to_tilesparse(x.to(dev), None, pack_sbit=True)
    bm, pf, v = O.compress(bits(x), code)
    assert sp.pack_sbit and sp.vals.dtype == torch.uint8 and sp.dtype == x.dtype
    assert (bits(sp.bitmask) == bm).all() and (bits(sp.prefix) == pf).all()
    b = O.bits_per_value(code)
    assert sp.vals.numel() == packed_storage_nbytes(v.size, b)
    stream = sp.vals.cpu().numpy()
    want = O.pack_bits(v, code, stream.copy(), 0)      # bytes outside the run: whatever is there
    assert (stream[:(v.size * b + 7) // 8] == want[:(v.size * b + 7) // 8]).all()
    assert torch.equal(_dense(sp).cpu().view(torch.uint8 if code else torch.int16),
                       x.view(torch.uint8 if code else torch.int16))


def test_compress_packed_tensorbuffer_sequence(dev):
    """Three activations in one packed TensorBuffer: each starts at the
    previous end rounded up to 8 values, the stream equals the oracle's packing
    of every run at its offset, and each decompresses to its input."""
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.bitsparse import TensorBuffer
    shapes = [(129, 131), (64, 200), (300, 77)]
    xs = [relu_input(s, 0.6, seed=10 + i) for i, s in enumerate(shapes)]
    buf = TensorBuffer(200_000, device=dev, pack_sbit=True)
    buf.vals.fill_(0xA5)                                # stale content of an earlier step
    sps = [F.dense_to_tilesparse(x.to(dev), None, buf, pack_sbit=True) for x in xs]
    stream_want = np.full(buf.vals.numel(), 0xA5, np.uint8)
    end = 0
    for x, sp in zip(xs, sps):
        off = int(sp.vals_offset.item())
        assert off == (end + 7) // 8 * 8
        _, _, v = O.compress(bits(x), O.BF16)
        O.pack_bits(v, O.BF16, stream_want, off)
        end = off + v.size
        assert torch.equal(_dense(sp).cpu(), x)
    assert int(buf.offset.item()) == end
    assert (buf.vals.cpu().numpy() == stream_want).all()
    assert not buf.overflowed()


def test_packed_tensorbuffer_overflow_flag(dev):
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.bitsparse import TensorBuffer
    x = relu_input((256, 256), 0.0, seed=5)
    buf = TensorBuffer(1000, device=dev, pack_sbit=True)
    F.dense_to_tilesparse(x.to(dev), None, buf, pack_sbit=True)
    assert buf.overflowed()


def test_relu2_unpack_and_grad_packed_equal_raw(dev):
    import bitsparse_amd.src.functions as F
    import bitsparse_amd.src.hip_operators as H
    from bitsparse_amd.bitsparse import TensorBuffer
    x = relu_input((200, 300), 0.5, seed=6)
    g = torch.randn((200, 300), generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(dev)
    for fp8 in (False, True):
        if fp8:
            _, _, raw = F.quantize_and_compress(x.to(dev))
            _, _, pk = F.quantize_and_compress(x.to(dev), TensorBuffer(100_000, device=dev, dtype=torch.float8_e4m3fn,
                                                                        pack_sbit=True), pack_sbit=True)
            assert torch.equal(raw.scale, pk.scale)
        else:
            raw = F.dense_to_tilesparse(x.to(dev), None)
            pk = F.dense_to_tilesparse(x.to(dev), None, pack_sbit=True)
        M, N = raw.shape
        o1 = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
        o2 = torch.empty_like(o1)
        H.unpack_relu2_batch_(raw, o1, 0, raw.grid_n, N, M, raw.grid_m * raw.grid_n)
        H.unpack_relu2_batch_(pk, o2, 0, pk.grid_n, N, M, pk.grid_m * pk.grid_n)
        assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
        g1 = H.relu2_grad_sparse_(g.clone(), raw)
        g2 = H.relu2_grad_sparse_(g.clone(), pk)
        assert torch.equal(g1.view(torch.int16), g2.view(torch.int16))


def test_unpack_row_batches_packed(dev):
    import bitsparse_amd.src.functions as F
    import bitsparse_amd.src.hip_operators as H
    x = relu_input((320, 200), 0.5, seed=8)
    pk = F.dense_to_tilesparse(x.to(dev), None, pack_sbit=True)
    gn = pk.grid_n
    for first, rows in ((0, 64), (1, 128), (3, 320 - 192)):
        out = torch.empty((rows, 200), device=dev, dtype=torch.bfloat16)
        H.unpack_batch_(pk, out, first, gn, 200, rows, ((rows + 63) // 64) * gn)
        assert torch.equal(out.cpu(), x[first * 64:first * 64 + rows])


@pytest.mark.parametrize("use_buffer", [False, True])
def test_ffn_relu_pack_sbit_equals_raw(dev, use_buffer):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.layers import FFNRelu
    g = torch.Generator().manual_seed(9)
    x = torch.randn((256, 128), generator=g).to(torch.bfloat16)
    W1 = (0.05 * torch.randn((512, 128), generator=g)).to(torch.bfloat16)
    W2 = (0.05 * torch.randn((128, 512), generator=g)).to(torch.bfloat16)
    dY = torch.randn((256, 128), generator=g).to(torch.bfloat16)
    res = []
    for pack in (False, True):
        buf = TensorBuffer(2 * 256 * 512, device=dev, pack_sbit=pack) if use_buffer else None
        xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
        y = FFNRelu.apply(xs, W1s, W2s, sparse_data=buf, pack_sbit=pack)
        y.backward(dY.to(dev))
        res.append((y, xs.grad, W1s.grad, W2s.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_ffn_relu2_fp8_pack_sbit_equals_raw(dev):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.layers import FFNRelu2
    g = torch.Generator().manual_seed(11)
    x = torch.randn((256, 128), generator=g).to(torch.bfloat16)
    W1 = (0.05 * torch.randn((512, 128), generator=g)).to(torch.bfloat16)
    W2 = (0.05 * torch.randn((128, 512), generator=g)).to(torch.bfloat16)
    dY = torch.randn((256, 128), generator=g).to(torch.bfloat16)
    res = []
    for pack in (False, True):
        buf = TensorBuffer(256 * 512, device=dev, dtype=torch.float8_e4m3fn, pack_sbit=pack)
        xs, W1s, W2s = (t.to(dev).requires_grad_() for t in (x, W1, W2))
        y = FFNRelu2.apply(xs, W1s, W2s, sparse_data=buf, pack_sbit=pack,
                           storage_dtype=torch.float8_e4m3fn)
        y.backward(dY.to(dev))
        res.append((y, xs.grad, W1s.grad, W2s.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def _call_compress_packed(dev, x, stream_np, start, nbytes=None, relu=False):
    """bs_compress_packed through the C ABI: (bitmask, prefix, stream bytes,
    aligned start, end cursor, err flags) on the CPU."""
    from bitsparse_amd import _lib
    from bitsparse_amd.src.hip_operators import dtype_code
    L = _lib.load()
    M, N = x.shape
    T = ((M + 63) // 64) * ((N + 63) // 64)
    xd = x.to(dev).contiguous()
    bm = torch.empty(T * 512, dtype=torch.uint8, device=dev)
    pf = torch.empty(T + 1, dtype=torch.uint32, device=dev)
    stream = torch.from_numpy(stream_np.copy()).to(dev)
    off_in = torch.tensor([start], dtype=torch.int64, device=dev)
    off_out = torch.full((1,), -7, dtype=torch.int64, device=dev)
    start_out = torch.full((1,), -7, dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = _lib.workspace_for(xd.device)
    ws.ensure(L.bs_compress_workspace_bytes(M, N))
    rc = L.bs_compress_packed(xd.data_ptr(), dtype_code(x.dtype), M, N, 0, None, 0, None, None,
                              bm.data_ptr(), pf.data_ptr(), stream.data_ptr(),
                              stream.numel() if nbytes is None else nbytes, off_in.data_ptr(),
                              off_out.data_ptr(), start_out.data_ptr(), err.data_ptr(),
                              ws.buf.data_ptr(), ws.nbytes, ws.next_epoch(), int(relu),
                              xd.data_ptr() if relu else None, _lib.stream_handle(dev))
    assert rc == 0, L.bs_last_error()
    torch.cuda.synchronize()
    return (bits(bm), bits(pf), stream.cpu().numpy(), int(start_out.item()), int(off_out.item()),
            int(err.item()), xd.cpu())


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN, O.E5M2])
@pytest.mark.parametrize("shape,sparsity", [((64, 64), 0.5), ((129, 131), 0.3), ((200, 70), 0.9),
                                            ((128, 1024), 0.0), ((77, 256), 1.0), ((1, 9), 0.2)])
@pytest.mark.parametrize("start", [0, 5, 8, 1003])
def test_fused_packed_compress_matches_oracle(dev, code, shape, sparsity, start):
    """One pass writes the packed stream: bytes equal the oracle's packing of
    the oracle's compacted values at the cursor rounded up to 8 values, every
    other stream byte keeps its (random) content."""
    x = relu_input(shape, sparsity, seed=sum(shape) + start + code, dtype=TORCH_DT[code])
    bm_w, pf_w, v = O.compress(bits(x), code)
    b = O.bits_per_value(code)
    a0 = (start + 7) // 8 * 8
    nbytes = ((a0 + v.size) * b + 7) // 8 // 4 * 4 + 16
    rng = np.random.default_rng(start + code)
    init = rng.integers(0, 256, nbytes).astype(np.uint8)
    bm, pf, got, s0, end, err, _ = _call_compress_packed(dev, x, init, start)
    want = O.pack_bits(v, code, init.copy(), a0)
    assert (bm == bm_w).all() and (pf == pf_w).all()
    assert (s0, end, err) == (a0, a0 + v.size, 0)
    assert (got == want).all()


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
def test_fused_packed_compress_large_matches_oracle(dev, code):
    """Many look-back units and every pass of the stream phase (whole-stream
    comparison at 1024 x 2048, unaligned cursor)."""
    x = relu_input((1024, 2048), 0.5, seed=31, dtype=TORCH_DT[code])
    _, _, v = O.compress(bits(x), code)
    b = O.bits_per_value(code)
    start = 13
    a0 = 16
    nbytes = ((a0 + v.size) * b + 7) // 8 // 4 * 4 + 8
    init = np.full(nbytes, 0x5A, np.uint8)
    _, _, got, s0, end, err, _ = _call_compress_packed(dev, x, init, start)
    want = O.pack_bits(v, code, init.copy(), a0)
    assert (s0, end, err) == (a0, a0 + v.size, 0)
    assert (got == want).all()


def test_fused_packed_compress_relu(dev):
    """Fused ReLU: the stream is that of relu(z) and z receives relu(z)."""
    from tests.helpers import preact_input
    z = preact_input((192, 320), 0.0, seed=8)
    h = torch.relu(z)
    _, _, v = O.compress(bits(h), O.BF16)
    nbytes = ((8 + v.size) * 15 + 7) // 8 // 4 * 4 + 8
    init = np.zeros(nbytes, np.uint8)
    _, _, got, s0, end, err, zout = _call_compress_packed(dev, z, init, 3, relu=True)
    assert (s0, end, err) == (8, 8 + v.size, 0)
    assert (got == O.pack_bits(v, O.BF16, init.copy(), 8)).all()
    assert torch.equal(zout.view(torch.int16), h.view(torch.int16))


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
def test_fused_packed_compress_capacity(dev, code):
    """A stream declared too small: bit 0 of the error flags is set, the
    dwords inside the declared size hold the oracle's bits and nothing past
    it is written."""
    x = relu_input((256, 256), 0.2, seed=12, dtype=TORCH_DT[code])
    _, _, v = O.compress(bits(x), code)
    b = O.bits_per_value(code)
    full = (v.size * b + 7) // 8 // 4 * 4 + 8
    declared = (full // 2) // 4 * 4
    init = np.random.default_rng(3).integers(0, 256, full).astype(np.uint8)
    _, _, got, s0, end, err, _ = _call_compress_packed(dev, x, init, 0, nbytes=declared)
    want = O.pack_bits(v, code, init.copy(), 0)
    assert err & 1 and end == v.size
    assert (got[:declared] == want[:declared]).all()
    assert (got[declared:] == init[declared:]).all()


def _tile_count_matrix(M, N, counts, code, seed):
    """[M, N] matrix (bits) whose tile t holds exactly counts[t] positive
    values at random positions."""
    rng = np.random.default_rng(seed)
    dt = _np_dt(code)
    x = np.zeros((M, N), dt)
    gn = N // 64
    one = {O.BF16: 0x3f80, O.E4M3FN: 0x38, O.E5M2: 0x3c}[code]
    for t, c in enumerate(counts):
        r0, c0 = (t // gn) * 64, (t % gn) * 64
        pos = rng.choice(4096, size=int(c), replace=False)
        x[r0 + pos // 64, c0 + pos % 64] = one + rng.integers(0, 8, size=int(c)).astype(dt)
    return x


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
@pytest.mark.parametrize("kind", ["tiny_runs", "aligned_runs"])
@pytest.mark.parametrize("start", [0, 3, 8, 21])
def test_fused_packed_compress_run_boundaries(dev, code, kind, start):
    """Tile runs of 0..3 values (several run boundaries inside one stream
    dword, empty runs) and runs of exactly 32 values (every boundary on a
    dword edge when the cursor is): stream equal to the oracle's packing."""
    M, N = 256, 1024                         # 64 tiles = 8 compress units
    rng = np.random.default_rng(start + 7 * code)
    counts = rng.integers(0, 4, 64) if kind == "tiny_runs" else np.full(64, 32)
    xb = _tile_count_matrix(M, N, counts, code, seed=start)
    x = from_bits(xb, TORCH_DT[code])
    _, _, v = O.compress(xb, code)
    assert v.size == counts.sum()
    b = O.bits_per_value(code)
    a0 = (start + 7) // 8 * 8
    nbytes = ((a0 + v.size) * b + 7) // 8 // 4 * 4 + 16
    init = np.random.default_rng(99).integers(0, 256, nbytes).astype(np.uint8)
    _, _, got, s0, end, err, _ = _call_compress_packed(dev, x, init, start)
    assert (s0, end, err) == (a0, a0 + v.size, 0)
    assert (got == O.pack_bits(v, code, init.copy(), a0)).all()


@pytest.mark.parametrize("shape", [(0, 64), (64, 0)])
def test_packed_tensorbuffer_empty_input_rounds_cursor(dev, shape):
    """An empty activation into a packed TensorBuffer takes no values but
    still rounds the cursor up to 8 values (functions.py:78-92): the next
    activation starts there, and the stream is untouched."""
    import bitsparse_amd.src.functions as F
    from bitsparse_amd.bitsparse import TensorBuffer
    buf = TensorBuffer(16384, device=dev, pack_sbit=True)
    buf.vals.fill_(0x3C)
    buf.offset = torch.tensor([5], dtype=torch.int64, device=dev)
    sp = F.dense_to_tilesparse(torch.zeros(shape, dtype=torch.bfloat16, device=dev), None, buf,
                               pack_sbit=True)
    assert int(sp.vals_offset.item()) == 8 and int(buf.offset.item()) == 8
    assert sp.nnz() == 0 and bits(sp.prefix).tolist() == [0]
    x = relu_input((64, 96), 0.5, seed=2)
    sp2 = F.dense_to_tilesparse(x.to(dev), None, buf, pack_sbit=True)
    _, _, v = O.compress(bits(x), O.BF16)
    assert int(sp2.vals_offset.item()) == 8 and int(buf.offset.item()) == 8 + v.size
    want = O.pack_bits(v, O.BF16, np.full(buf.vals.numel(), 0x3C, np.uint8), 8)
    assert (buf.vals.cpu().numpy() == want).all()
    assert torch.equal(_dense(sp2).cpu(), x)
    assert not buf.overflowed()


def test_fused_packed_compress_cursor_past_stream(dev):
    """A cursor far past the end of the stream (2^36 values): nothing is
    written, bit 0 of the error flags is set and the cursor still advances."""
    x = relu_input((128, 192), 0.5, seed=21)
    _, _, v = O.compress(bits(x), O.BF16)
    init = np.random.default_rng(5).integers(0, 256, 4096).astype(np.uint8)
    start = 1 << 36
    _, _, got, s0, end, err, _ = _call_compress_packed(dev, x, init, start)
    assert (s0, end) == (start, start + v.size) and err & 1
    assert (got == init).all()
