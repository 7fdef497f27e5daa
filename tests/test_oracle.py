"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, each chosen so that a plausible slip in the oracle fails one of them:
* brute force on tiny inputs with a different mechanism (torch float compare,
  explicit (tile, row, col) loops in Python);
* the independent numpy formulation (pad/reshape/packbits) at many shapes;
* torch's own CPU casts for fp32 -> e4m3fn / bf16 and fp8 -> fp32;
* torch arithmetic for the ReLU^2 square and gradient (the reference's dense
  comparator formula, experiments/experiment.py:368);
* invariants: round trip = relu(x), popcount = nnz, monotone prefix.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import all_fp8_patterns, bits, from_bits, preact_input, relu_input, special_bf16

SHAPES = [(1, 1), (1, 64), (64, 1), (64, 64), (65, 64), (128, 128), (129, 131), (200, 70),
          (5, 300), (192, 256)]


def torch_pos(x: torch.Tensor) -> torch.Tensor:
    return x.float() > 0


# ---------------------------------------------------------------------------
# conversions vs torch's CPU casts
# ---------------------------------------------------------------------------
def test_e4m3fn_from_f32_all_bf16_patterns():
    f = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    q = O.f32_to_e4m3fn(f)
    tq = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan = np.isnan(O.np_decode_f32(q, O.E4M3FN)) & np.isnan(O.np_decode_f32(tq, O.E4M3FN))
    assert ((q == tq) | nan).all()


def test_e4m3fn_from_f32_random_and_boundaries():
    rng = np.random.default_rng(1)
    f = rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    # values around every rounding boundary of the e4m3fn grid
    grid = O.np_decode_f32(np.arange(256, dtype=np.uint8), O.E4M3FN)
    grid = grid[np.isfinite(grid)]
    mids = (np.sort(grid)[1:] + np.sort(grid)[:-1]) / 2
    edges = np.concatenate([mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf),
                            np.float32([448, 464, np.nextafter(np.float32(464), np.float32(1e9)),
                                        480, 1e9, np.inf, -np.inf, 2.0**-6, 2.0**-9, 2.0**-10,
                                        3 * 2.0**-11])]).astype(np.float32)
    f = np.concatenate([f, edges, -edges])
    q = O.f32_to_e4m3fn(f)
    tq = torch.from_numpy(f).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    nan = np.isnan(O.np_decode_f32(q, O.E4M3FN)) & np.isnan(O.np_decode_f32(tq, O.E4M3FN))
    assert ((q == tq) | nan).all()
    assert O.f32_to_e4m3fn(np.float32([464.0]))[0] == 0x7E          # ties to even: 448
    assert O.f32_to_e4m3fn(np.float32([464.01]))[0] == 0x7F         # no saturation: NaN


def test_bf16_from_f32_random():
    rng = np.random.default_rng(2)
    f = rng.integers(0, 2**32, 300_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    ob = O.f32_to_bf16(f)
    tb = bits(torch.from_numpy(f).to(torch.bfloat16))
    nan = np.isnan(f)
    assert (ob[~nan] == tb[~nan]).all()
    assert np.isnan(O.np_decode_f32(ob[nan], O.BF16)).all()


@pytest.mark.parametrize("code,dt", [(O.E4M3FN, torch.float8_e4m3fn), (O.E5M2, torch.float8_e5m2)])
def test_fp8_decode_all_patterns(code, dt):
    p = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(p).view(dt).float().numpy()
    mine = O.np_decode_f32(p, code)
    both_nan = np.isnan(ref) & np.isnan(mine)
    assert ((ref == mine) | both_nan).all()
    L = O.lib()
    f = L.or_e4m3fn_to_f32 if code == O.E4M3FN else L.or_e5m2_to_f32
    c = np.array([f(int(v)) for v in p], np.float32)
    assert ((c == ref) | (np.isnan(c) & np.isnan(ref))).all()


# ---------------------------------------------------------------------------
# compress format
# ---------------------------------------------------------------------------
def brute_compress(x: torch.Tensor):
    """Per-element Python loops with torch's float compare."""
    M, N = x.shape
    gm, gn = (M + 63) // 64, (N + 63) // 64
    pos = torch_pos(x)
    xb = bits(x)
    bm = np.zeros(gm * gn * 512, np.uint8)
    pref = [0]
    vals = []
    for tm in range(gm):
        for tn in range(gn):
            t = tm * gn + tn
            c = 0
            for r in range(64):
                for cc in range(64):
                    i, j = tm * 64 + r, tn * 64 + cc
                    if i < M and j < N and bool(pos[i, j]):
                        f = r * 64 + cc
                        bm[t * 512 + f // 8] |= 1 << (f % 8)
                        vals.append(xb[i, j])
                        c += 1
            pref.append(pref[-1] + c)
    return bm, np.array(pref, np.uint32), np.array(vals, xb.dtype)


@pytest.mark.parametrize("shape", [(1, 1), (3, 70), (65, 66), (130, 129)])
def test_compress_brute_force(shape):
    x = special_bf16(shape, seed=3)
    bm, pf, v = O.compress(bits(x), O.BF16)
    bm2, pf2, v2 = brute_compress(x)
    assert (bm == bm2).all() and (pf == pf2).all() and (v == v2).all()


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("sparsity", [0.0, 0.5, 0.9, 1.0])
def test_compress_c_vs_numpy(shape, sparsity):
    x = bits(relu_input(shape, sparsity, seed=4))
    a = O.compress(x, O.BF16)
    b = O.np_compress(x, O.BF16)
    for u, w in zip(a, b):
        assert u.dtype == w.dtype and (u == w).all()


@pytest.mark.parametrize("code,dt", [(O.E4M3FN, torch.float8_e4m3fn), (O.E5M2, torch.float8_e5m2)])
@pytest.mark.parametrize("shape", [(64, 64), (129, 131), (70, 200)])
def test_compress_fp8_all_patterns(code, dt, shape):
    x = all_fp8_patterns(shape, seed=5)
    a = O.compress(x, code)
    b = O.np_compress(x, code)
    for u, w in zip(a, b):
        assert (u == w).all()
    # positivity agrees with torch's own fp8 -> fp32 conversion
    pos = (torch.from_numpy(x).view(dt).float() > 0).numpy()
    assert int(a[1][-1]) == int(pos.sum())


@pytest.mark.parametrize("shape", SHAPES)
def test_invariants_and_round_trip(shape):
    x = special_bf16(shape, seed=6)
    xb = bits(x)
    bm, pf, v = O.compress(xb, O.BF16)
    M, N = shape
    gm, gn, T = O.tile_grid(M, N)
    assert pf[0] == 0 and (np.diff(pf.astype(np.int64)) >= 0).all()
    assert int(pf[-1]) == int(torch_pos(x).sum()) == int(np.unpackbits(bm).sum()) == v.size
    # per-tile counts are the prefix differences
    per_tile = np.unpackbits(bm.reshape(T, 512), axis=1).sum(axis=1)
    assert (per_tile == np.diff(pf.astype(np.int64))).all()
    # stored values are strictly positive and are the input's own bits
    assert (O.np_decode_f32(v, O.BF16) > 0).all()
    # padding bits of partial tiles are zero
    dense_mask = O.np_bitmask_to_dense_mask(bm, M, N)
    assert (dense_mask == torch_pos(x).numpy()).all()
    assert int(np.unpackbits(bm).sum()) == int(dense_mask.sum())
    # round trip: relu(x) numerically (NaN and -0 become +0)
    d = O.decompress(v, O.BF16, bm, pf, M, N)
    rt = torch.from_numpy(d.view(np.int16)).view(torch.bfloat16).float()
    ref = torch.where(torch_pos(x), x.float(), torch.zeros(()))
    assert torch.equal(rt, ref)
    assert (d == O.np_decompress(v, bm, M, N)).all()


def test_unpack_row_batches():
    M, N = 300, 200
    x = bits(relu_input((M, N), 0.5, seed=7))
    bm, pf, v = O.compress(x, O.BF16)
    gm, gn, T = O.tile_grid(M, N)
    full = O.decompress(v, O.BF16, bm, pf, M, N)
    for first, ntile_rows in [(0, 1), (1, 2), (3, 2), (4, 1)]:
        rows = min(ntile_rows * 64, M - first * 64)
        out = O.unpack(v, O.BF16, bm, pf, 0, first, gn, N, rows, ntile_rows * gn)
        assert (out == full[first * 64:first * 64 + rows]).all()


def test_compact_offsets_and_first_tile():
    x = bits(relu_input((130, 200), 0.5, seed=8))
    bm, cnt = O.tile_pack(x, O.BF16)
    pf = O.prefix(cnt)
    nnz = int(pf[-1])
    vals = np.zeros(nnz + 37, np.uint16)
    O.compact(x, O.BF16, bm, pf, vals, vals_offset=37)
    _, _, v = O.compress(x, O.BF16)
    assert (vals[37:] == v).all() and (vals[:37] == 0).all()
    # a tile range writes relative to prefix[first_tile]
    part = np.zeros(nnz, np.uint16)
    O.compact(x, O.BF16, bm, pf, part, 0, first_tile=4, num_tiles=5)
    s, e = int(pf[4]), int(pf[9])
    assert (part[:e - s] == v[s:e]).all()


# ---------------------------------------------------------------------------
# ReLU^2 unpack and gradients vs torch arithmetic
# ---------------------------------------------------------------------------
def test_relu2_square_bf16_matches_torch():
    x = relu_input((129, 131), 0.5, seed=9)
    bm, pf, v = O.compress(bits(x), O.BF16)
    sq = O.decompress(v, O.BF16, bm, pf, 129, 131, square=True)
    ref = bits(x.square().mul_(1))            # dense comparator: r.square(), * RELU2_SCALE
    assert (sq == ref).all()


def test_relu2_square_fp8_matches_torch():
    x = all_fp8_patterns((64, 128), seed=10)
    bm, pf, v = O.compress(x, O.E4M3FN)
    sq = O.decompress(v, O.E4M3FN, bm, pf, 64, 128, square=True)
    r = torch.from_numpy(x).view(torch.float8_e4m3fn).float()
    ref = torch.where(r > 0, r * r, torch.zeros(())).to(torch.bfloat16)
    assert (sq == bits(ref)).all()


def test_relu_grad_matches_torch_where():
    x = special_bf16((129, 131), seed=11)
    g = preact_input((129, 131), seed=12)
    bm, pf, v = O.compress(bits(x), O.BF16)
    out = O.relu_grad(bits(g), bm)
    ref = torch.where(torch_pos(x), g, torch.zeros((), dtype=torch.bfloat16))
    assert (out == bits(ref)).all()


def test_relu2_grad_bf16_matches_dense_comparator():
    # experiments/experiment.py:368: grad_preact = grad_z * (2.0 * RELU2_SCALE * r)
    z = preact_input((129, 131), seed=13)
    r = z.relu()
    g = preact_input((129, 131), seed=14)
    bm, pf, v = O.compress(bits(r), O.BF16)
    out = O.relu2_grad(bits(g), v, O.BF16, bm, pf)
    ref = g * (2.0 * 1 * r)
    act = (r.float() > 0).numpy()
    # active entries: bit-identical to the dense formula; inactive: the sparse
    # kernel writes +0.0 (triton_kernels.py:329) where the dense product gives +-0
    assert (out[act] == bits(ref)[act]).all()
    assert (out[~act] == 0).all()


def test_relu2_grad_fp8_closed_form():
    x = all_fp8_patterns((64, 192), seed=15)
    g = preact_input((64, 192), seed=16)
    bm, pf, v = O.compress(x, O.E4M3FN)
    s = 0.0123
    out = O.relu2_grad(bits(g), v, O.E4M3FN, bm, pf, scale=s)
    r = torch.from_numpy(x).view(torch.float8_e4m3fn).float()
    step1 = torch.where(r > 0, g.float() * (2.0 * r), torch.zeros(())).to(torch.bfloat16)
    # torch on the GPU multiplies by a 0-d fp32 device tensor through bf16
    ref = (step1.float() * torch.tensor(s).to(torch.bfloat16).float()).to(torch.bfloat16)
    assert (out == bits(ref)).all()


def test_to_fp8_definition():
    x = preact_input((100, 77), seed=17) * 3
    q, s = O.to_fp8(bits(x))
    amax = x.float().abs().max()
    assert s == pytest.approx(float(amax / 448), rel=0, abs=0)
    ref = (x.float() / torch.tensor(s, dtype=torch.float32)).to(torch.float8_e4m3fn)
    assert (q == bits(ref)).all()
    z = torch.zeros((4, 4), dtype=torch.bfloat16)
    q0, s0 = O.to_fp8(bits(z))
    assert s0 == np.float32(1e-9) and (q0 == 0).all()
    n = x.clone()
    n[3, 3] = float("nan")
    assert np.isnan(O.amax_bf16(bits(n)))


# ---------------------------------------------------------------------------
# packed value stream (pack_sbit)
# ---------------------------------------------------------------------------
def test_pack_bits_hand_examples():
    """Worked by hand from the format (value i at stream bits [i*b, (i+1)*b),
    LSB first): bf16 1.0 = 0x3f80 and 2.0 = 0x4000 -> 0x3f80 | 0x4000 << 15 =
    0x20003f80; e4m3fn 1.0 = 0x38 and 2.0 = 0x40 -> 0x38 | 0x40 << 7 = 0x2038."""
    s = np.zeros(8, np.uint8)
    O.pack_bits(np.array([0x3F80, 0x4000], np.uint16), O.BF16, s)
    assert s[:4].tobytes() == bytes([0x80, 0x3F, 0x00, 0x20]) and not s[4:].any()
    s = np.zeros(8, np.uint8)
    O.pack_bits(np.array([0x38, 0x40], np.uint8), O.E4M3FN, s)
    assert s[:2].tobytes() == bytes([0x38, 0x20]) and not s[2:].any()
    # a value starting at stream bit 15 (start = 1, bf16): 0x7fff << 15
    s = np.zeros(8, np.uint8)
    O.pack_bits(np.array([0x7FFF], np.uint16), O.BF16, s, start=1)
    assert int.from_bytes(s[:4].tobytes(), "little") == 0x7FFF << 15


def _brute_pack(raw, b, nbytes, start, init):
    acc = int.from_bytes(init.tobytes(), "little")
    for i, v in enumerate(raw.tolist()):
        for k in range(b):
            bit = (start + i) * b + k
            acc = (acc & ~(1 << bit)) | (((v >> k) & 1) << bit)
    return np.frombuffer(acc.to_bytes(nbytes, "little"), np.uint8)


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN, O.E5M2])
@pytest.mark.parametrize("start", [0, 1, 3, 7, 8, 13, 67])
def test_pack_bits_brute_force_and_numpy(code, start):
    """C packer == bit-by-bit Python-int packer == numpy bit-vector packer on
    random values (sign bit set too: only the low b bits are stored), with
    the stream pre-filled with random bytes that must survive outside the run."""
    rng = np.random.default_rng(start + 10 * code)
    b = O.bits_per_value(code)
    dt = np.uint16 if code == O.BF16 else np.uint8
    n = 37
    raw = rng.integers(0, np.iinfo(dt).max + 1, n).astype(dt)
    nbytes = ((start + n) * b + 7) // 8 + 6
    init = rng.integers(0, 256, nbytes).astype(np.uint8)
    c = O.pack_bits(raw, code, init.copy(), start)
    brute = _brute_pack(raw & ((1 << b) - 1), b, nbytes, start, init)
    npv = O.np_pack_bits(raw, code, init.copy(), start)
    assert (c == brute).all()
    assert (npv == brute).all()


@pytest.mark.parametrize("code", [O.BF16, O.E4M3FN])
def test_unpack_bits_inverts_pack(code):
    """The reference's uint16-word decode (bitpacking.py:37-55) and the numpy
    bit-vector decode both return the low b bits of every packed value."""
    rng = np.random.default_rng(code)
    b = O.bits_per_value(code)
    dt = np.uint16 if code == O.BF16 else np.uint8
    n, start = 500, 16
    raw = rng.integers(0, np.iinfo(dt).max + 1, n).astype(dt)
    s = np.zeros(((start + n) * b + 7) // 8 + 8, np.uint8)
    O.pack_bits(raw, code, s, start)
    want = raw & ((1 << b) - 1)
    assert (O.unpack_bits(s, code, np.arange(start, start + n)) == want).all()
    assert (O.np_unpack_bits(s, code, start, n) == want).all()


def test_pack_bits_eight_value_groups_are_byte_aligned():
    """Eight values are exactly 15 (bf16) / 7 (fp8) bytes, so runs starting at
    multiples of 8 values share no stream byte (reference functions.py:78-81)."""
    for code, b in ((O.BF16, 15), (O.E4M3FN, 7)):
        dt = np.uint16 if code == O.BF16 else np.uint8
        s = np.zeros(64, np.uint8)
        O.pack_bits(np.full(8, (1 << b) - 1, dt), code, s, 8)
        assert not s[:b].any() and (s[b:2 * b] == 0xFF).all() and not s[2 * b:].any()


@pytest.mark.parametrize("threads", [1, 3, 8])
@pytest.mark.parametrize("shape", [(1, 1), (64, 64), (130, 129), (700, 300)])
def test_compress_mt_matches_single_thread(shape, threads):
    """The row-block threaded oracle (used at configs[2]'s full size) is the
    single-threaded compress: same bitmask, prefix and values."""
    x = bits(preact_input(shape, mu=-0.3, seed=11).relu())
    want = O.compress(x, O.BF16)
    got = O.compress_mt(x, O.BF16, threads)
    for a, b in zip(want, got):
        assert a.dtype == b.dtype and np.array_equal(a, b)
    q = all_fp8_patterns(shape, seed=2)
    for a, b in zip(O.compress(q, O.E4M3FN), O.compress_mt(q, O.E4M3FN, threads)):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("threads", [1, 5])
def test_to_fp8_mt_matches_single_thread(threads):
    x = bits(preact_input((257, 129), mu=0.2, seed=4))
    q1, s1 = O.to_fp8(x)
    q2, s2 = O.to_fp8_mt(x, threads)
    assert s1 == s2 and np.array_equal(q1, q2)
    y = x.copy()
    y[100, 7] = 0x7fc0                                     # a NaN anywhere -> NaN scale
    q1, s1 = O.to_fp8(y)
    q2, s2 = O.to_fp8_mt(y, threads)
    assert s1 != s1 and s2 != s2 and np.array_equal(q1, q2)
