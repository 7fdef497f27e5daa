"""CPU oracle for the BitSparse activation-compression path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``bitsparse_amd`` imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

Two independent restatements of the reference encoding live here:

* ``liboracle`` (``bitsparse_oracle.c``): element-by-element loops that follow
  the reference kernels line by line (citations in that file).
* ``np_*``: vectorised numpy formulations of the same format built from
  library routines (pad + reshape/transpose into tile order,
  ``np.packbits(bitorder="little")``, boolean selection in C order).

Tests check the two against each other, against brute force on tiny inputs,
against torch's own CPU casts (fp8 / bf16 rounding) and against invariants
(round trip, popcount == nnz, monotone prefix).

Every array is a raw bit pattern: bf16 -> uint16, e4m3fn / e5m2 -> uint8.
Codec ids follow reference ``lib_sparse/bitsparse.py:8-18`` (0 bf16,
1 e4m3fn, 2 e5m2).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

BF16, E4M3FN, E5M2 = 0, 1, 2
TILE = 64
TILE_NUMEL = 4096
TILE_BYTES = 512

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None
_lock = threading.Lock()

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float


def build(force: bool = False) -> str:
    """Compile the C restatement (gcc) into oracle/_build/liboracle.so."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []),
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    with _lock:
        if _lib is None:
            build()
            L = ctypes.CDLL(_LIB_PATH)
            sigs = {
                "or_bf16_to_f32": (_f32, [ctypes.c_uint16]),
                "or_f32_to_bf16": (ctypes.c_uint16, [_f32]),
                "or_e4m3fn_to_f32": (_f32, [ctypes.c_uint8]),
                "or_e5m2_to_f32": (_f32, [ctypes.c_uint8]),
                "or_f32_to_e4m3fn": (ctypes.c_uint8, [_f32]),
                "or_tile_pack": (None, [_ptr, _int, _i64, _i64, _ptr, _ptr]),
                "or_prefix": (None, [_ptr, _i64, _ptr]),
                "or_compact": (None, [_ptr, _int, _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _i64]),
                "or_amax_bf16": (_f32, [_ptr, _i64]),
                "or_fp8_scale": (_f32, [_f32]),
                "or_quantize_bf16_to_e4m3fn": (None, [_ptr, _i64, _f32, _ptr]),
                "or_unpack": (None, [_ptr, _int, _ptr, _ptr, _i64, _ptr, _i64, _i64, _i64, _i64,
                                     _i64, _int, _f32]),
                "or_bf16_mul_scalar_tensor": (None, [_ptr, _i64, _f32]),
                "or_relu_grad": (None, [_ptr, _i64, _i64, _ptr]),
                "or_relu2_grad": (None, [_ptr, _i64, _i64, _ptr, _int, _ptr, _ptr, _i64, _f32, _ptr]),
                "or_compress": (_i64, [_ptr, _int, _i64, _i64, _ptr, _ptr, _ptr, _ptr, _i64]),
                "or_pack_bits": (None, [_ptr, _int, _i64, _int, _ptr, _i64]),
                "or_unpack_bits_at": (ctypes.c_uint32, [_ptr, _int, _i64]),
            }
            for name, (res, args) in sigs.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
        return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _check_bits(x: np.ndarray, dtype: int) -> None:
    want = np.uint16 if dtype == BF16 else np.uint8
    if x.dtype != want:
        raise TypeError(f"codec {dtype} expects {want.__name__} bit patterns, got {x.dtype}")


def tile_grid(M: int, N: int) -> tuple[int, int, int]:
    gm, gn = (M + TILE - 1) // TILE, (N + TILE - 1) // TILE
    return gm, gn, gm * gn


# --------------------------------------------------------------------------
# C restatement wrappers
# --------------------------------------------------------------------------
def tile_pack(x: np.ndarray, dtype: int) -> tuple[np.ndarray, np.ndarray]:
    _check_bits(x, dtype)
    x = np.ascontiguousarray(x)
    M, N = x.shape
    T = tile_grid(M, N)[2]
    bm = np.zeros(T * TILE_BYTES, np.uint8)
    counts = np.zeros(T, np.int32)
    lib().or_tile_pack(_p(x), dtype, M, N, _p(bm), _p(counts))
    return bm, counts


def prefix(counts: np.ndarray) -> np.ndarray:
    counts = np.ascontiguousarray(counts, dtype=np.int32)
    out = np.zeros(counts.size + 1, np.uint32)
    lib().or_prefix(_p(counts), counts.size, _p(out))
    return out


def compact(x: np.ndarray, dtype: int, bitmask: np.ndarray, pref: np.ndarray,
            vals: np.ndarray, vals_offset: int = 0, first_tile: int = 0,
            num_tiles: int | None = None) -> np.ndarray:
    _check_bits(x, dtype)
    M, N = x.shape
    if num_tiles is None:
        num_tiles = tile_grid(M, N)[2] - first_tile
    lib().or_compact(_p(np.ascontiguousarray(x)), dtype, M, N, _p(bitmask), _p(pref),
                     _p(vals), vals_offset, first_tile, num_tiles)
    return vals


def compress(x: np.ndarray, dtype: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(bitmask uint8[T*512], prefix uint32[T+1], vals[nnz]) of a dense tile grid."""
    bm, counts = tile_pack(x, dtype)
    pref = prefix(counts)
    vals = np.zeros(int(pref[-1]), x.dtype)
    compact(x, dtype, bm, pref, vals)
    return bm, pref, vals


def unpack(vals: np.ndarray, vdtype: int, bitmask: np.ndarray, pref: np.ndarray,
           vals_offset: int, first_m_tile: int, grid_n: int, K: int, batch_rows: int,
           num_tiles: int, square: bool = False, relu2_scale: float = 1.0) -> np.ndarray:
    out_dtype = np.uint16 if (square or vdtype == BF16) else np.uint8
    out = np.zeros((batch_rows, K), out_dtype)
    if vals.size == 0:
        vals = np.zeros(1, vals.dtype)
    lib().or_unpack(_p(vals), vdtype, _p(bitmask), _p(pref), vals_offset, _p(out),
                    first_m_tile, grid_n, K, batch_rows, num_tiles, int(square), relu2_scale)
    return out


def decompress(vals, vdtype, bitmask, pref, M, N, vals_offset=0, square=False, relu2_scale=1.0):
    gm, gn, T = tile_grid(M, N)
    return unpack(vals, vdtype, bitmask, pref, vals_offset, 0, gn, N, M, T, square, relu2_scale)


def bf16_mul_scalar_tensor(x: np.ndarray, s: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16).copy()
    lib().or_bf16_mul_scalar_tensor(_p(x), x.size, s)
    return x


def relu_grad(grad: np.ndarray, bitmask: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(grad, dtype=np.uint16).copy()
    M, N = g.shape
    lib().or_relu_grad(_p(g), M, N, _p(bitmask))
    return g


def relu2_grad(grad: np.ndarray, vals: np.ndarray, vdtype: int, bitmask: np.ndarray,
               pref: np.ndarray, vals_offset: int = 0, relu2_scale: float = 1.0,
               scale: float | None = None) -> np.ndarray:
    g = np.ascontiguousarray(grad, dtype=np.uint16).copy()
    M, N = g.shape
    sc = np.array([scale if scale is not None else 0.0], np.float32)
    if vals.size == 0:
        vals = np.zeros(1, vals.dtype)
    lib().or_relu2_grad(_p(g), M, N, _p(vals), vdtype, _p(bitmask), _p(pref), vals_offset,
                        relu2_scale, _p(sc) if scale is not None else None)
    return g


def bits_per_value(dtype: int) -> int:
    """Stored bits per value of the packed stream (reference bitsparse.py:21-23)."""
    return 15 if dtype == BF16 else 7


def pack_bits(raw: np.ndarray, dtype: int, stream: np.ndarray, start: int = 0) -> np.ndarray:
    """C restatement of the stream packer: raw values into ``stream`` (uint8,
    modified in place) at value index ``start``."""
    _check_bits(raw, dtype)
    raw = np.ascontiguousarray(raw)
    assert stream.dtype == np.uint8 and stream.flags["C_CONTIGUOUS"]
    assert (start + raw.size) * bits_per_value(dtype) <= stream.size * 8
    lib().or_pack_bits(_p(raw), dtype, raw.size, bits_per_value(dtype), _p(stream), start)
    return stream


def unpack_bits(stream: np.ndarray, dtype: int, idx) -> np.ndarray:
    """Values at indices ``idx`` of a packed stream (C restatement of the
    reference's uint16-word decode; needs the guard word after the payload)."""
    bits = bits_per_value(dtype)
    out = np.array([lib().or_unpack_bits_at(_p(stream), bits, int(i)) for i in np.ravel(idx)],
                   dtype=np.uint16 if dtype == BF16 else np.uint8)
    return out


def amax_bf16(x: np.ndarray) -> float:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return float(lib().or_amax_bf16(_p(x), x.size))


def fp8_scale(amax: float) -> float:
    return float(lib().or_fp8_scale(amax))


def quantize_e4m3fn(x: np.ndarray, scale: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    q = np.zeros(x.shape, np.uint8)
    lib().or_quantize_bf16_to_e4m3fn(_p(x), x.size, scale, _p(q))
    return q


def to_fp8(x: np.ndarray) -> tuple[np.ndarray, float]:
    """(e4m3fn bits, fp32 scale): scale = max(amax/448, 1e-9), q = RNE(x/scale)."""
    s = fp8_scale(amax_bf16(x))
    return quantize_e4m3fn(x, s), s


def f32_to_e4m3fn(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32).reshape(-1)
    L = lib()
    return np.fromiter((L.or_f32_to_e4m3fn(float(v)) for v in f), np.uint8, f.size)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32).reshape(-1)
    L = lib()
    return np.fromiter((L.or_f32_to_bf16(float(v)) for v in f), np.uint16, f.size)


def _row_blocks(M: int, threads: int) -> list[tuple[int, int]]:
    """Split [0, M) into `threads` ranges whose starts are multiples of 64."""
    gm = (M + TILE - 1) // TILE
    per = max(1, (gm + threads - 1) // threads)
    return [(tm * TILE, min(M, (tm + per) * TILE)) for tm in range(0, gm, per)]


def _pool_map(fn, items, threads: int):
    from concurrent.futures import ThreadPoolExecutor   # ctypes calls drop the GIL
    with ThreadPoolExecutor(max_workers=threads) as ex:
        return list(ex.map(fn, items))


def compress_mt(x: np.ndarray, dtype: int, threads: int | None = None):
    """``compress`` with the C loops run over row blocks on `threads` host
    threads: the same per-tile functions (or_tile_pack on each block of tile
    rows, one or_prefix, or_compact over each block's tiles at that block's
    prefix), so the result is the single-threaded one."""
    _check_bits(x, dtype)
    x = np.ascontiguousarray(x)
    M, N = x.shape
    gm, gn, T = tile_grid(M, N)
    threads = threads or min(16, os.cpu_count() or 1)
    L, eb = lib(), x.itemsize
    bm = np.zeros(T * TILE_BYTES, np.uint8)
    counts = np.zeros(T, np.int32)
    blocks = _row_blocks(M, threads)

    def pack(b):
        r0, r1 = b
        t0 = (r0 // TILE) * gn
        L.or_tile_pack(_p(x) + r0 * N * eb, dtype, r1 - r0, N,
                       _p(bm) + t0 * TILE_BYTES, _p(counts) + 4 * t0)
    _pool_map(pack, blocks, threads)
    pref = prefix(counts)
    vals = np.zeros(int(pref[-1]), x.dtype)

    def comp(b):
        r0, r1 = b
        t0, t1 = (r0 // TILE) * gn, ((r1 + TILE - 1) // TILE) * gn
        L.or_compact(_p(x), dtype, M, N, _p(bm), _p(pref), _p(vals), int(pref[t0]), t0, t1 - t0)
    _pool_map(comp, blocks, threads)
    return bm, pref, vals


def to_fp8_mt(x: np.ndarray, threads: int | None = None) -> tuple[np.ndarray, float]:
    """``to_fp8`` over slices on `threads` host threads (amax is a max of
    per-slice maxima, NaN-propagating as or_amax_bf16 is; the quantizer is
    elementwise)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    flat = x.reshape(-1)
    threads = threads or min(16, os.cpu_count() or 1)
    step = (flat.size + threads - 1) // threads
    parts = [(i, min(flat.size, i + step)) for i in range(0, flat.size, step)]
    L = lib()
    maxima = _pool_map(lambda p: float(L.or_amax_bf16(_p(flat) + 2 * p[0], p[1] - p[0])),
                       parts, threads)
    amax = float("nan") if any(m != m for m in maxima) else max(maxima, default=0.0)
    s = fp8_scale(amax)
    q = np.zeros(flat.size, np.uint8)
    _pool_map(lambda p: L.or_quantize_bf16_to_e4m3fn(_p(flat) + 2 * p[0], p[1] - p[0], s,
                                                      _p(q) + p[0]), parts, threads)
    return q.reshape(x.shape), s


def compress_timed_call(x: np.ndarray, dtype: int, bm, pref, counts, vals) -> int:
    """Single C call doing the whole compress (the CPU baseline's unit of work)."""
    M, N = x.shape
    return int(lib().or_compress(_p(x), dtype, M, N, _p(bm), _p(pref), _p(counts), _p(vals), 0))


# --------------------------------------------------------------------------
# numpy restatement (independent of the C loops)
# --------------------------------------------------------------------------
def np_decode_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    """Exact fp32 values of bit patterns (NaN where the format says NaN)."""
    if dtype == BF16:
        return (x.astype(np.uint32) << 16).view(np.float32)
    x = x.astype(np.int64)
    s = np.where(x & 0x80, -1.0, 1.0)
    if dtype == E4M3FN:
        e, m = (x >> 3) & 15, x & 7
        v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e - 10.0))
        v = np.where((e == 15) & (m == 7), np.nan, v)
    else:
        e, m = (x >> 2) & 31, x & 3
        v = np.where(e == 0, m * 2.0 ** -16, (4 + m) * np.exp2(e - 17.0))
        v = np.where(e == 31, np.where(m == 0, np.inf, np.nan), v)
    return (s * v).astype(np.float32)


def _to_tiles(a: np.ndarray) -> np.ndarray:
    """[M, N] -> [T, 4096] in tile order (zero padded)."""
    M, N = a.shape
    gm, gn, T = tile_grid(M, N)
    p = np.zeros((gm * TILE, gn * TILE), a.dtype)
    p[:M, :N] = a
    return p.reshape(gm, TILE, gn, TILE).transpose(0, 2, 1, 3).reshape(T, TILE_NUMEL)


def _from_tiles(t: np.ndarray, M: int, N: int) -> np.ndarray:
    gm, gn, T = tile_grid(M, N)
    return t.reshape(gm, gn, TILE, TILE).transpose(0, 2, 1, 3).reshape(gm * TILE, gn * TILE)[:M, :N]


def np_compress(x: np.ndarray, dtype: int):
    with np.errstate(invalid="ignore"):
        pos = np_decode_f32(x, dtype) > 0
    tiles_pos = _to_tiles(pos)
    bm = np.packbits(tiles_pos, axis=1, bitorder="little").reshape(-1)
    counts = tiles_pos.sum(axis=1, dtype=np.int64)
    pref = np.zeros(counts.size + 1, np.uint64)
    pref[1:] = np.cumsum(counts)
    vals = _to_tiles(x)[tiles_pos]
    return bm, (pref & 0xFFFFFFFF).astype(np.uint32), vals


def np_decompress(vals: np.ndarray, bitmask: np.ndarray, M: int, N: int,
                  vals_offset: int = 0) -> np.ndarray:
    gm, gn, T = tile_grid(M, N)
    bits = np.unpackbits(bitmask.reshape(T, TILE_BYTES), axis=1, bitorder="little").astype(bool)
    tiles = np.zeros((T, TILE_NUMEL), vals.dtype)
    n = int(bits.sum())
    tiles[bits] = vals[vals_offset:vals_offset + n]
    return np.ascontiguousarray(_from_tiles(tiles, M, N))


def np_bitmask_to_dense_mask(bitmask: np.ndarray, M: int, N: int) -> np.ndarray:
    gm, gn, T = tile_grid(M, N)
    bits = np.unpackbits(bitmask.reshape(T, TILE_BYTES), axis=1, bitorder="little").astype(bool)
    return np.ascontiguousarray(_from_tiles(bits, M, N))


def np_pack_bits(raw: np.ndarray, dtype: int, stream: np.ndarray, start: int = 0) -> np.ndarray:
    """numpy restatement of the stream packer: each value's low b bits as a
    little-endian bit vector, concatenated, written at bit start*b (bits of
    ``stream`` outside the run are kept)."""
    b = bits_per_value(dtype)
    n = raw.size
    if n == 0:
        return stream
    vals = raw.astype(np.uint32) & ((1 << b) - 1)
    vbits = ((vals[:, None] >> np.arange(b, dtype=np.uint32)[None, :]) & 1).astype(np.uint8).reshape(-1)
    sbits = np.unpackbits(stream, bitorder="little")
    sbits[start * b:(start + n) * b] = vbits
    stream[:] = np.packbits(sbits, bitorder="little")
    return stream


def np_unpack_bits(stream: np.ndarray, dtype: int, start: int, n: int) -> np.ndarray:
    """numpy inverse of ``np_pack_bits``: n values from value index ``start``."""
    b = bits_per_value(dtype)
    sbits = np.unpackbits(stream, bitorder="little")[start * b:(start + n) * b].reshape(n, b)
    v = (sbits.astype(np.uint32) << np.arange(b, dtype=np.uint32)[None, :]).sum(axis=1)
    return v.astype(np.uint16 if dtype == BF16 else np.uint8)
