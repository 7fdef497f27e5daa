"""Dense -> BitsparseTensor conversion ("compress").

Mirrors reference lib_sparse/src/functions.py:23-99.  Two execution paths:

* TensorBuffer (``sparse_data`` given): ONE fused HIP kernel writes bitmask,
  prefix and values in a single read of ``dense`` and advances the buffer
  cursor on the device (no host sync).
* standalone (``sparse_data=None``): a count pass writes bitmask + prefix, the
  host reads nnz (one sync, as the reference does at
  triton_operators.py:50), allocates exactly nnz values, and a compact pass
  fills them.

With ``pack_sbit`` the values go to the 15/7-bit stream.  Into a TensorBuffer
this is the same single pass (``bs_compress_packed`` writes stream dwords
instead of raw values) at the cursor rounded up to a multiple of 8 values
(functions.py:78-81), so activations never share stream bytes.  The
standalone path, and an empty input into a TensorBuffer, compact raw values
first and pack them with ``bitpacking.pack_bits``.
"""
from __future__ import annotations

import math
from typing import NamedTuple

import torch
from torch import Tensor

from . import hip_operators as ops
from .bitpacking import pack_bits
from ..bitsparse import BitsparseTensor, TensorBuffer, tile_grid
from ..config import BLOCK_M, BLOCK_N
from ..fp8 import is_fp8


class _PreparedTiles(NamedTuple):
    M: int
    N: int
    grid_m: int
    grid_n: int
    num_tiles: int
    tile_numel: int
    bitmasks: Tensor
    prefix: Tensor


def _check_input(dense: Tensor) -> None:
    if dense.dtype != torch.bfloat16 and not is_fp8(dense.dtype):
        raise TypeError("BitsparseTensor supports bfloat16 and FP8 (e4m3fn/e5m2) values")
    if dense.dim() != 2:
        raise ValueError(f"dense_to_tilesparse expects a 2-D tensor, got {tuple(dense.shape)}")


def _prepare_tiles(dense: Tensor, relu: bool = False) -> _PreparedTiles:
    """Bitmask + uint32 prefix of ``dense`` (count pass, no values); ``relu``:
    of relu(dense), which is also written back into ``dense``.
    Reference: functions.py:23-45 (tile_pack + cumsum)."""
    _check_input(dense)
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    tile_bitmasks = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    tile_prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    ops.compress_into(dense, tile_bitmasks, tile_prefix, None, None, None, None, write_vals=False,
                      relu=relu, relu_out=dense if relu else None)
    return _PreparedTiles(M, N, grid_m, grid_n, num_tiles, TILE_NUMEL, tile_bitmasks, tile_prefix)


def dense_to_tilesparse(
    dense: Tensor, scale: Tensor | None,
    sparse_data: TensorBuffer | None = None,
    pack_sbit: bool = False,
) -> BitsparseTensor:
    """Convert a dense bf16 / fp8 [M, N] tensor into a BitsparseTensor.

    ``scale`` is carried as metadata (fp8 storage); values are stored bit for
    bit in ``dense``'s dtype.  Reference: functions.py:55-99.
    """
    _check_input(dense)
    ops.require_device(dense, "dense_to_tilesparse")
    return _to_tilesparse(dense.contiguous(), scale, sparse_data, pack_sbit, False)


def relu_and_compress(z: Tensor, sparse_data: TensorBuffer | None = None,
                      pack_sbit: bool = False) -> tuple[Tensor, BitsparseTensor]:
    """``h = z.relu_(); dense_to_tilesparse(h, None, sparse_data, pack_sbit)``
    (reference layers.py:29,37) with the ReLU fused into the compress pass:
    the kernel reads z once, writes relu(z) back into z and compresses it.
    Returns (h, BitsparseTensor) with h = z."""
    _check_input(z)
    ops.require_device(z, "relu_and_compress")
    if not z.is_contiguous():          # the in-place result must land in the caller's z
        h = z.relu_()
        return h, dense_to_tilesparse(h, None, sparse_data, pack_sbit)
    return z, _to_tilesparse(z, None, sparse_data, pack_sbit, True)


def linear_relu_and_compress(x: Tensor, W: Tensor, b: Tensor | None,
                             sparse_data: TensorBuffer) -> tuple[Tensor, BitsparseTensor]:
    """``z = x @ W.T; z = z + b; h = z.relu_(); dense_to_tilesparse(h, None,
    sparse_data)`` (reference layers.py:86-89, :29, :37) as one kernel: the
    up-projection GEMM writes h and its compressed form from its epilogue, so
    h is not read back to be compressed.  bf16 values into a (raw, not
    pack_sbit) TensorBuffer; ``fused_linear_relu_ok`` tells whether the
    operands qualify.  Returns (h, BitsparseTensor)."""
    if not fused_linear_relu_ok(x, W, b, sparse_data):
        raise ValueError("linear_relu_and_compress: operands do not qualify (fused_linear_relu_ok)")
    M, N = x.shape[0], W.shape[0]
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    h = torch.empty((M, N), device=x.device, dtype=torch.bfloat16)
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=x.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=x.device, dtype=torch.uint32)
    vals_offset, new_offset = sparse_data.cursor()
    ring = _flag_ring(x.device)
    slot, flag_addr = ring.take()
    ops.linear_relu_compress_into(x, W, b, h, bitmask, prefix, sparse_data.vals, vals_offset, new_offset,
                                  sparse_data.err_flags, flag_addr)
    sparse_data.advance(new_offset)
    sp = BitsparseTensor(sparse_data.vals, bitmask, prefix, (M, N), torch.bfloat16, grid_m, grid_n,
                         BLOCK_M, BLOCK_N, scale=None, vals_offset=vals_offset)
    sp.lookback_check = LookbackCheck(ring, slot)
    return h, sp


class LookbackTimeout(RuntimeError):
    """A fused up-projection's look-back wait gave up: its workgroups were not
    all resident (other work on the GPU), so the compressed activation it
    produced is wrong."""


class _FlagRing:
    """Time-out flags of fused up-projection launches in pinned host memory
    that the kernel stores into through its device address, so a launch adds
    no fill and no copy to the stream: the host clears a slot before the
    launch and reads it once the launch's event has completed.  Slot i is
    word 16 i (its own 64 bytes); a slot is reused only after the launch that
    last held it has ended and its check has taken the flag's value."""

    SLOTS = 256

    def __init__(self, device: torch.device):
        self.device = device
        self.host = torch.zeros(self.SLOTS * 16, dtype=torch.int32, pin_memory=True)
        self.words = self.host.numpy()
        self.base = ops.host_device_pointer(self.host)
        self.holders: list = [None] * self.SLOTS      # the LookbackCheck of each slot's last launch
        # one event per slot, recorded behind each launch that takes the slot
        # (re-recorded only after the previous holder has read its flag)
        self.events: list = [None] * self.SLOTS
        self.next = 0

    def take(self) -> tuple[int, int]:
        """(slot, device address of its word), cleared."""
        i = self.next
        self.next = (i + 1) % self.SLOTS
        if self.holders[i] is not None:
            self.holders[i].timed_out()                # waits for that launch, keeps its flag
            self.holders[i] = None
        self.words[16 * i] = 0
        return i, self.base + 64 * i


_FLAG_RINGS: dict[int, _FlagRing] = {}


def _flag_ring(device: torch.device) -> _FlagRing:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ring = _FLAG_RINGS.get(idx)
    if ring is None:
        ring = _FLAG_RINGS[idx] = _FlagRing(torch.device("cuda", idx))
    return ring


class LookbackCheck:
    """The time-out flag of one fused up-projection launch (a slot of the
    device's pinned flag ring) and an event recorded behind the launch, so
    that reading the flag waits for that kernel only (not for everything
    queued since)."""

    def __init__(self, ring: _FlagRing, slot: int):
        self.ring, self.slot = ring, slot
        if ring.events[slot] is None:
            ring.events[slot] = torch.cuda.Event()
        self.event = ring.events[slot]
        # on the stream the kernel went to (the ring's device, whichever is current)
        self.event.record(torch.cuda.current_stream(ring.device))
        self.result = None
        ring.holders[slot] = self

    def timed_out(self) -> bool:
        if self.result is None:
            self.event.synchronize()
            self.result = int(self.ring.words[16 * self.slot]) != 0
        return self.result

    def raise_if_timed_out(self) -> None:
        if self.timed_out():
            raise LookbackTimeout("fused up-projection: a look-back wait gave up (the GPU did not hold all "
                                  "of a strip's workgroups at once); its compressed activation is invalid")


def fused_linear_relu_ok(x: Tensor, W: Tensor, b: Tensor | None, sparse_data: TensorBuffer | None) -> bool:
    """The fused up-projection applies: bf16 operands the kernel takes as
    they are, and a raw bf16 TensorBuffer to compress into."""
    return (sparse_data is not None and not sparse_data.pack_sbit and sparse_data.vals.dtype == torch.bfloat16
            and x.is_cuda and ops.linear_relu_compress_supported(x, W, b))


def _to_tilesparse(dense: Tensor, scale: Tensor | None, sparse_data: TensorBuffer | None,
                   pack_sbit: bool, relu: bool) -> BitsparseTensor:
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)

    if sparse_data is None:
        prepared = _prepare_tiles(dense, relu)
        vals, vals_offset = ops.compact_vals(
            dense, prepared.bitmasks, prepared.prefix, None, None,
            M, N, grid_n, num_tiles, BLOCK_M, BLOCK_N, TILE_NUMEL, pack_sbit)
        return BitsparseTensor(vals, prepared.bitmasks, prepared.prefix, dense.shape, dense.dtype,
                               grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                               vals_offset=vals_offset, pack_sbit=pack_sbit)

    _check_buffer(sparse_data, dense.dtype, pack_sbit)
    fused = dict(relu=True, relu_out=dense) if relu else {}
    if pack_sbit:
        return _compress_packed_into_buffer(dense, scale, sparse_data, **fused)
    if sparse_data.vals.dtype != dense.dtype:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype} but the input is {dense.dtype}")
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    vals_offset, new_offset = sparse_data.cursor()        # the snapshot is never written again
    ops.compress_into(dense, bitmask, prefix, sparse_data.vals, vals_offset, new_offset,
                      sparse_data.err_flags, write_vals=True, **fused)
    sparse_data.advance(new_offset)
    return BitsparseTensor(sparse_data.vals, bitmask, prefix, dense.shape, dense.dtype,
                           grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                           vals_offset=vals_offset, pack_sbit=pack_sbit)


def _check_buffer(buf: TensorBuffer, dtype: torch.dtype, pack_sbit: bool) -> None:
    if bool(buf.pack_sbit) != bool(pack_sbit):
        raise ValueError(f"TensorBuffer(pack_sbit={buf.pack_sbit}) used with pack_sbit={pack_sbit}")
    if pack_sbit and buf.dtype != dtype:
        raise TypeError(f"packed TensorBuffer holds {buf.dtype} values but the input is {dtype}")


def _compress_packed_into_buffer(dense: Tensor, scale: Tensor | None, buf: TensorBuffer,
                                 **quant) -> BitsparseTensor:
    """One fused pass writes bitmask, prefix and the packed stream at the
    8-aligned cursor; no host synchronisation.  ``quant`` forwards the
    quantise / ReLU options of ``compress_into`` (quantize: e4m3fn values)."""
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    stored = torch.float8_e4m3fn if quant.get("quantize") else dense.dtype
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    if M * N == 0:
        return _compress_packed_staged(dense, scale, buf, bitmask, prefix, stored, **quant)
    vals_offset = torch.empty(1, device=dense.device, dtype=torch.int64)
    start, new_offset = buf.cursor()
    ops.compress_packed_into(dense, bitmask, prefix, buf.vals, start, new_offset, vals_offset,
                             buf.err_flags, **quant)
    buf.advance(new_offset)
    return BitsparseTensor(buf.vals, bitmask, prefix, dense.shape, stored,
                           grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                           vals_offset=vals_offset, pack_sbit=True)


def _compress_packed_staged(dense: Tensor, scale: Tensor | None, buf: TensorBuffer, bitmask: Tensor,
                            prefix: Tensor, stored: torch.dtype, **quant) -> BitsparseTensor:
    """Compress into a raw staging buffer, then pack at the 8-aligned cursor
    (the path for an empty input, whose cursor is still rounded up)."""
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    staging = torch.empty(max(M * N, 1), device=dense.device, dtype=stored)
    nnz = torch.empty(1, device=dense.device, dtype=torch.int64)
    ops.compress_into(dense, bitmask, prefix, staging, None, nnz, None, write_vals=True, **quant)
    vals_offset = (buf.offset + 7) // 8 * 8
    pack_bits(staging, buf.vals, vals_offset, M * N, prefix[num_tiles:num_tiles + 1], buf.err_flags)
    if buf.inplace_offset:
        buf.offset.copy_(vals_offset + nnz)
    else:
        buf.offset = vals_offset + nnz
    return BitsparseTensor(buf.vals, bitmask, prefix, dense.shape, stored,
                           grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                           vals_offset=vals_offset, pack_sbit=True)


# The ReLU^2 layer's square on the compress pass (bs_compress_relu2 +
# bs_amax_relu2_from) is switched off: a GPU memory fault ended a full GPU
# test run after it was added, and no out-of-bounds access has been found in
# it yet; the layer keeps its separate square / square-and-amax pass.
USE_FUSED_RELU2_SQUARE = False


def relu2_fused_ok(z: Tensor, sparse_data: TensorBuffer | None, pack_sbit: bool, k: float) -> bool:
    """The ReLU^2 layer's square can ride on the compress pass
    (``relu2_and_compress`` / ``relu2_quantize_and_compress``): the path is
    switched on (USE_FUSED_RELU2_SQUARE), a contiguous bf16 GPU z, a raw (not
    pack_sbit) TensorBuffer and a finite k."""
    return (USE_FUSED_RELU2_SQUARE and sparse_data is not None and not pack_sbit and not sparse_data.pack_sbit
            and z.is_cuda
            and z.dtype == torch.bfloat16 and z.dim() == 2 and z.is_contiguous() and math.isfinite(k))


def relu2_and_compress(z: Tensor, sparse_data: TensorBuffer, k: float) -> BitsparseTensor:
    """``h = z.relu_(); sp = dense_to_tilesparse(h, None, sparse_data);
    h.square_(); h.mul_(k)`` (reference layers.py:107-119, bf16 storage) in
    one pass: the compress of relu(z) writes bf16(bf16(r * r) * k) back into z
    (bs_compress_relu2).  Needs ``relu2_fused_ok``; returns the compressed r."""
    if not relu2_fused_ok(z, sparse_data, False, k):
        raise ValueError("relu2_and_compress: operands do not qualify (relu2_fused_ok)")
    _check_input(z)
    _check_buffer(sparse_data, z.dtype, False)
    if sparse_data.vals.dtype != z.dtype:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype} but the input is {z.dtype}")
    M, N = z.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=z.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=z.device, dtype=torch.uint32)
    vals_offset, new_offset = sparse_data.cursor()
    ops.compress_into(z, bitmask, prefix, sparse_data.vals, vals_offset, new_offset, sparse_data.err_flags,
                      write_vals=True, relu=True, relu_out=z, relu_square_k=k)
    sparse_data.advance(new_offset)
    return BitsparseTensor(sparse_data.vals, bitmask, prefix, z.shape, z.dtype, grid_m, grid_n, BLOCK_M, BLOCK_N,
                           scale=None, vals_offset=vals_offset)


def relu2_quantize_and_compress(z: Tensor, sparse_data: TensorBuffer,
                                k: float) -> tuple[Tensor, BitsparseTensor, int]:
    """The fp8 ReLU^2 forward's ``h = z.relu_(); (h8, s) = to_fp8(h);
    sp = dense_to_tilesparse(h8, s, sparse_data); h.square_(); h.mul_(k)``
    and the amax of ``to_fp8(h)`` (reference layers.py:107-119 with
    fp8.py:123-129): one amax pass over relu(z), one compress pass that also
    writes bf16(bf16(r * r) * k) back into z, and the amax of that square
    taken from the amax of r (the map is non-decreasing for a finite k, so its
    maximum is the image of r's: bs_amax_relu2_from).  Needs
    ``relu2_fused_ok``; returns (scale of the stored codes, compressed r, the
    workspace epoch of amax|h| for ``quantize_e4m3fn(z, epoch)``)."""
    if not relu2_fused_ok(z, sparse_data, False, k):
        raise ValueError("relu2_quantize_and_compress: operands do not qualify (relu2_fused_ok)")
    _check_buffer(sparse_data, torch.float8_e4m3fn, False)
    if sparse_data.vals.dtype != torch.float8_e4m3fn:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype}, need float8_e4m3fn")
    ops.require_device(z, "relu2_quantize_and_compress")
    M, N = z.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    amax_epoch = ops.amax_into_workspace(z, relu=True, reserve=3)   # + the compress and the derived amax
    scale = torch.empty((), device=z.device, dtype=torch.float32)
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=z.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=z.device, dtype=torch.uint32)
    vals_offset, new_offset = sparse_data.cursor()
    ops.compress_into(z, bitmask, prefix, sparse_data.vals, vals_offset, new_offset, sparse_data.err_flags,
                      write_vals=True, quantize=True, scale_out=scale, amax_epoch=amax_epoch,
                      relu=True, relu_out=z, relu_square_k=k)
    sparse_data.advance(new_offset)
    sp = BitsparseTensor(sparse_data.vals, bitmask, prefix, z.shape, torch.float8_e4m3fn, grid_m, grid_n,
                         BLOCK_M, BLOCK_N, scale=scale, vals_offset=vals_offset)
    return scale, sp, ops.amax_relu2_from(z.device, amax_epoch, k)


def relu_quantize_and_compress(
    z: Tensor, sparse_data: TensorBuffer | None = None, pack_sbit: bool = False,
    dense_out: bool = True,
) -> tuple[Tensor | None, Tensor, BitsparseTensor]:
    """``quantize_and_compress(z.relu_(), ...)`` with the ReLU fused into the
    amax and compress passes (relu(z) is written back into z, as the
    reference's in-place relu_ does, layers.py:29-37)."""
    if z.dtype != torch.bfloat16:
        raise TypeError("relu_quantize_and_compress expects a bfloat16 tensor")
    if not z.is_contiguous():
        return quantize_and_compress(z.relu_(), sparse_data, pack_sbit, dense_out=dense_out)
    return quantize_and_compress(z, sparse_data, pack_sbit, dense_out=dense_out, _relu=True)


def quantize_and_compress(
    dense: Tensor, sparse_data: TensorBuffer | None = None, pack_sbit: bool = False,
    dense_out: bool = True, _relu: bool = False,
) -> tuple[Tensor | None, Tensor, BitsparseTensor]:
    """bf16 [M, N] -> (e4m3fn dense, fp32 scale, BitsparseTensor of the e4m3fn
    values) with one amax pass and one fused quantize+compress pass.

    Equivalent to ``h8, s = to_fp8(h); dense_to_tilesparse(h8, s, sparse_data)``
    (reference layers.py:32-37) but reads ``h`` twice instead of three times.
    ``dense_out=False``: the e4m3fn dense copy is not written (None is
    returned in its place) when the caller only keeps the compressed form
    (the ReLU^2 layer multiplies the bf16 square, not h8).
    """
    if dense.dtype != torch.bfloat16:
        raise TypeError("quantize_and_compress expects a bfloat16 tensor")
    ops.require_device(dense, "quantize_and_compress")
    dense = dense.contiguous()
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    amax_epoch = ops.amax_into_workspace(dense, relu=_relu)
    fused = dict(relu=True, relu_out=dense) if _relu else {}
    # the standalone path compacts from the quantized dense copy
    need_q = dense_out or sparse_data is None
    q = torch.empty((M, N), device=dense.device, dtype=torch.float8_e4m3fn) if need_q else None
    scale = torch.empty((), device=dense.device, dtype=torch.float32)
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    if sparse_data is None:
        ops.compress_into(dense, bitmask, prefix, None, None, None, None, write_vals=False,
                          quantize=True, scale_out=scale, dense_q_out=q, amax_epoch=amax_epoch, **fused)
        vals, vals_offset = ops.compact_vals(q, bitmask, prefix, None, None, M, N, grid_n,
                                             num_tiles, BLOCK_M, BLOCK_N, TILE_NUMEL, pack_sbit)
        sp = BitsparseTensor(vals, bitmask, prefix, q.shape, q.dtype, grid_m, grid_n,
                             BLOCK_M, BLOCK_N, scale=scale, vals_offset=vals_offset,
                             pack_sbit=pack_sbit)
        return (q if dense_out else None), scale, sp
    _check_buffer(sparse_data, torch.float8_e4m3fn, pack_sbit)
    if pack_sbit:
        sp = _compress_packed_into_buffer(dense, scale, sparse_data, quantize=True, scale_out=scale,
                                          dense_q_out=q, amax_epoch=amax_epoch, **fused)
        return q, scale, sp
    if sparse_data.vals.dtype != torch.float8_e4m3fn:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype}, need float8_e4m3fn")
    vals_offset, new_offset = sparse_data.cursor()
    ops.compress_into(dense, bitmask, prefix, sparse_data.vals, vals_offset, new_offset,
                      sparse_data.err_flags, write_vals=True, quantize=True, scale_out=scale,
                      dense_q_out=q, amax_epoch=amax_epoch, **fused)
    sparse_data.advance(new_offset)
    sp = BitsparseTensor(sparse_data.vals, bitmask, prefix, (M, N), torch.float8_e4m3fn, grid_m, grid_n,
                         BLOCK_M, BLOCK_N, scale=scale, vals_offset=vals_offset)
    return q, scale, sp
