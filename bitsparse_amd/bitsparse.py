"""Compressed-activation container types.

Mirrors reference lib_sparse/bitsparse.py: ``pack_codec`` / ``bits_per_value``
(:8-23), ``BitsparseTensor`` (:26-87), ``TensorBuffer`` (:90-117) and
``tile_grid`` (:120-127), with the same constructor signatures, attributes
and storage-size accounting.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .fp8 import is_fp8
from .src.bitpacking import packed_nbytes


def pack_codec(dtype) -> int:
    """Codec id of a storage dtype: 0 = bf16, 1 = e4m3fn, 2 = e5m2.

    The id doubles as the dtype code of the HIP entry points.
    Reference: lib_sparse/bitsparse.py:8-18.
    """
    if dtype == getattr(torch, "float8_e4m3fn", None):
        return 1
    if dtype == getattr(torch, "float8_e5m2", None):
        return 2
    return 0


def bits_per_value(dtype) -> int:
    """Bits per value in the packed stream (sign dropped): 15 bf16, 7 fp8.
    Reference: lib_sparse/bitsparse.py:21-23."""
    return 7 if pack_codec(dtype) else 15


class BitsparseTensor:
    """A dense [M, N] matrix stored as 64x64-tile bitmasks, a uint32 tile
    prefix and the compacted positive values.

    vals        1-D storage-dtype tensor; this tensor's values start at
                ``vals_offset`` (shared TensorBuffer) or 0 (standalone)
    bitmask     uint8[T*512], bit f%8 of byte t*512 + f/8 = [x > 0]
    prefix      uint32[T+1], value offset of each tile relative to vals_offset
    vals_offset int64 device tensor
    scale       fp32 0-d tensor for fp8 storage (per-tensor scale) or None
    Reference: lib_sparse/bitsparse.py:26-87.
    """
    vals: Tensor
    bitmask: Tensor
    prefix: Tensor
    vals_offset: Tensor
    dtype: torch.dtype
    BLOCK_M: int
    BLOCK_N: int
    grid_m: int
    grid_n: int

    def __init__(self, vals, bitmask, prefix, shape, dtype,
                 grid_m, grid_n, BLOCK_M, BLOCK_N,
                 scale=None, vals_offset=None, pack_sbit=False):
        self.vals = vals
        self.bitmask = bitmask
        self.prefix = prefix
        if vals_offset is None:
            vals_offset = torch.zeros((), device=vals.device, dtype=torch.int64)
        self.vals_offset = vals_offset
        self.pack_sbit = pack_sbit
        self.dtype = dtype
        self.scale = scale
        self.grid_m = grid_m
        self.grid_n = grid_n
        self.BLOCK_M = BLOCK_M
        self.BLOCK_N = BLOCK_N
        self.shape = shape
        # produced by the fused up-projection: its look-back time-out flag
        # (functions.LookbackCheck), checked by the backward that reads it
        self.lookback_check = None

    @property
    def fp8(self) -> bool:
        """True when values are stored as FP8 (e4m3fn or e5m2)."""
        return is_fp8(self.dtype)

    @property
    def num_tiles(self) -> int:
        return self.grid_m * self.grid_n

    def __repr__(self):
        M, N = self.shape
        n = int(self.nnz().item())
        store = f"{self.dtype}".replace("torch.", "") + (" packed" if self.pack_sbit else "")
        return f"BitsparseTensor[{M}x{N}, {store}, {n} nonzeros, {100.0 * (1 - n / max(1, M * N)):.1f}% zeros]"

    def nnz(self):
        """Number of nonzeros as a 0-d int64 tensor (diagnostics): the last
        tile prefix, which counts every set bitmask bit.  Reference:
        lib_sparse/bitsparse.py:71-74."""
        return self.prefix[-1:].view(torch.int32).to(torch.int64)[0] & 0xFFFFFFFF

    def vram_size(self):
        """Stored bytes: values + bitmask + prefix (synchronises).
        Reference: lib_sparse/bitsparse.py:76-84."""
        nnz = int(self.prefix[-1].item())
        if self.pack_sbit:
            val_size = packed_nbytes(nnz, bits_per_value(self.dtype))
        else:
            val_size = nnz * self.vals.element_size()
        bitmask_size = self.bitmask.element_size() * self.bitmask.nelement()
        prefix_size = self.prefix.element_size() * self.prefix.nelement()
        return val_size + bitmask_size + prefix_size

    def sparsity_ratio(self):
        return 1 - self.nnz() / (self.shape[0] * self.shape[1])


class TensorBuffer:
    """Preallocated value storage shared by several BitsparseTensors.

    Each compress appends at ``offset`` and advances it on the device, so no
    host synchronisation is needed.  By default ``offset`` is rebound to a new
    1-element int64 tensor by every compress (the previous tensor becomes that
    BitsparseTensor's ``vals_offset`` snapshot, so no copy is made).  With
    ``inplace_offset=True`` the cursor keeps its identity as in the reference
    (lib_sparse/src/functions.py:80-94): each compress snapshots it with a
    device copy and writes the advanced cursor into the same tensor, so code
    that holds ``buf.offset`` across a compress sees it move.
    ``reset_buffer`` starts over.  Values that do not fit are dropped by the
    kernel and flagged; see ``overflowed``.  Reference:
    lib_sparse/bitsparse.py:90-117.
    """
    vals: Tensor
    offset: Tensor

    def __init__(self, size: int, device="cuda", dtype=torch.bfloat16,
                 pack_sbit: bool = False, *, inplace_offset: bool = False):
        """size: storage bytes; device: buffer device; dtype: stored dtype;
        inplace_offset: advance ``offset`` in place (the reference's cursor
        semantics) instead of rebinding it."""
        self.size = size
        self.device = device
        self.dtype = dtype
        self.pack_sbit = pack_sbit
        self.inplace_offset = bool(inplace_offset)
        if pack_sbit:
            storage_size = (self.size + 3) // 4 * 4 + 4
            self.vals = torch.zeros(storage_size, device=self.device, dtype=torch.uint8)
        else:
            if self.size % torch.empty((), dtype=dtype).element_size() != 0:
                raise ValueError("raw TensorBuffer size must be a multiple of dtype size")
            numel = self.size // torch.empty((), dtype=dtype).element_size()
            self.vals = torch.zeros(numel, device=self.device, dtype=self.dtype)
        self.offset = torch.zeros(1, device=self.device, dtype=torch.int64)
        self.err_flags = torch.zeros(1, device=self.device, dtype=torch.int32)

    def reset_buffer(self):
        """Start filling from offset 0 again (once per training step)."""
        if self.inplace_offset:
            self.offset.zero_()
        else:
            self.offset = torch.zeros(1, device=self.device, dtype=torch.int64)

    def cursor(self) -> tuple[Tensor, Tensor]:
        """(start, out) for one compress into this buffer: the kernel reads the
        cursor from ``start`` and writes the advanced cursor into ``out``;
        ``advance(out)`` afterwards.  In place: ``start`` is a snapshot copy and
        ``out`` the cursor tensor itself."""
        if self.inplace_offset:
            return self.offset.clone(), self.offset
        return self.offset, torch.empty(1, device=self.offset.device, dtype=torch.int64)

    def advance(self, out: Tensor) -> None:
        """Make ``out`` (from ``cursor``) the buffer's cursor."""
        if not self.inplace_offset:
            self.offset = out

    def overflowed(self) -> bool:
        """True if a compress ran out of capacity since construction
        (synchronises).  The reference has no such check."""
        return bool(self.err_flags.item() != 0)


def tile_grid(M: int, N: int, BLOCK_M: int, BLOCK_N: int) -> tuple[int, int, int, int, int]:
    """(grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES) of a dense shape.
    Reference: lib_sparse/bitsparse.py:120-127."""
    TILE_NUMEL = BLOCK_M * BLOCK_N
    TILE_BYTES = TILE_NUMEL // 8
    grid_m = (M + BLOCK_M - 1) // BLOCK_M
    grid_n = (N + BLOCK_N - 1) // BLOCK_N
    num_tiles = grid_m * grid_n
    return grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES
