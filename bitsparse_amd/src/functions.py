"""Dense -> BitsparseTensor conversion ("compress").

Mirrors reference lib_sparse/src/functions.py:23-99.  Two execution paths:

* TensorBuffer (``sparse_data`` given): ONE fused HIP kernel writes bitmask,
  prefix and values in a single read of ``dense`` and advances the buffer
  cursor on the device (no host sync).
* standalone (``sparse_data=None``): a count pass writes bitmask + prefix, the
  host reads nnz (one sync, as the reference does at
  triton_operators.py:50), allocates exactly nnz values, and a compact pass
  fills them.
"""
from __future__ import annotations

from typing import NamedTuple

import torch
from torch import Tensor

from . import hip_operators as ops
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


def _prepare_tiles(dense: Tensor) -> _PreparedTiles:
    """Bitmask + uint32 prefix of ``dense`` (count pass, no values).
    Reference: functions.py:23-45 (tile_pack + cumsum)."""
    _check_input(dense)
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    tile_bitmasks = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    tile_prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    ops.compress_into(dense, tile_bitmasks, tile_prefix, None, None, None, None, write_vals=False)
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
    if pack_sbit:
        raise NotImplementedError(ops._SBIT_MSG)
    _check_input(dense)
    ops.require_device(dense, "dense_to_tilesparse")
    dense = dense.contiguous()
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)

    if sparse_data is None:
        prepared = _prepare_tiles(dense)
        vals, vals_offset = ops.compact_vals(
            dense, prepared.bitmasks, prepared.prefix, None, None,
            M, N, grid_n, num_tiles, BLOCK_M, BLOCK_N, TILE_NUMEL, pack_sbit)
        return BitsparseTensor(vals, prepared.bitmasks, prepared.prefix, dense.shape, dense.dtype,
                               grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                               vals_offset=vals_offset, pack_sbit=pack_sbit)

    if sparse_data.pack_sbit:
        raise NotImplementedError(ops._SBIT_MSG)
    if sparse_data.vals.dtype != dense.dtype:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype} but the input is {dense.dtype}")
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    vals_offset = sparse_data.offset                      # snapshot: never written again
    new_offset = torch.empty(1, device=dense.device, dtype=torch.int64)
    ops.compress_into(dense, bitmask, prefix, sparse_data.vals, vals_offset, new_offset,
                      sparse_data.err_flags, write_vals=True)
    sparse_data.offset = new_offset
    return BitsparseTensor(sparse_data.vals, bitmask, prefix, dense.shape, dense.dtype,
                           grid_m, grid_n, BLOCK_M, BLOCK_N, scale=scale,
                           vals_offset=vals_offset, pack_sbit=pack_sbit)


def quantize_and_compress(
    dense: Tensor, sparse_data: TensorBuffer | None = None,
) -> tuple[Tensor, Tensor, BitsparseTensor]:
    """bf16 [M, N] -> (e4m3fn dense, fp32 scale, BitsparseTensor of the e4m3fn
    values) with one amax pass and one fused quantize+compress pass.

    Equivalent to ``h8, s = to_fp8(h); dense_to_tilesparse(h8, s, sparse_data)``
    (reference layers.py:32-37) but reads ``h`` twice instead of three times.
    """
    if dense.dtype != torch.bfloat16:
        raise TypeError("quantize_and_compress expects a bfloat16 tensor")
    ops.require_device(dense, "quantize_and_compress")
    dense = dense.contiguous()
    M, N = dense.shape
    grid_m, grid_n, num_tiles, TILE_NUMEL, TILE_BYTES = tile_grid(M, N, BLOCK_M, BLOCK_N)
    amax_epoch = ops.amax_into_workspace(dense)
    q = torch.empty((M, N), device=dense.device, dtype=torch.float8_e4m3fn)
    scale = torch.empty((), device=dense.device, dtype=torch.float32)
    bitmask = torch.empty(num_tiles * TILE_BYTES, device=dense.device, dtype=torch.uint8)
    prefix = torch.empty(num_tiles + 1, device=dense.device, dtype=torch.uint32)
    if sparse_data is None:
        ops.compress_into(dense, bitmask, prefix, None, None, None, None, write_vals=False,
                          quantize=True, scale_out=scale, dense_q_out=q, amax_epoch=amax_epoch)
        vals, vals_offset = ops.compact_vals(q, bitmask, prefix, None, None, M, N, grid_n,
                                             num_tiles, BLOCK_M, BLOCK_N, TILE_NUMEL, False)
        sp = BitsparseTensor(vals, bitmask, prefix, q.shape, q.dtype, grid_m, grid_n,
                             BLOCK_M, BLOCK_N, scale=scale, vals_offset=vals_offset)
        return q, scale, sp
    if sparse_data.vals.dtype != torch.float8_e4m3fn:
        raise TypeError(f"TensorBuffer stores {sparse_data.vals.dtype}, need float8_e4m3fn")
    vals_offset = sparse_data.offset
    new_offset = torch.empty(1, device=dense.device, dtype=torch.int64)
    ops.compress_into(dense, bitmask, prefix, sparse_data.vals, vals_offset, new_offset,
                      sparse_data.err_flags, write_vals=True, quantize=True, scale_out=scale,
                      dense_q_out=q, amax_epoch=amax_epoch)
    sparse_data.offset = new_offset
    sp = BitsparseTensor(sparse_data.vals, bitmask, prefix, q.shape, q.dtype, grid_m, grid_n,
                         BLOCK_M, BLOCK_N, scale=scale, vals_offset=vals_offset)
    return q, scale, sp
