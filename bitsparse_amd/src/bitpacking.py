"""Packed 15/7-bit value stream (``pack_sbit`` storage).

Mirrors reference lib_sparse/src/bitpacking.py: value i of a stream occupies
stream bits [i*b, (i+1)*b), least significant bit first, b = 15 for bf16 and
7 for fp8 (the sign bit of a ReLU value is always 0 and is dropped).  The
size helpers follow bitpacking.py:27-34; ``pack_bits`` replaces the
``_pack_kernel`` launch (bitpacking.py:58-117) with the HIP kernel behind
``bs_pack_bits``.  Reading a packed stream is done by the decompress and
ReLU^2-gradient kernels (``bs_decompress_packed`` / ``bs_relu2_grad_packed``).
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib
from .._lib import check, ptr, require_device, stream_handle


def packed_nbytes(numel: int, bits_per_value: int) -> int:
    """Payload bytes of ``numel`` values of ``bits_per_value`` bits."""
    return (int(numel) * bits_per_value + 7) // 8


def packed_storage_nbytes(numel: int, bits_per_value: int) -> int:
    """Word-aligned storage with one guard word for vectorised reads."""
    return ((packed_nbytes(numel, bits_per_value) + 3) // 4) * 4 + 4


def pack_bits(raw: Tensor, stream: Tensor, start: Tensor | None, count: int,
              count_tensor: Tensor | None = None, err_flags: Tensor | None = None) -> Tensor:
    """Pack raw[0:count] (bf16 / fp8 values) into ``stream`` (uint8 storage)
    at value index ``start`` (0-d / 1-element int64 device tensor, None = 0).

    ``count_tensor``: a uint32 device element (e.g. ``prefix[-1:]``) holding
    the actual count, which may be smaller than ``count`` (an upper bound);
    the pack then needs no host synchronisation.  Returns ``stream``."""
    require_device(raw, "pack_bits")
    if stream.dtype != torch.uint8:
        raise TypeError("pack_bits: the stream storage is uint8")
    from .hip_operators import dtype_code
    L = _lib.load()
    check(L.bs_pack_bits(raw.data_ptr(), dtype_code(raw.dtype), ptr(count_tensor), int(count),
                         stream.data_ptr(), stream.numel(), ptr(start), ptr(err_flags),
                         stream_handle(raw.device)), "bs_pack_bits")
    return stream
