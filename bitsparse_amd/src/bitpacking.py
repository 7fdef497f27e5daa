"""Size helpers of the packed 15/7-bit value stream.

Mirrors reference lib_sparse/src/bitpacking.py:27-34.  The stream codec
itself (``_pack_kernel`` / ``load_packed_at_indices``, bitpacking.py:37-117)
is not part of this build yet: ``pack_sbit=True`` raises NotImplementedError
where the reference would pack.
"""


def packed_nbytes(numel: int, bits_per_value: int) -> int:
    """Payload bytes of ``numel`` values of ``bits_per_value`` bits."""
    return (int(numel) * bits_per_value + 7) // 8


def packed_storage_nbytes(numel: int, bits_per_value: int) -> int:
    """Word-aligned storage with one guard word for vectorised reads."""
    return ((packed_nbytes(numel, bits_per_value) + 3) // 4) * 4 + 4
