"""Launchers of the HIP codec kernels (libbitsparse_hip.so) on torch tensors.

Same function names, argument meaning and in-place conventions as reference
lib_sparse/src/triton_operators.py (:21-202); ``triton_operators`` is kept as
an alias module of this one.  Every function enqueues on torch's current
stream of the tensors' device and raises on CPU tensors (no CPU path).
"""
from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from .. import _lib
from .._lib import check, ptr, require_device, stream_handle
from ..bitsparse import BitsparseTensor, bits_per_value, pack_codec
from ..config import RELU2_SCALE
from .bitpacking import pack_bits, packed_storage_nbytes


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.DT_BF16
    if dtype == torch.float8_e4m3fn:
        return _lib.DT_E4M3FN
    if dtype == torch.float8_e5m2:
        return _lib.DT_E5M2
    raise TypeError("BitsparseTensor supports bfloat16 and FP8 (e4m3fn/e5m2) values")


def _contig(t: Tensor, what: str) -> Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous (row-major)")
    return t


# ---------------------------------------------------------------------------
# compress
# ---------------------------------------------------------------------------
def tile_pack(
    dense: Tensor, tile_counts: Tensor, tile_bitmasks: Tensor,
    M: int, N: int, grid_m: int, grid_n: int,
    BLOCK_M: int, BLOCK_N: int,
    TILE_NUMEL: int, TILE_BYTES: int,
) -> None:
    """Per-tile bitmask and int32 nonzero counts (in-place outputs).
    Reference: triton_operators.py:21-33."""
    require_device(dense, "tile_pack")
    _contig(dense, "dense")
    if tile_counts.dtype != torch.int32 or tile_bitmasks.dtype != torch.uint8:
        raise TypeError("tile_pack: counts must be int32 and bitmasks uint8")
    L = _lib.load()
    check(L.bs_tile_pack(dense.data_ptr(), dtype_code(dense.dtype), M, N,
                         tile_counts.data_ptr(), tile_bitmasks.data_ptr(),
                         stream_handle(dense.device)), "bs_tile_pack")


def prefix_from_counts(tile_counts: Tensor, tile_prefix: Tensor) -> None:
    """prefix[0] = 0, prefix[1:] = cumsum(counts) as uint32 (reference
    functions.py:38-40)."""
    L = _lib.load()
    check(L.bs_prefix_from_counts(tile_counts.data_ptr(), tile_counts.numel(),
                                  tile_prefix.data_ptr(), stream_handle(tile_counts.device)),
          "bs_prefix_from_counts")


def compact_vals(
    dense: Tensor, tile_bitmasks: Tensor, tile_prefix: Tensor,
    vals: Tensor | None, vals_offset: Tensor | None,
    M: int, N: int, grid_n: int, num_tiles: int,
    BLOCK_M: int, BLOCK_N: int, TILE_NUMEL: int, pack_sbit: bool,
) -> tuple[Tensor, Tensor]:
    """Compact positive values into standalone (vals=None: exact-size, after
    one host sync for nnz) or preallocated storage.  ``pack_sbit``: ``vals``
    is the uint8 packed stream; the values are compacted into a raw staging
    buffer and packed at ``vals_offset`` (a value index).
    Reference: triton_operators.py:36-115."""
    require_device(dense, "compact_vals")
    _contig(dense, "dense")
    if pack_sbit:
        return _compact_vals_packed(dense, tile_bitmasks, tile_prefix, vals, vals_offset, M, N,
                                    num_tiles)
    if vals is None:
        nnz = int(tile_prefix[-1].item())
        vals = torch.empty(nnz, device=dense.device, dtype=dense.dtype)
        vals_offset = torch.zeros((), device=dense.device, dtype=torch.int64)
    elif vals.dtype != dense.dtype:
        raise TypeError(f"compact_vals: storage dtype {vals.dtype} differs from input {dense.dtype}")
    L = _lib.load()
    check(L.bs_compact_vals(dense.data_ptr(), dtype_code(dense.dtype), M, N,
                            tile_bitmasks.data_ptr(), tile_prefix.data_ptr(),
                            vals.data_ptr(), vals.numel(), ptr(vals_offset), 0, num_tiles,
                            None, stream_handle(dense.device)), "bs_compact_vals")
    return vals, vals_offset


def _compact_vals_packed(dense: Tensor, tile_bitmasks: Tensor, tile_prefix: Tensor,
                         vals: Tensor | None, vals_offset: Tensor | None,
                         M: int, N: int, num_tiles: int) -> tuple[Tensor, Tensor]:
    bits = bits_per_value(dense.dtype)
    if vals is None:
        nnz = int(tile_prefix[-1].item())
        vals = torch.empty(packed_storage_nbytes(nnz, bits), device=dense.device, dtype=torch.uint8)
        vals_offset = torch.zeros((), device=dense.device, dtype=torch.int64)
        staging = torch.empty(max(nnz, 1), device=dense.device, dtype=dense.dtype)
        count, count_t = nnz, None
    else:
        if vals.dtype != torch.uint8:
            raise TypeError("compact_vals(pack_sbit=True): storage must be the uint8 packed stream")
        # values of tiles [0, num_tiles) are prefix[num_tiles] - prefix[0] <= M*N
        staging = torch.empty(max(M * N, 1), device=dense.device, dtype=dense.dtype)
        count, count_t = M * N, tile_prefix[num_tiles:num_tiles + 1]
    L = _lib.load()
    check(L.bs_compact_vals(dense.data_ptr(), dtype_code(dense.dtype), M, N,
                            tile_bitmasks.data_ptr(), tile_prefix.data_ptr(),
                            staging.data_ptr(), staging.numel(), None, 0, num_tiles,
                            None, stream_handle(dense.device)), "bs_compact_vals")
    pack_bits(staging, vals, vals_offset, count, count_t)
    return vals, vals_offset


def compress_into(dense: Tensor, bitmask: Tensor, prefix: Tensor, vals: Tensor | None,
                  vals_offset_in: Tensor | None, vals_offset_out: Tensor | None,
                  err_flags: Tensor | None, write_vals: bool = True,
                  quantize: bool = False, scale_out: Tensor | None = None,
                  dense_q_out: Tensor | None = None, amax_epoch: int = 0,
                  relu: bool = False, relu_out: Tensor | None = None,
                  relu_square_k: float | None = None) -> None:
    """Single-pass compress (bitmask + prefix + values in one read of dense).

    ``quantize``: dense is bf16 and is quantized to e4m3fn with the scale of
    the amax computed by ``amax_into_workspace`` under ``amax_epoch``.
    ``relu``: dense is a pre-activation z and relu(z) is compressed (fused
    ReLU); ``relu_out`` (may be ``dense`` itself) receives relu(z), or with
    ``relu_square_k`` = k (bs_compress_relu2: bf16 z, values into a buffer,
    relu_out required) the ReLU^2 layer's bf16(bf16(r * r) * k), r = relu(z)."""
    require_device(dense, "compress")
    _contig(dense, "dense")
    M, N = dense.shape
    L = _lib.load()
    ws = _lib.workspace_for(dense.device)
    ws.ensure(L.bs_compress_workspace_bytes(M, N))
    epoch = ws.next_epoch()
    cap = vals.numel() if (vals is not None and write_vals) else 0
    args = (dense.data_ptr(), dtype_code(dense.dtype), M, N, int(quantize),
            ws.amax_slot_ptr() if quantize else None, amax_epoch, ptr(scale_out), ptr(dense_q_out),
            bitmask.data_ptr(), prefix.data_ptr(),
            ptr(vals) if write_vals else None, cap, ptr(vals_offset_in), 0,
            ptr(vals_offset_out), None, int(write_vals), ptr(err_flags),
            ws.buf.data_ptr(), ws.nbytes, epoch)
    if relu:
        if relu_out is not None and (relu_out.shape != dense.shape or relu_out.dtype != dense.dtype
                                     or not relu_out.is_contiguous()):
            raise ValueError("compress: relu_out must be a contiguous tensor like dense")
        if relu_square_k is not None:
            if relu_out is None or not write_vals:
                raise ValueError("compress: the ReLU^2 write-back needs relu_out and a value buffer")
            check(L.bs_compress_relu2(dense.data_ptr(), int(quantize), M, N,
                                      ws.amax_slot_ptr() if quantize else None, amax_epoch, ptr(scale_out),
                                      ptr(dense_q_out), bitmask.data_ptr(), prefix.data_ptr(), ptr(vals), cap,
                                      ptr(vals_offset_in), ptr(vals_offset_out), ptr(err_flags),
                                      ws.buf.data_ptr(), ws.nbytes, epoch, ptr(relu_out), float(relu_square_k),
                                      stream_handle(dense.device)), "bs_compress_relu2")
            return
        check(L.bs_compress_relu(*args, ptr(relu_out), stream_handle(dense.device)), "bs_compress_relu")
    else:
        check(L.bs_compress(*args, stream_handle(dense.device)), "bs_compress")


# Look-back patience of the fused up-projection in s_memrealtime ticks
# (100 MHz); -1: the library's default (20 ms); 0: every unit but the first
# gives up at once (a test hook: the time-out path with every wave ending).
UP_LOOKBACK_PATIENCE_TICKS = -1


def linear_relu_compress_into(x: Tensor, W: Tensor, bias: Tensor | None, h_out: Tensor | None,
                              bitmask: Tensor, prefix: Tensor, vals: Tensor,
                              vals_offset_in: Tensor | None, vals_offset_out: Tensor | None,
                              err_flags: Tensor | None, timeout_flag: Tensor | int | None = None) -> None:
    """h = relu(x @ W.T + bias) with its compressed form, in one kernel
    (bs_linear_relu_compress): x [M, K], W [N, K], bias [N] (or None), bf16,
    rows contiguous; h_out (or None) [M, N] bf16 receives h; bitmask / prefix /
    vals / cursors as for ``compress_into`` (bf16 values); ``timeout_flag``
    (a zeroed int32 device tensor, the device address of a zeroed pinned host
    word from ``host_device_pointer``, or None) is set to 1 if a look-back
    wait gave up, in which case the compressed form is wrong."""
    require_device(x, "linear_relu_compress")
    for t, what in ((x, "x"), (W, "W")):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"linear_relu_compress: {what} must be a bf16 matrix with contiguous rows")
    M, K = x.shape
    N = W.shape[0]
    if W.shape[1] != K:
        raise ValueError("linear_relu_compress: x and W disagree on K")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != N or not bias.is_contiguous()):
        raise ValueError("linear_relu_compress: bias must be a contiguous bf16 [N]")
    if h_out is not None and (h_out.shape != (M, N) or h_out.dtype != torch.bfloat16 or h_out.stride(1) != 1):
        raise ValueError("linear_relu_compress: h_out must be a bf16 [M, N] matrix with contiguous rows")
    if vals.dtype != torch.bfloat16:
        raise TypeError("linear_relu_compress: the values are bf16")
    L = _lib.load()
    ws = _lib.workspace_for(x.device)
    ws.ensure(L.bs_compress_workspace_bytes(M, N))
    epoch = ws.next_epoch()
    check(L.bs_linear_relu_compress(x.data_ptr(), M, K, x.stride(0), W.data_ptr(), N, W.stride(0), ptr(bias),
                                    ptr(h_out), h_out.stride(0) if h_out is not None else N,
                                    bitmask.data_ptr(), prefix.data_ptr(), vals.data_ptr(), vals.numel(),
                                    ptr(vals_offset_in), 0, ptr(vals_offset_out), None, ptr(err_flags),
                                    timeout_flag if isinstance(timeout_flag, int) else ptr(timeout_flag),
                                    int(UP_LOOKBACK_PATIENCE_TICKS),
                                    ws.buf.data_ptr(), ws.nbytes, epoch, stream_handle(x.device)),
          "bs_linear_relu_compress")


def host_device_pointer(t: Tensor) -> int:
    """Device address of a pinned host tensor's storage (bs_host_device_pointer),
    for flags a kernel stores into directly; raises if the memory is not
    mapped for the device."""
    if not t.is_pinned():
        raise ValueError("host_device_pointer: the tensor must be in pinned host memory")
    out = ctypes.c_void_p()
    check(_lib.load().bs_host_device_pointer(t.data_ptr(), ctypes.byref(out)), "bs_host_device_pointer")
    return int(out.value)


_UP_MAX_N: dict[int, int] = {}


def linear_relu_compress_max_n(device: torch.device) -> int:
    """Largest N the fused up-projection takes on ``device`` (its strips'
    workgroups must be co-resident: half of what the device holds)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _UP_MAX_N:
        n = int(_lib.load().bs_linear_relu_compress_max_n(idx))
        _UP_MAX_N[idx] = max(n, 0)
    return _UP_MAX_N[idx]


def linear_relu_compress_supported(x: Tensor, W: Tensor, bias: Tensor | None) -> bool:
    """Whether bs_linear_relu_compress takes these operands as they are."""
    if x.dim() != 2 or W.dim() != 2 or x.dtype != torch.bfloat16 or W.dtype != torch.bfloat16:
        return False
    M, K = x.shape
    N = W.shape[0]
    if M == 0 or N == 0 or K % 8 or N % 8 or not x.is_cuda or N > linear_relu_compress_max_n(x.device):
        return False
    for t in (x, W):
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
            return False
    if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous() or bias.numel() != N):
        return False
    return True


def compress_packed_into(dense: Tensor, bitmask: Tensor, prefix: Tensor, stream: Tensor,
                         vals_offset_in: Tensor | None, vals_offset_out: Tensor | None,
                         vals_start_out: Tensor | None, err_flags: Tensor | None,
                         quantize: bool = False, scale_out: Tensor | None = None,
                         dense_q_out: Tensor | None = None, amax_epoch: int = 0,
                         relu: bool = False, relu_out: Tensor | None = None) -> None:
    """Single-pass compress straight into a 15/7-bit packed stream (uint8
    storage) at the cursor rounded up to a multiple of 8 values.  Options as
    for ``compress_into``; ``vals_start_out`` receives the aligned start."""
    require_device(dense, "compress_packed")
    _contig(dense, "dense")
    if stream.dtype != torch.uint8:
        raise TypeError("compress_packed: the stream storage is uint8")
    if relu_out is not None and (relu_out.shape != dense.shape or relu_out.dtype != dense.dtype
                                 or not relu_out.is_contiguous()):
        raise ValueError("compress_packed: relu_out must be a contiguous tensor like dense")
    M, N = dense.shape
    L = _lib.load()
    ws = _lib.workspace_for(dense.device)
    ws.ensure(L.bs_compress_workspace_bytes(M, N))
    epoch = ws.next_epoch()
    check(L.bs_compress_packed(dense.data_ptr(), dtype_code(dense.dtype), M, N, int(quantize),
                               ws.amax_slot_ptr() if quantize else None, amax_epoch, ptr(scale_out),
                               ptr(dense_q_out), bitmask.data_ptr(), prefix.data_ptr(),
                               stream.data_ptr(), stream.numel(), ptr(vals_offset_in),
                               ptr(vals_offset_out), ptr(vals_start_out), ptr(err_flags),
                               ws.buf.data_ptr(), ws.nbytes, epoch, int(relu), ptr(relu_out),
                               stream_handle(dense.device)), "bs_compress_packed")


def amax_into_workspace(x: Tensor, relu: bool = False, reserve: int = 2) -> int:
    """amax(|x|) (``relu``: amax of relu(x)) of a bf16 tensor into the
    stream's workspace; returns the epoch that tags it.  ``reserve``: the
    epochs the caller's sequence takes from here (this one included)."""
    require_device(x, "amax")
    _contig(x, "x")
    if x.dtype != torch.bfloat16:
        raise TypeError("amax expects a bfloat16 tensor")
    L = _lib.load()
    ws = _lib.workspace_for(x.device)
    ws.ensure(256)
    epoch = ws.next_epoch(reserve=reserve)   # the compress that reads this amax takes the next one
    fn = L.bs_amax_relu if relu else L.bs_amax
    check(fn(x.data_ptr(), x.numel(), ws.buf.data_ptr(), ws.nbytes, epoch,
             stream_handle(x.device)), "bs_amax")
    return epoch


def amax_relu2_from(device: torch.device, epoch_in: int, k: float) -> int:
    """amax|bf16(bf16(r * r) * k)| from the amax|r| of ``epoch_in`` (r = relu(z),
    bs_amax_relu2_from) into the stream's workspace; returns the epoch that
    tags it.  k must be finite."""
    L = _lib.load()
    ws = _lib.workspace_for(device)
    epoch = ws.next_epoch()
    check(L.bs_amax_relu2_from(ws.buf.data_ptr(), ws.nbytes, epoch_in, epoch, float(k), stream_handle(device)),
          "bs_amax_relu2_from")
    return epoch


def relu2_square_amax_(h: Tensor, k: float) -> int:
    """h <- bf16(bf16(h * h) * k) in place (torch's h.square_(); h.mul_(k))
    and amax|h| into the stream's workspace; returns the epoch that tags it
    (quantize_e4m3fn(h, epoch) is then to_fp8(h))."""
    require_device(h, "relu2_square_amax_")
    _contig(h, "h")
    if h.dtype != torch.bfloat16:
        raise TypeError("relu2_square_amax_ expects a bfloat16 tensor")
    L = _lib.load()
    ws = _lib.workspace_for(h.device)
    ws.ensure(256)
    epoch = ws.next_epoch(reserve=2)
    check(L.bs_relu2_square_amax(h.data_ptr(), h.numel(), float(k), ws.buf.data_ptr(), ws.nbytes, epoch,
                                 stream_handle(h.device)), "bs_relu2_square_amax")
    return epoch


def quantize_e4m3fn(x: Tensor, amax_epoch: int) -> tuple[Tensor, Tensor]:
    """(e4m3fn tensor, fp32 0-d scale) from the amax of ``amax_epoch``."""
    L = _lib.load()
    ws = _lib.workspace_for(x.device)
    q = torch.empty(x.shape, device=x.device, dtype=torch.float8_e4m3fn)
    scale = torch.empty((), device=x.device, dtype=torch.float32)
    check(L.bs_quantize_e4m3fn(x.data_ptr(), x.numel(), q.data_ptr(), scale.data_ptr(),
                               ws.buf.data_ptr(), ws.nbytes, amax_epoch,
                               stream_handle(x.device)), "bs_quantize_e4m3fn")
    return q, scale


def transpose_u8(x: Tensor, out: Tensor | None = None) -> Tensor:
    """x.T as a new row-major tensor for a 2-D row-major 1-byte tensor (fp8,
    uint8) through bs_transpose_u8: the fp8 GEMM operands' layout change
    (reference fp8.py:36-43, :111).  Needs x.shape[1] % 16 == 0 and
    x.shape[0] % 4 == 0 (``transpose_u8_supported``)."""
    if x.dim() != 2 or x.element_size() != 1 or x.stride(1) != 1:
        raise ValueError("transpose_u8 expects a row-major 2-D tensor of 1-byte elements")
    R, C = x.shape
    if out is None:
        out = torch.empty((C, R), device=x.device, dtype=x.dtype)
    if out.shape != (C, R) or out.stride(1) != 1 or out.element_size() != 1:
        raise ValueError("transpose_u8: out must be a row-major [C, R] 1-byte tensor")
    L = _lib.load()
    check(L.bs_transpose_u8(x.data_ptr(), R, C, x.stride(0), out.data_ptr(), out.stride(0),
                            stream_handle(x.device)), "bs_transpose_u8")
    return out


def transpose_u8_supported(x: Tensor) -> bool:
    return (x.dim() == 2 and x.element_size() == 1 and x.stride(1) == 1 and x.shape[1] % 16 == 0 and
            x.shape[0] % 4 == 0 and x.stride(0) % 16 == 0 and x.data_ptr() % 16 == 0)


def widen_e4m3fn(x: Tensor) -> Tensor:
    """bf16 copy of an e4m3fn tensor (exact; NaN -> 0x7fc0 as torch's cast)
    through bs_widen_e4m3fn, in x's layout when x is row-major or a
    transposed view of row-major storage."""
    if x.dtype != torch.float8_e4m3fn:
        raise TypeError("widen_e4m3fn expects a float8_e4m3fn tensor")
    if x.dim() == 2 and not x.is_contiguous() and x.t().is_contiguous():
        return widen_e4m3fn(x.t()).t()
    x = x.contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=torch.bfloat16)
    if x.data_ptr() % 16 != 0:
        return x.to(torch.bfloat16)
    L = _lib.load()
    check(L.bs_widen_e4m3fn(x.data_ptr(), x.numel(), out.data_ptr(), stream_handle(x.device)),
          "bs_widen_e4m3fn")
    return out


def row_major_bytes(x: Tensor) -> Tensor:
    """A 2-D 1-byte tensor in row-major layout: x itself when it is, the
    transpose kernel's copy when x is a transposed view of row-major storage
    of supported shape, torch's copy otherwise."""
    if x.is_contiguous():
        return x
    if x.dim() == 2 and x.stride(0) == 1 and transpose_u8_supported(x.t()):
        return transpose_u8(x.t())
    return x.contiguous()


# ---------------------------------------------------------------------------
# decompress
# ---------------------------------------------------------------------------
def _unpack(sparse: BitsparseTensor, output: Tensor, first_m_tile: int, grid_n: int, K: int,
            batch_rows: int, num_tiles_in_batch: int, square: bool, scale: Tensor | None) -> Tensor:
    require_device(output, "unpack")
    _contig(output, "output")
    stored = sparse.dtype if sparse.pack_sbit else sparse.vals.dtype
    want = torch.bfloat16 if square else stored
    if output.dtype != want:
        raise TypeError(f"unpack: output dtype {output.dtype}, expected {want}")
    if output.numel() < batch_rows * K:
        raise ValueError("unpack: output smaller than batch_rows x K")
    if first_m_tile + (num_tiles_in_batch + grid_n - 1) // grid_n > sparse.grid_m:
        raise ValueError("unpack: tile batch runs past the tile grid")
    L = _lib.load()
    fn = L.bs_decompress_packed if sparse.pack_sbit else L.bs_decompress
    check(fn(sparse.vals.data_ptr(), dtype_code(stored), sparse.vals.numel(),
             sparse.bitmask.data_ptr(), sparse.prefix.data_ptr(),
             sparse.vals_offset.data_ptr(), output.data_ptr(), first_m_tile, grid_n, K,
             batch_rows, num_tiles_in_batch, int(square), float(RELU2_SCALE),
             ptr(scale), stream_handle(output.device)), "bs_decompress")
    return output


def unpack_batch_(
    sparse: BitsparseTensor, output: Tensor,
    first_m_tile: int, grid_n: int, K: int, batch_rows: int,
    num_tiles_in_batch: int,
) -> Tensor:
    """Unpack a row batch of tiles into a dense [batch_rows, K] output in the
    stored dtype (in place).  Reference: triton_operators.py:118-138."""
    return _unpack(sparse, output, first_m_tile, grid_n, K, batch_rows, num_tiles_in_batch,
                   False, None)


def unpack_relu2_batch_(
    sparse: BitsparseTensor, output: Tensor,
    first_m_tile: int, grid_n: int, K: int, batch_rows: int,
    num_tiles_in_batch: int,
) -> Tensor:
    """Unpack stored r = relu(a) as k * r^2 into a bf16 output (in place),
    times scale^2 for fp8 storage.  Reference: triton_operators.py:141-162."""
    return _unpack(sparse, output, first_m_tile, grid_n, K, batch_rows, num_tiles_in_batch,
                   True, sparse.scale)


# ---------------------------------------------------------------------------
# gradients
# ---------------------------------------------------------------------------
def _check_grad(grad: Tensor, sparse: BitsparseTensor, what: str) -> None:
    require_device(grad, what)
    _contig(grad, "grad")
    if grad.dtype != torch.bfloat16:
        raise TypeError(f"{what}: grad must be bfloat16")
    if tuple(grad.shape) != tuple(sparse.shape):
        raise ValueError(f"{what}: grad shape {tuple(grad.shape)} != {tuple(sparse.shape)}")


def mask_with_bitmask_(grad: Tensor, sparse: BitsparseTensor) -> Tensor:
    """grad <- grad * bitmask, in place.  Reference: triton_operators.py:165-175."""
    _check_grad(grad, sparse, "mask_with_bitmask_")
    M, N = sparse.shape
    L = _lib.load()
    check(L.bs_relu_grad(grad.data_ptr(), M, N, sparse.bitmask.data_ptr(),
                         stream_handle(grad.device)), "bs_relu_grad")
    return grad


def relu2_grad_sparse_(grad: Tensor, sparse_z: BitsparseTensor) -> Tensor:
    """grad <- grad * 2k*r where set, 0 elsewhere, then * scale for fp8
    storage, in place.  Reference: triton_operators.py:178-202."""
    _check_grad(grad, sparse_z, "relu2_grad_sparse_")
    M, N = sparse_z.shape
    L = _lib.load()
    stored = sparse_z.dtype if sparse_z.pack_sbit else sparse_z.vals.dtype
    fn = L.bs_relu2_grad_packed if sparse_z.pack_sbit else L.bs_relu2_grad
    check(fn(grad.data_ptr(), M, N, sparse_z.vals.data_ptr(), dtype_code(stored),
             sparse_z.vals.numel(), sparse_z.bitmask.data_ptr(), sparse_z.prefix.data_ptr(),
             sparse_z.vals_offset.data_ptr(), float(RELU2_SCALE), ptr(sparse_z.scale),
             stream_handle(grad.device)), "bs_relu2_grad")
    return grad
