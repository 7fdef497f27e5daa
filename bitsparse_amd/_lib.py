"""ctypes binding of libbitsparse_hip.so (the C ABI in include/bitsparse_hip.h).

The shared library is built in-tree next to this file by
``bitsparse_amd.build.build_library()`` (or ``__graft_entry__.build()``).
There is no fallback: if the library is missing or a call fails, an
exception is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libbitsparse_hip.so"
# BITSPARSE_HIP_LIB points at another build of the same sources (tuning sweeps)
LIB_PATH = os.environ.get("BITSPARSE_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 15

BS_OK = 0
BS_ERR_INVALID = 1
BS_ERR_HIP = 2

# dtype codes == reference codec ids (lib_sparse/bitsparse.py:8-18)
DT_BF16, DT_E4M3FN, DT_E5M2 = 0, 1, 2

_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_int = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> argtypes (restype int unless listed in _RESTYPES)
_SIGNATURES = {
    "bs_last_error": [],
    "bs_abi_version": [],
    "bs_compress_workspace_bytes": [_i64, _i64],
    "bs_compress": [_vp, _int, _i64, _i64, _int, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp,
                    _int, _vp, _vp, _int, _vp, _vp, _i64, _u32, _vp],
    "bs_compress_relu": [_vp, _int, _i64, _i64, _int, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp,
                         _int, _vp, _vp, _int, _vp, _vp, _i64, _u32, _vp, _vp],
    "bs_linear_relu_compress": [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64,
                                _vp, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _u32, _vp],
    "bs_linear_relu_compress_max_n": [_int],
    "bs_host_device_pointer": [_vp, _vp],
    "bs_compress_packed": [_vp, _int, _i64, _i64, _int, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp,
                           _vp, _vp, _vp, _vp, _i64, _u32, _int, _vp, _vp],
    "bs_amax_relu": [_vp, _i64, _vp, _i64, _u32, _vp],
    "bs_tile_pack": [_vp, _int, _i64, _i64, _vp, _vp, _vp],
    "bs_prefix_from_counts": [_vp, _i64, _vp, _vp],
    "bs_compact_vals": [_vp, _int, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp],
    "bs_decompress": [_vp, _int, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _f32,
                      _vp, _vp],
    "bs_relu_grad": [_vp, _i64, _i64, _vp, _vp],
    "bs_relu2_grad": [_vp, _i64, _i64, _vp, _int, _i64, _vp, _vp, _vp, _f32, _vp, _vp],
    "bs_amax": [_vp, _i64, _vp, _i64, _u32, _vp],
    "bs_quantize_e4m3fn": [_vp, _i64, _vp, _vp, _vp, _i64, _u32, _vp],
    "bs_transpose_u8": [_vp, _i64, _i64, _i64, _vp, _i64, _vp],
    "bs_widen_e4m3fn": [_vp, _i64, _vp, _vp],
    "bs_relu2_square_amax": [_vp, _i64, ctypes.c_float, _vp, _i64, _u32, _vp],
    "bs_compress_relu2": [_vp, _int, _i64, _i64, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                          _vp, _i64, _u32, _vp, ctypes.c_float, _vp],
    "bs_amax_relu2_from": [_vp, _i64, _u32, _u32, ctypes.c_float, _vp],
    "bs_gemm_compressed_b_workspace_bytes": [_i64, _i64, _i64, _int],
    "bs_gemm_compressed_b": [_vp, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _vp, _vp, _i64, _int, _f32,
                             _vp, _vp, _vp, _i64, _vp],
    "bs_gemm_compressed_b_fp8_workspace_bytes": [_i64, _i64, _i64, _int, _int],
    "bs_gemm_compressed_b_fp8": [_vp, _vp, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _vp, _vp, _i64, _int,
                                 _f32, _vp, _vp, _vp, _vp, _i64, _vp],
    "bs_gemm_compressed_b_packed_workspace_bytes": [_i64, _i64, _i64, _int],
    "bs_gemm_compressed_b_packed": [_vp, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _vp, _vp, _i64, _int,
                                    _f32, _vp, _vp, _vp, _i64, _vp],
    "bs_gemm_compressed_b_fp8_packed": [_vp, _vp, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _vp, _vp, _i64,
                                        _int, _f32, _vp, _vp, _vp, _vp, _i64, _vp],
    "bs_pack_bits": [_vp, _int, _vp, _i64, _vp, _i64, _vp, _vp, _vp],
    "bs_decompress_packed": [_vp, _int, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int,
                             _f32, _vp, _vp],
    "bs_relu2_grad_packed": [_vp, _i64, _i64, _vp, _int, _i64, _vp, _vp, _vp, _f32, _vp, _vp],
    "bs_workspace_amax_slot": [_vp, _i64],
    "bs_workspace_fallback_counter": [_vp, _i64],
    "bs_compress_noalloc": [_vp, _int, _i64, _i64, _int, _int, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _int,
                            _vp, _vp, _int, _vp, _vp, _vp],
    "bs_compress_noalloc_max_tiles": [],
    "bs_launch_timing": [_int],
    "bs_nontemporal_min_bytes": [_i64],
    "bs_launch_timing_read": [_vp, _vp, _int, _vp],
    "bs_stream_probe": [_int, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _int, _vp],
}
_RESTYPES = {
    "bs_last_error": ctypes.c_char_p,
    "bs_compress_workspace_bytes": _i64,
    "bs_gemm_compressed_b_workspace_bytes": _i64,
    "bs_gemm_compressed_b_fp8_workspace_bytes": _i64,
    "bs_gemm_compressed_b_packed_workspace_bytes": _i64,
    "bs_compress_noalloc_max_tiles": _i64,
    "bs_linear_relu_compress_max_n": _i64,
    "bs_nontemporal_min_bytes": _i64,
    "bs_workspace_amax_slot": _vp,
    "bs_workspace_fallback_counter": _vp,
}

_lib = None
_lock = threading.Lock()


class LaunchTimer:
    """Kernel durations of this thread's compress / decompress launches,
    recorded by the library at each kernel's own start and end
    (``bs_launch_timing``), so launch gaps between kernels are not counted.

        with LaunchTimer() as t:
            ... compress / decompress calls ...
        t.times("compress")   # ms per launch, in launch order

    Leaving the block waits for the recorded kernels."""
    KINDS = {0: "compress", 1: "decompress"}
    MAX_LAUNCHES = 1 << 16

    def __enter__(self):
        check(load().bs_launch_timing(1), "bs_launch_timing")
        self.records = []
        return self

    def __exit__(self, *exc):
        L = load()
        ms = (ctypes.c_float * self.MAX_LAUNCHES)()
        kinds = (ctypes.c_int * self.MAX_LAUNCHES)()
        n = ctypes.c_int(0)
        rc = L.bs_launch_timing_read(ms, kinds, self.MAX_LAUNCHES, ctypes.byref(n))
        check(L.bs_launch_timing(0), "bs_launch_timing")
        check(rc, "bs_launch_timing_read")
        self.records = [(self.KINDS.get(kinds[i], str(kinds[i])), ms[i])
                        for i in range(min(n.value, self.MAX_LAUNCHES))]
        return False

    def times(self, kind: str) -> list:
        return [t for k, t in self.records if k == kind]


class BitsparseHipError(RuntimeError):
    """A libbitsparse_hip.so call returned an error status."""


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def load() -> ctypes.CDLL:
    """Load the in-tree library (raises if it was not built)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (hipcc --offload-arch=gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        v = L.bs_abi_version()
        if v != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {v}, expected {ABI_VERSION}; rebuild it")
        _lib = L
        return L


def check(rc: int, what: str) -> None:
    if rc != BS_OK:
        msg = load().bs_last_error().decode(errors="replace")
        if rc == BS_ERR_INVALID:
            raise ValueError(f"{what}: {msg}")
        raise BitsparseHipError(f"{what} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, what: str) -> None:
    """The HIP kernels run on ROCm device tensors only; there is no CPU path."""
    if not t.is_cuda:
        raise RuntimeError(
            f"{what}: bitsparse_amd runs on a ROCm GPU; got a tensor on {t.device}")


# ---------------------------------------------------------------------------
# per-(device, stream) workspace for the single-pass compress and the amax
# ---------------------------------------------------------------------------
_EPOCH_LIMIT = (1 << 30) - 1


class Workspace:
    """Zero-initialised device scratch with an epoch counter.

    Each compress / amax call takes a fresh epoch; status words written under
    older epochs are ignored by the kernels, so the buffer never needs
    clearing between calls.  When the epoch counter wraps the buffer is
    zeroed again.
    """

    def __init__(self, device: torch.device):
        self.device = device
        self.buf = torch.zeros(0, dtype=torch.uint8, device=device)
        self.epoch = 0

    def ensure(self, nbytes: int) -> None:
        if self.buf.numel() < nbytes:
            # grow geometrically; the old contents (amax slot, status words of
            # earlier epochs) move along and the new tail is zero, so epochs
            # already handed out stay meaningful
            size = max(nbytes, 2 * self.buf.numel(), 1 << 16)
            new = torch.zeros(size, dtype=torch.uint8, device=self.device)
            if self.buf.numel():
                new[:self.buf.numel()].copy_(self.buf)
            self.buf = new

    def next_epoch(self, reserve: int = 1) -> int:
        """A fresh epoch.  ``reserve`` = how many epochs the caller's sequence
        takes in total (the amax of a quantizing compress reserves 2), so the
        wrap -- which zeroes the buffer, amax slot included -- never falls
        between the amax and the compress that reads it."""
        if self.epoch + reserve > _EPOCH_LIMIT:
            self.buf.zero_()
            self.epoch = 0
        self.epoch += 1
        return self.epoch

    @property
    def nbytes(self) -> int:
        return self.buf.numel()

    def amax_slot_ptr(self) -> int:
        return load().bs_workspace_amax_slot(self.buf.data_ptr(), self.nbytes)

    def fallback_count(self) -> int:
        """Look-back fallbacks recorded in this workspace (synchronises)."""
        if self.buf.numel() < 12:
            return 0
        return int(self.buf[8:12].view(torch.int32).item())


_workspaces: dict[tuple[int, int], Workspace] = {}


def workspace_for(device: torch.device) -> Workspace:
    dev = device.index if device.index is not None else torch.cuda.current_device()
    key = (dev, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None:
        ws = Workspace(torch.device("cuda", dev))
        _workspaces[key] = ws
    return ws
