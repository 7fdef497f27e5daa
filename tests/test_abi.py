"""C ABI of libbitsparse_hip.so on the CPU: the library loads, exports every
entry point include/bitsparse_hip.h declares, and rejects bad arguments on
the host (before any GPU work is enqueued)."""
import ctypes
import os
import re

import pytest
import torch

from bitsparse_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    txt = open(os.path.join(ROOT, "include", "bitsparse_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(bs_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    names = header_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.exported_symbols())


def test_abi_version_and_workspace_size():
    L = _lib.load()
    assert L.bs_abi_version() == _lib.ABI_VERSION
    # header + one status word per tile (+2), rounded up to 256 bytes, then the
    # quantizer's windowed code table (per sign of x: 24 exponents x 128
    # mantissas + 2 end entries; rounded up to 16 bytes)
    def want(T):
        return (256 + 8 * (T + 2) + 255) // 256 * 256 + 6160
    assert L.bs_compress_workspace_bytes(4096, 4096) == want(4096)
    assert L.bs_compress_workspace_bytes(129, 131) == want(9)
    assert L.bs_compress_workspace_bytes(0, 0) == want(0)


def test_nontemporal_threshold_round_trip():
    """bs_nontemporal_min_bytes sets the process threshold and returns the
    previous one; a negative value restores the default (192 MiB)."""
    L = _lib.load()
    prev = L.bs_nontemporal_min_bytes(12345)
    try:
        assert L.bs_nontemporal_min_bytes(-1) == 12345
        assert L.bs_nontemporal_min_bytes(7) == 192 << 20
    finally:
        L.bs_nontemporal_min_bytes(prev)


def _err():
    return _lib.load().bs_last_error().decode()


def test_invalid_arguments_rejected_on_host():
    L = _lib.load()
    fake = 0x10000   # never dereferenced: validation fails first
    # unknown dtype
    rc = L.bs_compress(fake, 7, 64, 64, 0, None, 0, None, None, fake, fake, fake, 10, None, 0,
                       None, None, 1, None, fake, 1 << 20, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "dtype" in _err()
    # quantize needs bf16
    rc = L.bs_compress(fake, 1, 64, 64, 1, fake, 1, None, None, fake, fake, fake, 10, None, 0,
                       None, None, 1, None, fake, 1 << 20, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "bf16" in _err()
    # packed stream: 4-byte alignment, non-empty input, the usual dense checks
    rc = L.bs_compress_packed(fake, 0, 64, 64, 0, None, 0, None, None, fake, fake, fake + 2, 64, None,
                              None, None, None, fake, 1 << 20, 1, 0, None, None)
    assert rc == _lib.BS_ERR_INVALID and "aligned" in _err()
    rc = L.bs_compress_packed(fake, 0, 0, 64, 0, None, 0, None, None, fake, fake, fake, 64, None,
                              None, None, None, fake, 1 << 20, 1, 0, None, None)
    assert rc == _lib.BS_ERR_INVALID and "empty" in _err()
    rc = L.bs_compress_packed(fake, 9, 64, 64, 0, None, 0, None, None, fake, fake, fake, 64, None,
                              None, None, None, fake, 1 << 20, 1, 0, None, None)
    assert rc == _lib.BS_ERR_INVALID and "dtype" in _err()
    rc = L.bs_compress_packed(fake, 0, 64, 64, 0, None, 0, None, None, fake, fake, fake, 64, None,
                              None, None, None, fake, 64, 1, 0, None, None)
    assert rc == _lib.BS_ERR_INVALID and "workspace" in _err()
    # workspace too small
    rc = L.bs_compress(fake, 0, 4096, 4096, 0, None, 0, None, None, fake, fake, fake, 10, None, 0,
                       None, None, 1, None, fake, 64, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "workspace" in _err()
    # epoch 0 is reserved for a zeroed workspace
    rc = L.bs_compress(fake, 0, 64, 64, 0, None, 0, None, None, fake, fake, fake, 10, None, 0,
                       None, None, 1, None, fake, 1 << 20, 0, None)
    assert rc == _lib.BS_ERR_INVALID and "epoch" in _err()
    # matrices of 2^32 elements or more (the uint32 prefix's range) are
    # refused by every codec / GEMM entry; the paths not yet run past 2^31
    # elements on the GPU (everything but the raw bf16 compress, bf16
    # decompress and the bf16 dW GEMM) already at 2^31
    big_m, big_n = 1 << 16, 1 << 16
    mid_m = 1 << 15                     # mid_m * big_n = 2^31
    rc = L.bs_compress(fake, 0, big_m, big_n, 0, None, 0, None, None, fake, fake, fake, 10, fake, 0,
                       fake + 64, None, 1, None, fake, 1 << 30, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "2^32" in _err()
    rc = L.bs_decompress(fake, 0, 10, fake, fake, None, fake, 0, big_n // 64, big_n, big_m, 64, 0, 1.0,
                         None, None)
    assert rc == _lib.BS_ERR_INVALID and "2^32" in _err()
    rc = L.bs_gemm_compressed_b(fake, 64, big_m, 64, 0, fake, 0, 10, fake, fake, None, big_n, 0, 1.0,
                                None, fake, fake, 1 << 30, None)
    assert rc == _lib.BS_ERR_INVALID and "2^32" in _err()
    rc = L.bs_compact_vals(fake, 0, big_m, big_n, fake, fake, fake, 10, None, 0, 1, None, None)
    assert rc == _lib.BS_ERR_INVALID and "2^32" in _err()
    for m in (big_m, mid_m):
        rc = L.bs_tile_pack(fake, 0, m, big_n, fake, fake, None)
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_compact_vals(fake, 1, m, big_n, fake, fake, fake, 10, None, 0, 1, None, None)
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()                     # e4m3fn values
        rc = L.bs_compress(fake, 0, m, big_n, 1, fake, 1, None, None, fake, fake, fake, 10, fake, 0,
                           fake + 64, None, 1, None, fake, 1 << 30, 1, None)      # quantizing
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_compress_packed(fake, 0, m, big_n, 0, None, 0, None, None, fake, fake, fake, 64, fake,
                                  fake + 64, None, None, fake, 1 << 30, 1, 0, None, None)
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_decompress(fake, 1, 10, fake, fake, None, fake, 0, big_n // 64, big_n, m, 64, 0, 1.0,
                             None, None)                                           # e4m3fn values
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_decompress(fake, 0, 10, fake, fake, None, fake, 0, big_n // 64, big_n, m, 64, 1, 1.0,
                             None, None)                                           # ReLU^2 square
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_relu_grad(fake, m, big_n, fake, None)
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_relu2_grad(fake, m, big_n, fake, 0, 10, fake, fake, None, 1.0, None, None)
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
        rc = L.bs_gemm_compressed_b(fake, 64, m, 64, 0, fake, 0, 10, fake, fake, None, big_n, 1, 1.0,
                                    None, fake, fake, 1 << 30, None)              # ReLU^2 square
        assert rc == _lib.BS_ERR_INVALID and "2^31" in _err()
    # aliasing cursors
    rc = L.bs_compress(fake, 0, 64, 64, 0, None, 0, None, None, fake, fake, fake, 10, fake + 64, 0,
                       fake + 64, None, 1, None, fake, 1 << 20, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "alias" in _err()
    # tile range of compact_vals
    rc = L.bs_compact_vals(fake, 0, 64, 64, fake, fake, fake, 10, None, 0, 2, None, None)
    assert rc == _lib.BS_ERR_INVALID and "tile range" in _err()
    # decompress geometry and scale misuse
    rc = L.bs_decompress(fake, 0, 10, fake, fake, None, fake, 0, 0, 64, 64, 1, 0, 1.0, None, None)
    assert rc == _lib.BS_ERR_INVALID
    rc = L.bs_decompress(fake, 0, 10, fake, fake, None, fake, 0, 1, 64, 64, 1, 0, 1.0, fake, None)
    assert rc == _lib.BS_ERR_INVALID and "square" in _err()
    rc = L.bs_relu2_grad(fake, 64, 64, fake, 5, 10, fake, fake, None, 1.0, None, None)
    assert rc == _lib.BS_ERR_INVALID
    rc = L.bs_amax(fake, -1, fake, 1 << 20, 1, None)
    assert rc == _lib.BS_ERR_INVALID
    rc = L.bs_host_device_pointer(None, None)
    assert rc == _lib.BS_ERR_INVALID and "null" in _err()
    # fused up-projection: a W row stride whose 192-row slab passes 2^31 bytes
    # (the 128-row x block alone would not) is refused before any launch
    ld = 5592408                                   # 128 * ld * 2 < 2^31 <= 192 * ld * 2
    rc = L.bs_linear_relu_compress(fake, 64, 64, 64, fake, 64, ld, None, None, 64, fake, fake, fake, 4096,
                                   None, 0, None, None, None, None, -1, fake, 1 << 20, 1, None)
    assert rc == _lib.BS_ERR_INVALID and "row stride" in _err()


def test_python_api_rejects_cpu_tensors_and_bad_dtypes():
    """No CPU path: the product API refuses host tensors (loudly) and
    unsupported dtypes with the reference's exception types."""
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from bitsparse_amd.fp8 import to_fp8
    with pytest.raises(TypeError):
        dense_to_tilesparse(torch.zeros(4, 4, dtype=torch.float32), None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        dense_to_tilesparse(torch.zeros(4, 4, dtype=torch.bfloat16), None)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        to_fp8(torch.zeros(4, 4, dtype=torch.bfloat16))


def test_container_helpers_match_reference_definitions():
    import numpy as np
    from bitsparse_amd.bitsparse import BitsparseTensor, TensorBuffer, bits_per_value, pack_codec, tile_grid
    from oracle import oracle as O
    from tests.helpers import bits, relu_input
    assert tile_grid(129, 131, 64, 64) == (3, 3, 9, 4096, 512)
    assert tile_grid(16384, 16384, 64, 64)[2] == 65536
    assert [pack_codec(d) for d in (torch.bfloat16, torch.float8_e4m3fn, torch.float8_e5m2)] == [0, 1, 2]
    assert [bits_per_value(d) for d in (torch.bfloat16, torch.float8_e4m3fn)] == [15, 7]
    with pytest.raises(ValueError):
        TensorBuffer(3, device="cpu", dtype=torch.bfloat16)
    # vram_size = nnz*vb + T*512 + 4*(T+1) (reference bitsparse.py:76-84), on
    # a container filled from the oracle
    x = relu_input((129, 131), 0.5, seed=0)
    bm, pf, v = O.compress(bits(x), O.BF16)
    sp = BitsparseTensor(torch.from_numpy(v.view(np.int16)).view(torch.bfloat16),
                         torch.from_numpy(bm), torch.from_numpy(pf.view(np.int32)).view(torch.uint32),
                         x.shape, torch.bfloat16, 3, 3, 64, 64)
    assert sp.vram_size() == v.size * 2 + 9 * 512 + 4 * 10
    assert int(sp.nnz()) == v.size == int((x.float() > 0).sum())
    assert not sp.fp8
    assert "BitsparseTensor" in repr(sp)


def test_lib_sparse_alias():
    import bitsparse_amd
    bitsparse_amd.install_lib_sparse_alias()
    import lib_sparse.layers as L
    from lib_sparse.src.triton_operators import unpack_batch_
    from lib_sparse.src.functions import dense_to_tilesparse
    assert L.FFNRelu is bitsparse_amd.layers.FFNRelu
    assert callable(unpack_batch_) and callable(dense_to_tilesparse)
