"""The committed golden vectors (tests/golden/, written by make_golden.py).

CPU: the oracle still produces every committed output from the committed
inputs (a change to the oracle that alters the format fails here), and the
configs[0] input regenerated from its seed hashes to the committed digests
together with its compressed form.

GPU: the HIP path produces the committed bytes from the committed inputs --
bitmask, prefix and value run (standalone and into a TensorBuffer), the packed
stream, the decompressed matrix, the ReLU^2 unpack and gradient, to_fp8 -- and
the configs[0] compress hashes to the committed digests.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, from_bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CODES = {"bf16": O.BF16, "e4m3fn": O.E4M3FN, "e5m2": O.E5M2}
TORCH = {"bf16": torch.bfloat16, "e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
FP8_SCALE = 0.0625


def _golden():
    return np.load(os.path.join(HERE, "codec_small.npz"), allow_pickle=False)


def _cases():
    with np.load(os.path.join(HERE, "codec_small.npz"), allow_pickle=False) as d:
        return sorted({k.split("/")[0] for k in d.files})


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _configs0_input() -> np.ndarray:
    g = torch.Generator().manual_seed(0)
    return bits(torch.randn((4096, 4096), generator=g, dtype=torch.float32).to(torch.bfloat16).relu())


@pytest.mark.parametrize("case", _cases())
def test_oracle_reproduces_golden(case):
    d = _golden()
    name = case.split("_")[0]
    code = CODES[name]
    x = d[f"{case}/x"]
    M, N = x.shape
    scale = None if name == "bf16" else FP8_SCALE
    bm, pf, v = O.compress(x, code)
    assert np.array_equal(bm, d[f"{case}/bitmask"]) and np.array_equal(pf, d[f"{case}/prefix"])
    assert np.array_equal(v, d[f"{case}/vals"])
    stream = np.zeros_like(d[f"{case}/stream"])
    assert np.array_equal(O.pack_bits(v, code, stream, 0), d[f"{case}/stream"])
    assert np.array_equal(O.decompress(v, code, bm, pf, M, N), d[f"{case}/decompress"])
    sq = O.decompress(v, code, bm, pf, M, N, square=True)
    if scale is not None:
        sq = O.bf16_mul_scalar_tensor(sq, float(np.float32(scale) * np.float32(scale)))
    assert np.array_equal(sq, d[f"{case}/relu2_unpack"])
    assert np.array_equal(O.relu2_grad(d[f"{case}/grad"], v, code, bm, pf, scale=scale), d[f"{case}/relu2_grad"])
    if name == "bf16":
        q, s = O.to_fp8(x)
        assert np.array_equal(q, d[f"{case}/to_fp8_q"]) and np.float32(s) == d[f"{case}/to_fp8_scale"][0]


def test_configs0_digests_cpu():
    want = json.load(open(os.path.join(HERE, "configs0_digests.json")))
    x = _configs0_input()
    assert _sha(x) == want["input"]
    bm, pf, v = O.compress_mt(x, O.BF16)
    assert v.size == want["nnz"]
    assert (_sha(bm), _sha(pf), _sha(v)) == (want["bitmask"], want["prefix"], want["vals"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", _cases())
def test_hip_reproduces_golden(dev, case):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.fp8 import to_fp8
    from bitsparse_amd.src import hip_operators as H
    from bitsparse_amd.src.functions import dense_to_tilesparse
    d = _golden()
    name = case.split("_")[0]
    dt = TORCH[name]
    x = from_bits(d[f"{case}/x"], dt).to(dev)
    M, N = x.shape
    scale = None if name == "bf16" else torch.tensor(FP8_SCALE, dtype=torch.float32, device=dev)
    nv = d[f"{case}/vals"].size
    for buf in (None, TensorBuffer(max(1, M * N) * x.element_size(), device=dev, dtype=dt)):
        sp = dense_to_tilesparse(x, scale, buf)
        assert np.array_equal(bits(sp.bitmask), d[f"{case}/bitmask"])
        assert np.array_equal(bits(sp.prefix), d[f"{case}/prefix"])
        assert np.array_equal(bits(sp.vals)[:nv], d[f"{case}/vals"])
    out = torch.empty((M, N), device=dev, dtype=dt)
    H.unpack_batch_(sp, out, 0, sp.grid_n, N, M, sp.grid_m * sp.grid_n)
    assert np.array_equal(bits(out), d[f"{case}/decompress"])
    sq = torch.empty((M, N), device=dev, dtype=torch.bfloat16)
    H.unpack_relu2_batch_(sp, sq, 0, sp.grid_n, N, M, sp.grid_m * sp.grid_n)
    assert np.array_equal(bits(sq), d[f"{case}/relu2_unpack"])
    g = from_bits(d[f"{case}/grad"], torch.bfloat16).to(dev)
    assert np.array_equal(bits(H.relu2_grad_sparse_(g, sp)), d[f"{case}/relu2_grad"])
    pk = dense_to_tilesparse(x, scale, pack_sbit=True)
    nbits = nv * O.bits_per_value(CODES[name])
    got, want = pk.vals.cpu().numpy(), d[f"{case}/stream"]
    assert np.array_equal(got[:nbits // 8], want[:nbits // 8])
    if nbits % 8:      # the last byte's bits past the run are unspecified (padding)
        keep = (1 << (nbits % 8)) - 1
        assert got[nbits // 8] & keep == want[nbits // 8] & keep
    if name == "bf16":
        q, s = to_fp8(x)
        assert np.array_equal(bits(q), d[f"{case}/to_fp8_q"])
        assert np.float32(s.item()) == d[f"{case}/to_fp8_scale"][0]


@pytest.mark.gpu
def test_configs0_digests_gpu(dev):
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import dense_to_tilesparse
    want = json.load(open(os.path.join(HERE, "configs0_digests.json")))
    x = from_bits(_configs0_input(), torch.bfloat16).to(dev)
    buf = TensorBuffer(2 * x.numel(), device=dev)
    sp = dense_to_tilesparse(x, None, buf)
    n = int(buf.offset.item())
    assert n == want["nnz"]
    assert _sha(bits(sp.bitmask)) == want["bitmask"]
    assert _sha(bits(sp.prefix)) == want["prefix"]
    assert _sha(bits(sp.vals[:n])) == want["vals"]
