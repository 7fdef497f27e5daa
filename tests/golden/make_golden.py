"""Writes the committed golden vectors of the BitSparse format.

Inputs are drawn on the CPU (torch.Generator().manual_seed(...), so every
machine regenerates the same bits); expected outputs come from the CPU oracle
(oracle/bitsparse_oracle.c through oracle/oracle.py), whose functions are
pinned in tests/test_oracle.py.  The files are data only (numpy .npz, no
pickles; a JSON file of SHA-256 digests):

* ``codec_small.npz``: for each tiny case -- shapes 1x1, 3x70, 65x66,
  130x129, value types bf16 / e4m3fn / e5m2 -- the input bits, the bitmask,
  prefix and value run, the packed 15 / 7-bit stream of the run, the
  decompressed matrix, the ReLU^2 unpack (k = 1, fp8 with scale^2) and the
  ReLU^2 gradient of a drawn gradient (fp8 with the scale), and for bf16 the
  e4m3fn quantization (to_fp8) with its scale;
* ``configs0_digests.json``: SHA-256 of the bitmask, prefix and value run of
  BASELINE configs[0] (4096 x 4096, X = randn fp32 seed 0 -> bf16, ReLU).

Run from the repository root: ``python tests/golden/make_golden.py``.
Reference layout followed: lib_sparse/src/triton_kernels.py:67-146 (bitmask,
prefix, values), :158-241 (unpack), :290-330 (ReLU^2 gradient),
bitpacking.py:58-117 (stream), fp8.py:123-129 (to_fp8).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

SHAPES = [(1, 1), (3, 70), (65, 66), (130, 129)]
CODES = {"bf16": O.BF16, "e4m3fn": O.E4M3FN, "e5m2": O.E5M2}
TORCH = {"bf16": torch.bfloat16, "e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
FP8_SCALE = 0.0625


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.view(torch.uint8).numpy().copy()


def small_cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for i, (M, N) in enumerate(SHAPES):
        g = torch.Generator().manual_seed(100 + i)
        pre = torch.randn((M, N), generator=g) - 0.3
        grad = _bits(torch.randn((M, N), generator=g).to(torch.bfloat16))
        for name, code in CODES.items():
            key = f"{name}_{M}x{N}"
            x = _bits(pre.to(torch.bfloat16).relu() if name == "bf16" else pre.clamp(min=-4, max=4).to(TORCH[name]))
            bm, pf, v = O.compress(x, code)
            gm, gn, T = O.tile_grid(M, N)
            b = O.bits_per_value(code)
            stream = np.zeros(((v.size * b + 7) // 8 + 11) // 4 * 4, np.uint8)
            O.pack_bits(v, code, stream, 0)
            scale = None if name == "bf16" else FP8_SCALE
            out[f"{key}/x"] = x
            out[f"{key}/bitmask"] = bm
            out[f"{key}/prefix"] = pf
            out[f"{key}/vals"] = v
            out[f"{key}/stream"] = stream
            out[f"{key}/decompress"] = O.decompress(v, code, bm, pf, M, N)
            sq = O.decompress(v, code, bm, pf, M, N, square=True)
            if scale is not None:                       # unpack_relu2_batch_: out *= scale^2 (bf16)
                sq = O.bf16_mul_scalar_tensor(sq, float(np.float32(scale) * np.float32(scale)))
            out[f"{key}/relu2_unpack"] = sq
            out[f"{key}/grad"] = grad
            out[f"{key}/relu2_grad"] = O.relu2_grad(grad, v, code, bm, pf, scale=scale)
            if name == "bf16":
                q, s = O.to_fp8(x)
                out[f"{key}/to_fp8_q"] = q
                out[f"{key}/to_fp8_scale"] = np.array([s], np.float32)
    return out


def configs0_digests() -> dict[str, str | int]:
    g = torch.Generator().manual_seed(0)
    x = _bits(torch.randn((4096, 4096), generator=g, dtype=torch.float32).to(torch.bfloat16).relu())
    bm, pf, v = O.compress_mt(x, O.BF16)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    return {"shape": [4096, 4096], "nnz": int(v.size), "input": h(x), "bitmask": h(bm),
            "prefix": h(pf), "vals": h(v)}


def main() -> None:
    np.savez_compressed(os.path.join(HERE, "codec_small.npz"), **small_cases())
    with open(os.path.join(HERE, "configs0_digests.json"), "w") as f:
        json.dump(configs0_digests(), f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
