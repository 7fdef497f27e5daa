"""Shared input generators and bit-view helpers for the tests."""
from __future__ import annotations

import numpy as np
import torch

BITS_DTYPE = {torch.bfloat16: torch.int16, torch.float8_e4m3fn: torch.uint8,
              torch.float8_e5m2: torch.uint8}


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a bf16 / fp8 tensor as uint16 / uint8 numpy."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        return t.view(torch.uint8).numpy()
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def from_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dtype == torch.bfloat16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.astype(np.uint8).copy()).view(dtype)


def relu_input(shape, sparsity: float, seed: int = 0, dtype=torch.bfloat16) -> torch.Tensor:
    """Non-negative data with about `sparsity` zeros (experiments/validate.py:18-32
    semantics, drawn on the CPU so every machine sees the same bits)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32).to(torch.bfloat16).abs_()
    zero = torch.rand(shape, generator=g) < sparsity
    x.masked_fill_(zero, 0)
    if dtype != torch.bfloat16:
        x = x.to(dtype)
    return x


def preact_input(shape, mu: float = 0.0, seed: int = 0) -> torch.Tensor:
    """Pre-activation N(mu, 1) in bf16 (negative values included)."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) + mu).to(torch.bfloat16)


def special_bf16(shape, seed: int = 0) -> torch.Tensor:
    """bf16 matrix salted with every edge case of the x > 0 test: +-0, +-denormals,
    +-Inf, NaNs of both signs, the largest finite values, negatives."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32).to(torch.bfloat16)
    b = x.view(torch.int16).numpy().view(np.uint16).copy()
    specials = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x007f, 0x807f, 0x0080,
                         0x7f80, 0xff80, 0x7fc0, 0xffc0, 0x7f81, 0x7fff, 0xffff,
                         0x7f7f, 0xff7f, 0x3f80, 0xbf80], np.uint16)
    rng = np.random.default_rng(seed)
    idx = rng.choice(b.size, size=min(b.size, 4 * specials.size), replace=False)
    b.reshape(-1)[idx] = np.resize(specials, idx.size)
    return from_bits(b, torch.bfloat16)


def all_fp8_patterns(shape, seed: int = 0) -> np.ndarray:
    """uint8 matrix cycling through all 256 fp8 bit patterns in random order."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    return rng.permutation(np.resize(np.arange(256, dtype=np.uint8), n)).reshape(shape)
