"""CPU check of the claim behind bs_amax_relu2_from: for a finite k the ReLU^2
layer's h(r) = bf16(bf16(r * r) * k) (torch's in-place h.square_() then
h.mul_(k) on bf16), with NaN as 0x7fc0, has |h| non-decreasing in r over every
non-negative bf16 r and NaN, in the order of the amax kernel's magnitude bits
(NaN above Inf).  So the amax of the squared tensor is the image of the amax
of r, which the fp8 ReLU^2 forward uses instead of a second pass over h."""
import numpy as np
import pytest
import torch

POS = np.arange(0, 0x8000, dtype=np.int64)          # every non-negative bf16 pattern, NaNs included


def _h_mag_bits(k: float) -> np.ndarray:
    r = torch.from_numpy(POS.astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    h = r.clone()
    h.square_()
    h.mul_(k)
    b = h.view(torch.int16).numpy().view(np.uint16).astype(np.int64)
    nan = (b & 0x7FFF) > 0x7F80
    b = np.where(nan, 0x7FC0, b)
    return b & 0x7FFF


@pytest.mark.parametrize("k", [1.0, 0.5, 3.0, 1e-30, 1e30, -2.0, 0.0, -0.0])
def test_relu2_magnitude_is_monotonic(k):
    m = _h_mag_bits(k)
    assert (np.diff(m) >= 0).all()


@pytest.mark.parametrize("k", [1.0, 0.25, -3.0])
def test_amax_of_square_is_square_of_amax(k):
    rng = np.random.default_rng(7)
    m = _h_mag_bits(k)
    for _ in range(200):
        sub = rng.choice(POS, size=64)
        assert m[sub].max() == m[sub.max()]
