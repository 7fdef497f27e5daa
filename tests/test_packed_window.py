"""CPU check of the packed compress's dword construction (no GPU).

The packed compress (``stream_packed`` in bitsparse_amd/csrc/codec.hip)
builds each stream dword d of a run that starts at stream bit sb from a
64-bit window: the values v0..v1 overlapping the dword side by side (value
v0 + j at bit PB*j, at most MAXV of them: MAXV*PB <= 60), shifted right by
s0 = 32 d - (sb + v0 PB) -- or left by -s0 for the run's first dword, where
s0 is negative -- and cut to 32 bits; bits outside the run's part of the
dword are merged, not stored.  This test restates that arithmetic with
Python integers and compares every dword, for every start bit sb in [0, 32),
run lengths 1..80 and PB = 15 (bf16) / 7 (fp8), against a bit-by-bit
packer: stream bit k of value i is bit (k - i PB) of the value's low PB bits
(reference lib_sparse/src/bitpacking.py:58-117, LSB-first stream).
"""
import numpy as np
import pytest


def _bitwise_stream(vals, pb, sb, nbits):
    out = np.zeros(nbits, np.uint8)
    for i, v in enumerate(vals):
        for b in range(pb):
            out[sb + i * pb + b] = (int(v) >> b) & 1
    return out


def _kernel_dword(vals, pb, sb, cnt, d):
    """(word, mask) of dword d as the kernel forms them."""
    maxv = 4 if pb == 15 else 6
    vmask = (1 << pb) - 1
    eb = sb + cnt * pb
    lo, hi = max(d * 32, sb), min(d * 32 + 32, eb)
    v0, v1 = (lo - sb) // pb, (hi - 1 - sb) // pb
    assert v1 - v0 + 1 <= maxv and maxv * pb <= 60
    win = 0
    for j in range(maxv):
        v = v0 + j
        x = int(vals[v]) if v <= v1 else 0
        win |= (x & vmask) << (pb * j)
    assert win < (1 << 64)
    s0 = d * 32 - (sb + v0 * pb)
    assert -32 < s0 < pb                      # in [0, PB) except the first dword
    word = (win >> s0) if s0 >= 0 else ((win << -s0) & ((1 << 64) - 1))
    word &= 0xFFFFFFFF
    lb, hbit = lo - d * 32, hi - d * 32
    mask = ((1 << hbit) - 1 if hbit < 32 else 0xFFFFFFFF) & ~((1 << lb) - 1 if lb < 32 else 0xFFFFFFFF)
    return word, mask & 0xFFFFFFFF


@pytest.mark.parametrize("pb", [15, 7])
def test_window_dwords_match_bitwise_packer(pb):
    rng = np.random.default_rng(pb)
    for sb in range(32):
        for cnt in range(1, 81):
            # the sign bit set too: the kernel keeps only the low PB bits
            vals = rng.integers(0, 1 << (pb + 1), cnt)
            eb = sb + cnt * pb
            dend = (eb + 31) // 32
            bits = _bitwise_stream(vals, pb, sb, dend * 32)
            for d in range(dend):
                word, mask = _kernel_dword(vals, pb, sb, cnt, d)
                want = sum(int(bits[d * 32 + b]) << b for b in range(32))
                assert word & mask == want & mask, (pb, sb, cnt, d)
                # bits outside the mask belong to neighbouring runs
                assert mask == sum(1 << b for b in range(32) if sb <= d * 32 + b < eb)
