"""CPU check of the packed bit identities in the codec kernels (no GPU).

* ``mask_bf16x8_pk`` (bitsparse_amd/csrc/compact.h), the bitmask byte of 8
  bf16 values in the streaming compress and the fused up-projection: per
  half, ((bits + 0x807f) mod 2^16) saturating-minus 0x80 has bit 15 set
  exactly when the value is > 0 (bits in [1, 0x7f80]); v_perm selectors 8-11
  replicate bits 15 / 31 of its sources into whole bytes; two masks and a
  byte dot product with 0x01010101 gather the 8 bits.  Restated op by op and
  compared with the definition of the format's bitmask (x > 0, reference
  lib_sparse/src/triton_kernels.py:67-97) over every bf16 pattern.
* ``relu2x`` (bitsparse_amd/csrc/up_gemm.hip), torch's GPU relu on two bf16
  halves (x <= 0 -> +0, NaN kept): a half is kept iff its saturating int16
  sum with 127 is nonnegative.  Compared with that rule over every pattern.
* ``mask_fp8x8`` (bitsparse_amd/csrc/bs_device.h), the bitmask byte of 8 fp8
  codes in the quantizing and fp8 compress: per byte, bit 7 of
  (l + 0x7f) & ~(l + 0x7f - MAXP) & ~code, l = code & 0x7f; two byte dot
  products gather the 8 flags.  Compared with the format's x > 0 over every
  code in every byte position.
"""
import numpy as np
import torch

ALL = np.arange(65536, dtype=np.int64)


def _positive(bits):
    return ((bits >= 1) & (bits <= 0x7F80)).astype(np.int64)


def _pk_half(bits):
    """(bits + 0x807f) mod 2^16, then unsigned saturating minus 0x80."""
    return np.maximum(((bits + 0x807F) & 0xFFFF) - 0x80, 0)


def _perm_sign_bytes(s0, s1):
    """v_perm_b32(s0, s1, 0x0b0a0908): selector 8 + k gives 0xff or 0x00 from
    bit 15 / 31 of s1 (k = 0, 1) and of s0 (k = 2, 3)."""
    bits = [(s1 >> 15) & 1, (s1 >> 31) & 1, (s0 >> 15) & 1, (s0 >> 31) & 1]
    return sum((b * 0xFF) << (8 * k) for k, b in enumerate(bits))


def _mask_pk(chunks):
    """mask_bf16x8_pk of [n, 8] bf16 bit patterns, as the kernel forms it."""
    w = chunks[:, 0::2] | (chunks[:, 1::2] << 16)            # the 4 dwords
    u = _pk_half(w & 0xFFFF) | (_pk_half(w >> 16) << 16)
    x = _perm_sign_bytes(u[:, 1], u[:, 0])
    y = _perm_sign_bytes(u[:, 3], u[:, 2])
    z = (y & 0x80402010) | (x & 0x08040201)
    return sum((z >> (8 * k)) & 0xFF for k in range(4))      # v_dot4_u32_u8(z, 0x01010101, 0)


def test_positive_bit_of_every_pattern():
    assert (((_pk_half(ALL) >> 15) & 1) == _positive(ALL)).all()


def test_mask_byte_of_chunks():
    rng = np.random.default_rng(0)
    special = np.array([0, 0x8000, 1, 0x7F80, 0x7F81, 0x7FFF, 0xFF80, 0xFF81, 0xFFFF, 0x807F, 0x8080, 0x3F80,
                        0xBF80, 0x0080], np.int64)
    chunks = np.concatenate([rng.integers(0, 65536, (100000, 8)), rng.choice(special, (100000, 8)),
                             np.stack([np.roll(ALL, -8 * i)[:8192] for i in range(8)], 1)])
    want = sum(_positive(chunks[:, e]) << e for e in range(8))
    assert (_mask_pk(chunks) == want).all()


def test_relu_of_every_pattern():
    i16 = ALL.astype(np.uint16).view(np.int16).astype(np.int64)
    d = np.clip(i16 + 127, -32768, 32767)                    # v_pk_add_i16 ... clamp
    got = ALL & ~np.where(d < 0, 0xFFFF, 0)                  # & ~(d >> 15)
    x = torch.from_numpy(ALL.astype(np.uint16).view(np.int16)).view(torch.bfloat16).float().numpy()
    want = np.where(np.isnan(x) | (x > 0), ALL, 0)           # x <= 0 -> +0, NaN and positives keep their bits
    assert (got == want).all()


def _fp8_flags(w, maxp):
    lo = w & 0x7F7F7F7F
    return (lo + 0x7F7F7F7F) & ~(lo + (0x7F - maxp) * 0x01010101) & ~w & 0x80808080 & 0xFFFFFFFF


def _dot4(a, wts):
    return sum(((a >> (8 * k)) & 0xFF) * ((wts >> (8 * k)) & 0xFF) for k in range(4))


def test_fp8_mask_byte():
    """``mask_fp8x8`` (bitsparse_amd/csrc/bs_device.h): the byte-parallel
    positive flags of 8 fp8 codes against the format's definition (x > 0:
    codes 0x01..0x7e for e4m3fn, 0x01..0x7c for e5m2), every code in every
    byte position and random chunks."""
    b = np.arange(256, dtype=np.int64)
    rng = np.random.default_rng(1)
    v = rng.integers(0, 256, (100000, 8))
    for maxp in (0x7E, 0x7C):
        want_b = ((b >= 1) & (b <= maxp)).astype(np.int64)
        for k in range(4):
            w = (b << (8 * k)) | (0xA5 << (8 * ((k + 1) % 4)))
            assert ((_fp8_flags(w, maxp) >> (8 * k + 7)) & 1 == want_b).all()
        x0 = sum(v[:, k] << (8 * k) for k in range(4))
        x1 = sum(v[:, 4 + k] << (8 * k) for k in range(4))
        got = (_dot4(_fp8_flags(x1, maxp), 0x80402010) + _dot4(_fp8_flags(x0, maxp), 0x08040201)) >> 7
        want = sum((((v[:, e] >= 1) & (v[:, e] <= maxp)).astype(np.int64)) << e for e in range(8))
        assert (got == want).all()
