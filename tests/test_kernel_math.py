"""CPU emulation of the device-side dequantization arithmetic (mq_common.h).

The HIP kernels dequantize with a bit trick: codes are masked in place into
the mantissa bits of 16-bit lanes, read as IEEE half subnormals
(q * 2^-24 or q * 2^-20), converted exactly to float and fed to one fused
multiply-add with the scale pre-multiplied by 2^24 / 2^20 (v_fma_mix_f32).
This test replays exactly those masks and shifts with numpy float16 views
and a float64 fma (exact product, one rounding to float32), and requires
the result to equal the oracle bit for bit, so a wrong mask, shift or
scale factor fails here on the CPU before any GPU run.
"""

import numpy as np
import pytest

from oracle import oracle as O


def _half_pair(v):
    """uint32 -> (low half, high half) as float64 through IEEE float16."""
    v = np.asarray(v, np.uint32)
    lo = (v & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (v >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    return lo, hi


def _fma_f32(a, s, b):
    """fma with exact product and one rounding to float32 (float64 holds the
    exact product of a 24-bit-scaled bf16 scale and a <= 8-bit code)."""
    return (a * s + b).astype(np.float32)


def emulate_deq4(w, s, b):
    """deq4_word: returns float32 values for codes k0..k7 of each word."""
    s = np.asarray(s, np.float64)
    b = np.asarray(b, np.float64)
    s24, s20 = s * 2.0**24, s * 2.0**20
    t = w >> np.uint32(8)
    h0, h1 = w & np.uint32(0x000F000F), w & np.uint32(0x00F000F0)
    h2, h3 = t & np.uint32(0x000F000F), t & np.uint32(0x00F000F0)
    (a0, a4), (a1, a5) = _half_pair(h0), _half_pair(h1)
    (a2, a6), (a3, a7) = _half_pair(h2), _half_pair(h3)
    vals = [_fma_f32(a0, s24, b), _fma_f32(a1, s20, b), _fma_f32(a2, s24, b), _fma_f32(a3, s20, b),
            _fma_f32(a4, s24, b), _fma_f32(a5, s20, b), _fma_f32(a6, s24, b), _fma_f32(a7, s20, b)]
    return np.stack(vals, axis=-1)


def emulate_deq8(w, s, b):
    s24 = np.asarray(s, np.float64) * 2.0**24
    b = np.asarray(b, np.float64)
    h0 = w & np.uint32(0x00FF00FF)
    h1 = (w >> np.uint32(8)) & np.uint32(0x00FF00FF)
    (a0, a2), (a1, a3) = _half_pair(h0), _half_pair(h1)
    return np.stack([_fma_f32(a0, s24, b), _fma_f32(a1, s24, b), _fma_f32(a2, s24, b),
                     _fma_f32(a3, s24, b)], axis=-1)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("bits", [4, 8])
def test_device_dequant_trick_matches_oracle(bits, dtype):
    rng = np.random.default_rng(20 + bits)
    N, K, gs = 64, 512, 64
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    scale = np.float32(10.0) ** rng.integers(-8, 3, (N, K // gs)).astype(np.float32)
    s = O.from_f32((rng.standard_normal((N, K // gs)) * scale).astype(np.float32), dtype)
    b = O.from_f32((rng.standard_normal((N, K // gs)) * scale * 3).astype(np.float32), dtype)
    w[0] = 0xFFFFFFFF
    per = 32 // bits
    sw = np.repeat(O.to_f32(s, dtype), gs // per, axis=1)          # per word
    bw = np.repeat(O.to_f32(b, dtype), gs // per, axis=1)
    emu = (emulate_deq4 if bits == 4 else emulate_deq8)(w, sw, bw).reshape(N, K)
    np.testing.assert_array_equal(O.from_f32(emu, dtype), O.dequantize(w, s, b, gs, bits, dtype))


def test_half_mantissa_bound():
    """A code must stay inside bits 0..9 of its half: bits 10..14 are the
    exponent.  (w & 0x0F000F00) would put codes 2 and 6 partly in the
    exponent field -- the emulation shows that form is wrong."""
    w = np.uint32(0x00000F00)                                  # code 2 = 15
    lo, _ = _half_pair(w & np.uint32(0x0F000F00))
    assert lo != 15 * 2.0**-16
    lo2, _ = _half_pair((w >> np.uint32(8)) & np.uint32(0x000F000F))
    assert lo2 == 15 * 2.0**-24
