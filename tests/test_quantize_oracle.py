"""Pins of the oracle's bit packing for every MLX width and of its affine
quantizer (CPU only).

MLX's quantizer source is not in the reference (only its call sites are:
mlxturbo/rebit.py:119, kernels/moe_verify_gather.py:887), so
``oracle.quantize`` is checked against what the mathematics of an affine
code fixes, independently of how the oracle computes it:

* exact affine grids round-trip bit for bit (codes, scale, bias and the
  dequantized values), for both sign orientations of the scale;
* points placed a known fraction of a step off the grid get the
  round-half-to-even code;
* a group whose range does not divide its dominant edge gets the edge-exact
  scale ``edge / round(edge / scale0)`` (hand-derived value) and the edge
  maps to code 0;
* constant and all-zero groups decode to themselves;
* on Gaussian data every code is within half a step of its value, and a
  clipped far end within ``n_bins * |scale - range/n_bins|`` (the most the
  edge snap can move the far end; ranges computed here in float64).

``test_quantize_checks_reject_planted_mistakes`` runs the same checks on
quantizers with one planted mistake each and requires every one to fail.
MLX's exact conventions at the edges this cannot see (e.g. how a tie
between |min| and |max| picks the sign) stay unpinned.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O


# ----------------------------------------------------------------- packing

def _ref_decode(byte_rows: np.ndarray, bits: int) -> np.ndarray:
    """Decode packed bytes with the reference's per-code formulas
    (_steel_flat.py:1184-1254), one byte group at a time."""
    out = []
    for row in byte_rows:
        r = [int(v) for v in row]
        codes = []
        if bits == 2:
            for w in r:
                codes += [w & 0x03, (w & 0x0C) >> 2, (w & 0x30) >> 4, (w & 0xC0) >> 6]
        elif bits == 3:
            for i in range(0, len(r), 3):
                w = r[i:i + 3]
                codes += [w[0] & 0x7, (w[0] & 0x38) >> 3,
                          ((w[0] & 0xC0) >> 6) + ((w[1] & 0x1) << 2), (w[1] & 0xE) >> 1,
                          (w[1] & 0x70) >> 4, ((w[1] & 0x80) >> 7) + ((w[2] & 0x3) << 1),
                          (w[2] & 0x1C) >> 2, (w[2] & 0xE0) >> 5]
        elif bits == 4:
            for w in r:
                codes += [w & 0x0F, (w & 0xF0) >> 4]
        elif bits == 5:
            for i in range(0, len(r), 5):
                w = r[i:i + 5]
                codes += [w[0] & 0x1F, ((w[0] & 0xE0) >> 5) + ((w[1] & 0x3) << 3),
                          (w[1] & 0x7C) >> 2, ((w[1] & 0x80) >> 7) + ((w[2] & 0xF) << 1),
                          ((w[2] & 0xF0) >> 4) + ((w[3] & 0x1) << 4), (w[3] & 0x3E) >> 1,
                          ((w[3] & 0xC0) >> 6) + ((w[4] & 0x7) << 2), (w[4] & 0xF8) >> 3]
        elif bits == 6:
            for i in range(0, len(r), 3):
                w = r[i:i + 3]
                codes += [w[0] & 0x3F, ((w[0] >> 6) & 0x03) + ((w[1] & 0x0F) << 2),
                          ((w[1] >> 4) & 0x0F) + ((w[2] & 0x03) << 4), (w[2] >> 2) & 0x3F]
        elif bits == 8:
            codes += r
        out.append(codes)
    return np.array(out, dtype=np.uint32)


@pytest.mark.parametrize("bits", O.BITS)
def test_unpack_matches_reference_decode(bits):
    """Random words decode identically through the oracle's bitstream and
    through the reference's per-width formulas; pack inverts unpack."""
    rng = np.random.default_rng(bits)
    K = 96 if bits in (3, 5, 6) else 64          # whole words and whole byte groups
    w = rng.integers(0, 2**32, size=(5, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    byte_rows = w.view(np.uint8).reshape(5, -1)   # little-endian bytes of each row
    ref = _ref_decode(byte_rows, bits)
    np.testing.assert_array_equal(O.unpack(w, bits), ref)
    np.testing.assert_array_equal(O.pack(ref, bits), w)


def test_pack_known_words():
    # 3-bit codes 0..7 -> bits 000 001 010 011 100 101 110 111 (lowest first)
    # = 0b111_110_101_100_011_010_001_000 = 0xFAC688 in the first 3 bytes
    w = O.pack(np.tile(np.arange(8), 4)[None], 3)
    assert w.shape == (1, 3)
    assert int(w[0, 0]) & 0xFFFFFF == 0xFAC688
    # 6-bit: codes 1, 2, 3, 63 -> 000001 000010 000011 111111
    w6 = O.pack(np.array([[1, 2, 3, 63] * 4]), 6)
    assert int(w6[0, 0]) & 0xFFFFFF == (1 | 2 << 6 | 3 << 12 | 63 << 18)
    # 5-bit: code 31 at index 1 occupies bits 5..9
    c5 = np.zeros((1, 32), dtype=np.int64)
    c5[0, 1] = 31
    assert int(O.pack(c5, 5)[0, 0]) == 31 << 5


# ------------------------------------------------------------ quantize pins

def _grid_case(rng, bits, gs, orient, dtype):
    """Groups lying exactly on an affine grid.  orient 'min': |min| > |max|
    (MLX keeps a positive scale, bias = min); 'max': |max| >= |min| (negative
    scale, bias = max, codes counted down from the max)."""
    nb = (1 << bits) - 1
    G = 6
    s = np.float32(2.0 ** -7) if bits == 8 else np.float32(3 * 2.0 ** -9)
    codes = rng.integers(0, nb + 1, size=(G, gs))
    codes[:, 0], codes[:, 1] = 0, nb                      # both ends present
    if orient == "min":
        q0 = -(nb // 2) - 1 - rng.integers(0, nb // 2 + 1, size=G)   # |q0| > nb/2
        w = (q0[:, None] + codes) * s
        exp_scale = np.full(G, s, np.float32)
        exp_bias = (q0 * s).astype(np.float32)
        exp_codes = codes
    else:
        p = nb // 2 + 1 + rng.integers(0, nb // 2 + 1, size=G)       # p >= nb/2
        w = (p[:, None] - codes) * s
        exp_scale = np.full(G, -s, np.float32)
        exp_bias = (p * s).astype(np.float32)
        exp_codes = codes
    w = w.astype(np.float32).reshape(1, G * gs)
    if dtype != "float32":
        # every value is exact in the 16-bit type (at most 8 significant bits)
        back = O.to_f32(O.from_f32(w, dtype), dtype)
        assert np.array_equal(back, w)
    return w, exp_codes.reshape(1, -1), exp_scale[None], exp_bias[None]


def _check_grid(qfn, fails):
    rng = np.random.default_rng(11)
    for bits in O.BITS:
        for gs in (32, 64, 128):
            for orient in ("min", "max"):
                for dtype in ("float32", "bfloat16", "float16"):
                    w, codes, sc, bi = _grid_case(rng, bits, gs, orient, dtype)
                    tag = f"grid b{bits} g{gs} {orient} {dtype}"
                    try:
                        wq, s, b = qfn(w, gs, bits, dtype)
                        got = O.unpack(wq, bits)
                    except Exception as exc:          # noqa: BLE001 (a mutant may raise)
                        fails.append(f"{tag}: raised {exc!r}")
                        continue
                    if not np.array_equal(got, codes):
                        fails.append(f"{tag}: codes")
                    if not np.array_equal(O.to_f32(s, dtype), O.to_f32(O.from_f32(sc, dtype), dtype)):
                        fails.append(f"{tag}: scales")
                    if not np.array_equal(O.to_f32(b, dtype), O.to_f32(O.from_f32(bi, dtype), dtype)):
                        fails.append(f"{tag}: biases")
                    deq = O.to_f32(O.dequantize(wq, s, b, gs, bits, dtype), dtype)
                    if not np.array_equal(deq, w):
                        fails.append(f"{tag}: dequantized values")


def _check_rounding(qfn, fails):
    """Values a fraction f of a step above grid code q get rint(q + f):
    f = 0.25 -> q, 0.75 -> q + 1, 0.5 -> the even one of q, q + 1."""
    s = np.float32(2.0 ** -6)
    nb = 15
    q0 = -12                                             # |min| dominant, bias = q0 s
    q = np.array([0, nb] + [2, 3, 4, 5, 6, 7, 8, 9] * 3)
    f = np.array([0, 0] + [0.25] * 8 + [0.75] * 8 + [0.5] * 8)
    w = ((q0 + q + f) * s).astype(np.float32)
    want = np.array([0, nb] + [2, 3, 4, 5, 6, 7, 8, 9] + [3, 4, 5, 6, 7, 8, 9, 10]
                    + [2, 4, 4, 6, 6, 8, 8, 10])
    w = np.concatenate([w, np.full(32 - w.size, q0 * s, np.float32)])[None]
    want = np.concatenate([want, np.zeros(32 - want.size, dtype=want.dtype)])[None]
    try:
        wq, _, _ = qfn(w, 32, 4, "float32")
        got = O.unpack(wq, 4)
    except Exception as exc:                              # noqa: BLE001
        fails.append(f"rounding: raised {exc!r}")
        return
    if not np.array_equal(got, want):
        fails.append(f"rounding: codes {got[0, :26].tolist()} != {want[0, :26].tolist()}")


def _check_edge_snap(qfn, fails):
    """min -1, max 0.55, 4 bits: range/15 = 0.10333 would not land -1 on a
    code; the edge-exact scale is -1 / round(-1 / 0.10333) = -1 / -10 = 0.1
    (float32(0.1)), bias -1, and the far end 0.55 clips to code 15."""
    w = np.zeros((1, 32), np.float32)
    w[0, 0], w[0, 1], w[0, 2] = -1.0, 0.55, 0.0
    try:
        wq, s, b = qfn(w, 32, 4, "float32")
        codes = O.unpack(wq, 4)
    except Exception as exc:                              # noqa: BLE001
        fails.append(f"edge snap: raised {exc!r}")
        return
    if float(s[0, 0]) != float(np.float32(0.1)):
        fails.append(f"edge snap: scale {float(s[0, 0])!r} != float32(0.1)")
    if float(b[0, 0]) != -1.0:
        fails.append(f"edge snap: bias {float(b[0, 0])!r} != -1")
    if codes[0, 0] != 0 or codes[0, 1] != 15 or codes[0, 2] != 10:
        fails.append(f"edge snap: codes {codes[0, :3].tolist()} != [0, 15, 10]")


def _check_constant_groups(qfn, fails):
    w = np.zeros((2, 64), np.float32)
    w[1, :] = 0.3
    for dtype in ("float32", "bfloat16"):
        wv = O.to_f32(O.from_f32(w, dtype), dtype)
        try:
            wq, s, b = qfn(wv, 64, 4, dtype)
            codes = O.unpack(wq, 4)
        except Exception as exc:                          # noqa: BLE001
            fails.append(f"constant {dtype}: raised {exc!r}")
            continue
        deq = O.to_f32(O.dequantize(wq, s, b, 64, 4, dtype), dtype)
        if not np.array_equal(codes, np.zeros_like(codes)):
            fails.append(f"constant {dtype}: codes not all zero")
        if not np.array_equal(deq, wv):
            fails.append(f"constant {dtype}: group does not decode to itself")
        if not np.all(np.abs(O.to_f32(s, dtype)) < 1e-6):
            fails.append(f"constant {dtype}: scale not the 1e-7 floor")
    # a constant below half the 1e-7 floor: round(3e-8 / -1e-7) = round(-0.3) = 0,
    # so the bias is 0 (not the edge) and the group decodes to 0
    tiny = np.full((1, 64), 3e-8, np.float32)
    try:
        wq, s, b = qfn(tiny, 64, 4, "float32")
    except Exception as exc:                              # noqa: BLE001
        fails.append(f"tiny constant: raised {exc!r}")
        return
    if float(b[0, 0]) != 0.0 or not np.all(O.dequantize(wq, s, b, 64, 4, "float32") == 0.0):
        fails.append(f"tiny constant: bias {float(b[0, 0])!r}, expected 0 and a zero decode")


def _check_error_bounds(qfn, fails):
    """Gaussian groups: interior codes within half a step (plus the storage
    roundings), clipped far ends within n_bins * |scale - range/n_bins|."""
    rng = np.random.default_rng(5)
    for bits in (2, 3, 4, 8):
        nb = (1 << bits) - 1
        w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
        try:
            wq, s, b = qfn(w, 64, bits, "float32")
            codes = O.unpack(wq, bits)
        except Exception as exc:                          # noqa: BLE001
            fails.append(f"bounds b{bits}: raised {exc!r}")
            continue
        deq = O.dequantize(wq, s, b, 64, bits, "float32").astype(np.float64)
        g = w.reshape(16, 4, 64).astype(np.float64)
        rng_g = g.max(-1) - g.min(-1)                     # float64 range per group
        s64 = np.abs(s.astype(np.float64))
        snap = np.abs(s64 - rng_g / nb)                   # how far the snap moved the scale
        err = np.abs(deq - w).reshape(16, 4, 64)
        eps = 4 * np.abs(w).max() * 2.0 ** -23            # float32 arithmetic slack
        c = codes.reshape(16, 4, 64)
        half = 0.5 * s64[..., None] + eps
        clipped = nb * snap[..., None] + eps
        interior = (c > 0) & (c < nb)
        if not np.all(err[interior] <= np.broadcast_to(half, err.shape)[interior]):
            fails.append(f"bounds b{bits}: interior code off by more than half a step")
        far = ~interior
        lim = np.maximum(np.broadcast_to(half, err.shape), np.broadcast_to(clipped, err.shape))
        if not np.all(err[far] <= lim[far]):
            fails.append(f"bounds b{bits}: end code beyond the edge-snap bound")


def quantize_check_failures(qfn) -> list:
    fails: list = []
    _check_grid(qfn, fails)
    _check_rounding(qfn, fails)
    _check_edge_snap(qfn, fails)
    _check_constant_groups(qfn, fails)
    _check_error_bounds(qfn, fails)
    return fails


def test_oracle_quantize_passes_every_check():
    fails = quantize_check_failures(O.quantize)
    assert not fails, "\n".join(fails[:20])


# ------------------------------------------------------- planted mistakes

def _mutant(kind):
    """A quantizer with one planted mistake, written independently of the
    oracle (float32 numpy)."""
    def q(w_fp, gs, bits, dtype):
        w = np.asarray(w_fp, np.float32)
        g = w.reshape(*w.shape[:-1], w.shape[-1] // gs, gs)
        hi, lo = g.max(-1), g.min(-1)
        nb = np.float32((1 << bits) if kind == "nbins" else (1 << bits) - 1)
        s0 = np.maximum((hi - lo) / nb, np.float32(1e-7)).astype(np.float32)
        if kind == "no_sign":
            scale, bias = s0, lo
        else:
            neg_dom = np.abs(lo) > np.abs(hi)
            sc = np.where(neg_dom, s0, -s0).astype(np.float32)
            edge = np.where(neg_dom, lo, hi).astype(np.float32)
            if kind == "no_snap":
                scale, bias = sc, edge
            else:
                q0 = np.rint(edge / sc).astype(np.float32)
                nz = q0 != 0
                scale = np.where(nz, edge / np.where(nz, q0, np.float32(1)), sc).astype(np.float32)
                bias = edge if kind == "bias_at_zero" else np.where(nz, edge, np.float32(0))
                bias = bias.astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            r = (g - bias[..., None]) / scale[..., None]
        r = np.nan_to_num(r, nan=0.0)
        if kind == "trunc":
            r = np.floor(r)
        elif kind == "half_away":
            r = np.sign(r) * np.floor(np.abs(r) + 0.5)
        else:
            r = np.rint(r)
        top = (1 << bits) - 1
        r = np.clip(r, 0, top - 1 if kind == "clip_low" else top)
        codes = r.astype(np.uint32).reshape(w.shape)
        return O.pack(codes, bits), O.from_f32(scale, dtype), O.from_f32(bias, dtype)
    return q


@pytest.mark.parametrize("kind", ["nbins", "no_sign", "no_snap", "bias_at_zero", "trunc",
                                  "half_away", "clip_low"])
def test_quantize_checks_reject_planted_mistakes(kind):
    assert quantize_check_failures(_mutant(kind)), f"planted mistake {kind!r} went unnoticed"


def test_unmutated_mutant_passes():
    """The mutant template itself, with no mistake planted, passes: each
    failure above is due to its one planted mistake."""
    assert not quantize_check_failures(_mutant("none"))
