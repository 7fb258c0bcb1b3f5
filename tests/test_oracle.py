"""Pins the CPU oracle (oracle/oracle.py, oracle/qmm_oracle.c) with checks that
do not restate its formulas: hand-derived known answers, independent
implementations (torch's casts, a float64 route, pure-Python loops, the C
restatement), mathematical invariants, and planted mistakes that must fail.
"""

import struct

import numpy as np
import pytest
import torch

from oracle import cref
from oracle import oracle as O


# ------------------------------------------------------------------ packing

def test_pack_known_words():
    # nibble j of the word is element j, low bits first (fast_qmm.py:96-106)
    assert int(O.pack(np.arange(8), 4)[0]) == 0x76543210
    assert int(O.pack(np.array([1, 2, 3, 4]), 8)[0]) == 0x04030201
    assert int(O.pack(np.array([15] + [0] * 7), 4)[0]) == 0x0000000F
    assert int(O.pack(np.array([0] * 7 + [15]), 4)[0]) == 0xF0000000
    np.testing.assert_array_equal(O.unpack(np.array([0xFEDCBA98], np.uint32), 4),
                                  np.arange(8, 16))


def test_pack_matches_bitstring_construction():
    rng = np.random.default_rng(0)
    for bits in (2, 4, 8):
        codes = rng.integers(0, 1 << bits, size=(3, 64))
        words = O.pack(codes, bits)
        per = 32 // bits
        for r in range(3):
            for i in range(64 // per):
                # little-endian: the first code is the least significant field
                s = "".join(format(int(c), f"0{bits}b") for c in reversed(codes[r, i * per:(i + 1) * per]))
                assert int(words[r, i]) == int(s, 2)
        np.testing.assert_array_equal(O.unpack(words, bits), codes)


# ------------------------------------------------------------ float formats

def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-8 + 2**-20,
            3.0234375, 65504.0, 65520.0, 65519.99, 2.0**-14, 2.0**-24, 2.0**-25, 2.0**-26,
            3 * 2.0**-26, 2.0**-133, 1e-40, 3.3895314e38, 3.4e38, float("inf"), -float("inf")]
    rng = np.random.default_rng(1)
    rnd = rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-40, 38, 4000)
    bits = rng.integers(0, 2**32, 4000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    bits = bits[np.isfinite(bits)]
    return np.concatenate([np.array(vals, np.float32), rnd.astype(np.float32), bits])


def test_bf16_rounding_matches_torch():
    f = _special_f32()
    ours = O.bf16_bits(f)
    theirs = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    # and the C restatement
    c = np.array([cref.lib().oracle_round_bf16(float(v)) for v in f[:600]], np.uint16)
    np.testing.assert_array_equal(c, ours[:600])


def test_bf16_rounding_known_answers():
    # ties go to even: 1+2^-8 is halfway between 1 and 1+2^-7 -> 1.0
    assert int(O.bf16_bits(np.float32(1.0 + 2**-8))) == 0x3F80
    # 1+3*2^-8 is halfway between 1+2^-7 (odd) and 1+2^-6 (even) -> 1+2^-6
    assert int(O.bf16_bits(np.float32(1.0 + 3 * 2**-8))) == 0x3F82
    # carry into the exponent: largest value below 2 rounds to 2.0
    assert int(O.bf16_bits(np.float32(1.9999999))) == 0x4000
    assert int(O.bf16_bits(np.float32(np.inf))) == 0x7F80
    assert int(O.bf16_bits(np.float32(3.4e38))) == 0x7F80  # above bf16 max + half ulp


def test_f16_rounding_matches_torch_and_c():
    f = _special_f32()
    ours = O.f16_bits(f)
    theirs = torch.from_numpy(f).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    c = np.array([cref.lib().oracle_round_f16(float(v)) for v in f[:1500]], np.uint16)
    np.testing.assert_array_equal(c, ours[:1500])


# ------------------------------------------------------------------ dequant

def _bf16(v):
    return np.array([O.bf16_bits(np.float32(v))], np.uint16)


def test_dequant_known_answers():
    # word 0x76543210 holds codes 0..7; s=0.5, b=-1 -> 0.5*q-1, all exact in bf16
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    s = _bf16(0.5)[None, :]
    b = _bf16(-1.0)[None, :]
    # group_size 32 needs 32 codes: pad the row with zero words
    w = np.concatenate([w, np.zeros((1, 2), np.uint32)], axis=1)
    got = O.bf16_to_f32(O.dequantize(w, s, b, 32, 4, "bfloat16"))[0]
    want = [0.5 * q - 1.0 for q in range(16)] + [-1.0] * 16
    np.testing.assert_array_equal(got, np.array(want, np.float32))


def test_dequant_double_rounding_known_answer():
    """MLX rounds s*q+b to float32, then to bf16 (two roundings).

    s = 1+2^-7, q = 3: s*q = 3.0234375 sits exactly on a bf16 tie.  With
    b = -2^-40 the exact sum is just below the tie: one rounding would give
    3.015625, but float32 first rounds back onto the tie and RNE then goes
    to the even neighbour 3.03125 (0x4042).
    """
    s = np.array([[0x3F81]], np.uint16)                  # 1 + 2^-7
    b = _bf16(-(2.0 ** -40))[None, :]
    w = np.zeros((1, 4), np.uint32)
    w[0, 0] = 3                                          # code 3 at k=0
    got = O.dequantize(w, s, b, 32, 4, "bfloat16")[0]
    assert int(got[0]) == 0x4042
    assert int(got[1]) == int(b[0, 0])                   # q = 0 -> b exactly


def test_dequant_closed_form_cases():
    rng = np.random.default_rng(2)
    for bits in (4, 8):
        N, K, gs = 5, 128, 64
        w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
        b = O.from_f32(rng.standard_normal((N, K // gs)).astype(np.float32), "bfloat16")
        zero_s = np.zeros_like(b)
        # s = 0 -> every weight equals its bias
        got = O.dequantize(w, zero_s, b, gs, bits, "bfloat16")
        np.testing.assert_array_equal(got, np.repeat(b, gs, axis=1))
        # codes all zero -> bias
        s = O.from_f32(rng.random((N, K // gs)).astype(np.float32), "bfloat16")
        got = O.dequantize(np.zeros_like(w), s, b, gs, bits, "bfloat16")
        np.testing.assert_array_equal(got, np.repeat(b, gs, axis=1))


def test_dequant_float64_route():
    """float64 s*q+b rounded once to float32 equals MLX's float32 arithmetic
    because s*q is exact; rounding that to bf16/f16 must equal the oracle."""
    rng = np.random.default_rng(3)
    for dtype in ("bfloat16", "float16"):
        for bits in (4, 8):
            N, K, gs = 9, 256, 32
            w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
            scale = np.float32(10.0) ** rng.integers(-6, 3, (N, K // gs)).astype(np.float32)
            s = O.from_f32((rng.standard_normal((N, K // gs)) * scale).astype(np.float32), dtype)
            b = O.from_f32((rng.standard_normal((N, K // gs)) * scale * 4).astype(np.float32), dtype)
            codes = np.array([[(int(w[n, k * bits // 32]) >> (bits * (k % (32 // bits)))) & ((1 << bits) - 1)
                               for k in range(K)] for n in range(N)], np.float64)
            s64 = np.repeat(O.to_f32(s, dtype).astype(np.float64), gs, axis=1)
            b64 = np.repeat(O.to_f32(b, dtype).astype(np.float64), gs, axis=1)
            exact = s64 * codes + b64
            want = O.from_f32(exact.astype(np.float32), dtype)
            np.testing.assert_array_equal(O.dequantize(w, s, b, gs, bits, dtype), want)
            # the independent C restatement agrees bit for bit
            np.testing.assert_array_equal(cref.dequantize(w, s, b, gs, bits, dtype), want)


def test_golden_dequant_fixture():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "dequant.npz"))
    keys = sorted({k.rsplit("_", 1)[0] for k in d.files})
    assert len(keys) == 12
    for key in keys:
        bits = int(key.split("_")[0][1:])
        gs = int(key.split("_")[1][1:])
        dtype = key.split("_")[2]
        got = O.dequantize(d[key + "_w"], d[key + "_s"], d[key + "_b"], gs, bits, dtype)
        np.testing.assert_array_equal(got, d[key + "_deq"])
        np.testing.assert_array_equal(
            cref.dequantize(d[key + "_w"], d[key + "_s"], d[key + "_b"], gs, bits, dtype),
            d[key + "_deq"])


# ------------------------------------------------------------------- matmul

def _py_bf16(u16):
    return struct.unpack("<f", struct.pack("<I", int(u16) << 16))[0]


def test_qmm_bruteforce_python_loop():
    """Pure-Python decode (struct-based bf16, manual nibbles, float64 sums)."""
    rng = np.random.default_rng(4)
    M, N, K, gs, bits = 2, 3, 64, 32, 4
    wq, s, b = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.1, gs, bits)
    x = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), "bfloat16")
    ref = O.quantized_matmul_ref(x, wq, s, b, gs, bits)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                q = (int(wq[n, k // 8]) >> (4 * (k % 8))) & 0xF
                v = np.float32(np.float32(_py_bf16(s[n, k // gs])) * np.float32(q)
                               + np.float32(_py_bf16(b[n, k // gs])))
                deq = _py_bf16(O.bf16_bits(v))
                acc += _py_bf16(x[m, k]) * deq
            assert abs(float(ref[m, n]) - acc) <= 1e-6 * max(1.0, abs(acc))


def test_qmm_invariants():
    rng = np.random.default_rng(5)
    M, N, K, gs, bits = 4, 16, 256, 64, 4
    wq, s, b = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02, gs, bits)
    # small integers: exact in bf16, so x1 + 2*x2 is exact too
    x1 = rng.integers(-3, 4, (M, K)).astype(np.float32)
    x2 = rng.integers(-3, 4, (M, K)).astype(np.float32)
    r1 = O.quantized_matmul_ref(O.from_f32(x1, "bfloat16"), wq, s, b, gs, bits)
    r2 = O.quantized_matmul_ref(O.from_f32(x2, "bfloat16"), wq, s, b, gs, bits)
    r12 = O.quantized_matmul_ref(O.from_f32(x1 + 2 * x2, "bfloat16"), wq, s, b, gs, bits)
    np.testing.assert_allclose(r12, r1 + 2 * r2, rtol=1e-5, atol=1e-5)
    # row independence
    for m in range(M):
        rm = O.quantized_matmul_ref(O.from_f32(x1[m:m + 1], "bfloat16"), wq, s, b, gs, bits)
        np.testing.assert_array_equal(rm[0], r1[m])
    # column n depends only on row n of w/s/b
    w2 = wq.copy()
    w2[5] ^= np.uint32(0x11111111)
    r_mod = O.quantized_matmul_ref(O.from_f32(x1, "bfloat16"), w2, s, b, gs, bits)
    changed = np.any(r_mod != r1, axis=0)
    assert changed[5] and changed.sum() == 1


def test_qmm_c_oracle_agrees():
    rng = np.random.default_rng(6)
    for bits, dtype in ((4, "bfloat16"), (8, "bfloat16"), (4, "float16")):
        M, N, K, gs = 3, 50, 512, 64
        wq, s, b = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02, gs, bits, dtype)
        x = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), dtype)
        ref = O.quantized_matmul_ref(x, wq, s, b, gs, bits, dtype)
        c = cref.qmm(x, wq, s, b, gs, bits, dtype)
        # the C oracle returns float32 sums; outputs are compared after the
        # final rounding to dtype, as the kernels emit them
        out = O.to_f32(O.from_f32(c, dtype), dtype)
        res = O.check_output(out, ref, dtype)
        assert res["ok"], res


def test_golden_qmm_fixture():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "qmm.npz"))
    keys = sorted({k.rsplit("_", 1)[0] for k in d.files})
    assert len(keys) == 4
    for key in keys:
        M, N, K, gs, bits, dt = (int(v) for v in d[key + "_meta"])
        dtype = "bfloat16" if dt == 0 else "float16"
        ref = O.quantized_matmul_ref(d[key + "_x"], d[key + "_w"], d[key + "_s"], d[key + "_b"],
                                     gs, bits, dtype)
        np.testing.assert_array_equal(ref, d[key + "_ref"])


# ------------------------------------------------------------------- gather

def test_gather_equals_dense_per_pair():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "gather.npz"))
    E, N, K, gs, bits = (int(v) for v in d["meta"])
    ref = O.gather_qmm_ref(d["x"], d["w"], d["s"], d["b"], d["lhs"], d["rhs"], gs, bits)
    np.testing.assert_array_equal(ref, d["ref"])
    lhs, rhs = d["lhs"].reshape(-1), d["rhs"].reshape(-1)
    for p in range(lhs.size):
        dense = O.quantized_matmul_ref(d["x"][lhs[p]], d["w"][rhs[p]], d["s"][rhs[p]],
                                       d["b"][rhs[p]], gs, bits)
        np.testing.assert_array_equal(ref[p], dense)
    # sorting the pairs by expert permutes the outputs and nothing else
    order = np.argsort(rhs, kind="stable")
    ref_sorted = O.gather_qmm_ref(d["x"], d["w"], d["s"], d["b"], lhs[order], rhs[order], gs, bits)
    np.testing.assert_array_equal(ref_sorted, ref[order])


# --------------------------------------------------------------- gather glu

def _const_bank(E, N, row_vals, bits=4, gs=64, K=64):
    """Bank whose dequantized row n of expert e is the constant row_vals[e][n]
    (codes 0, scale 1, bias = the value), exact in bf16 for the values used."""
    w = np.zeros((E, N, K * bits // 32), dtype=np.uint32)
    s = np.full((E, N, K // gs), O.bf16_bits(np.float32(1.0)), dtype=np.uint16)
    b = O.bf16_bits(np.asarray(row_vals, dtype=np.float32).reshape(E, N, 1)
                    .repeat(K // gs, axis=2))
    return w, s, b


def test_gather_glu_closed_forms():
    K = 64
    x = np.full((2, 1, K), O.bf16_bits(np.float32(1.0)), dtype=np.uint16)   # sum(x) = 64
    # gate / up rows give g = 64 * value: g in {0, 1, 2, 20, -20}
    gv = np.array([[0, 1, 2, 20, -20], [1, 2, 0, 1, 1]], dtype=np.float64) / 64
    uv = np.array([[5, 2, 1, 1, 1], [2, 1, 7, -3, 0]], dtype=np.float64) / 64
    gate, up = _const_bank(2, 5, gv), _const_bank(2, 5, uv)
    lhs, rhs = np.array([0, 1, 1]), np.array([0, 1, 0])
    out = O.gather_glu_ref(x, gate, up, lhs, rhs)
    e0 = [0.0, 2 * 0.7310585786300049, 2 * 0.8807970779778823,
          20 * 0.9999999979388463, -20 * 2.0611536181902037e-09]
    e1 = [2 * 0.7310585786300049, 2 * 0.8807970779778823, 0.0,
          -3 * 0.7310585786300049, 0.0]
    np.testing.assert_allclose(out[0, 0], e0, rtol=1e-7, atol=1e-12)
    np.testing.assert_allclose(out[1, 0], e1, rtol=1e-7, atol=1e-12)
    np.testing.assert_allclose(out[2, 0], e0, rtol=1e-7, atol=1e-12)
    # swapping the banks applies SiLU to the other product: pair 0, row 1
    # becomes g = 2, u = 1 -> 2 * sigmoid(2) instead of 2 * sigmoid(1)
    swapped = O.gather_glu_ref(x, up, gate, lhs, rhs)
    np.testing.assert_allclose(swapped[0, 0, 1], 2 * 0.8807970779778823, rtol=1e-7)
    assert not np.allclose(swapped, out)


def test_gather_glu_zero_gate_and_up_linearity():
    rng = np.random.default_rng(21)
    E, N, K = 3, 32, 128
    def bank():
        parts = [O.quantize((rng.standard_normal((N, K)) * 0.05).astype(np.float32), 64, 4)
                 for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    gate, up = bank(), bank()
    x = O.from_f32(rng.standard_normal((4, 2, K)).astype(np.float32), "bfloat16")
    lhs, rhs = np.array([0, 1, 2, 3, 0]), np.array([2, 0, 1, 2, 1])
    out = O.gather_glu_ref(x, gate, up, lhs, rhs)
    # a zero gate bank (scale 0, bias 0) zeroes every output
    zero = [gate[0], np.zeros_like(gate[1]), np.zeros_like(gate[2])]
    np.testing.assert_array_equal(O.gather_glu_ref(x, zero, up, lhs, rhs), 0.0)
    # doubling the up bank's scales and biases doubles the output exactly
    up2 = [up[0], O.bf16_bits(O.bf16_to_f32(up[1]) * 2), O.bf16_bits(O.bf16_to_f32(up[2]) * 2)]
    np.testing.assert_array_equal(O.gather_glu_ref(x, gate, up2, lhs, rhs), 2 * out)
    # and the gate product alone is gather_qmm's
    g = O.gather_qmm_ref(x, *gate, lhs, rhs)
    assert np.all(np.sign(out) == np.sign(g * O.gather_qmm_ref(x, *up, lhs, rhs)))


# quantize and the 3/5/6-bit packing are pinned in test_quantize_oracle.py


# --------------------------------------------------------------- tolerance

def test_tolerance_accepts_reordered_fp32_sum():
    rng = np.random.default_rng(8)
    M, N, K = 2, 256, 5120
    wq, s, b = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02, 64, 4)
    x = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), "bfloat16")
    ref = O.quantized_matmul_ref(x, wq, s, b, 64, 4)
    # a float32 accumulation in another order, rounded to bf16, must pass
    c = cref.qmm(x, wq, s, b, 64, 4)
    out = O.bf16_to_f32(O.bf16_bits(c))
    assert O.check_output(out, ref)["ok"]


def test_float32_tolerance_accepts_reordered_sums_and_rejects_bf16():
    """The composed routes' float32 outputs: a float32 GEMM summing in any
    order passes; the same product rounded through bf16 (a route that
    silently computed in 16 bits) fails; so does a dropped bias."""
    rng = np.random.default_rng(31)
    M, N, K, gs = 3, 96, 512, 64
    wq, s, b = O.quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float32), gs, 4,
                          "float32")
    x = rng.standard_normal((M, K)).astype(np.float32)
    ref = O.quantized_matmul_ref(x, wq, s, b, gs, 4, "float32")
    deq = O.dequantize(wq, s, b, gs, 4, "float32")
    # float32 accumulation in two different orders
    fwd = np.zeros((M, N), np.float32)
    for k in range(K):
        fwd += x[:, k:k + 1] * deq[:, k][None, :]
    blocked = sum((x[:, i:i + 64] @ deq[:, i:i + 64].T).astype(np.float32)
                  for i in range(K - 64, -1, -64))
    assert O.check_output(fwd, ref, "float32")["ok"]
    assert O.check_output(blocked, ref, "float32")["ok"]
    through_bf16 = O.bf16_to_f32(O.bf16_bits(ref))
    assert not O.check_output(through_bf16, ref, "float32")["ok"]
    nob = O.quantized_matmul_ref(x, wq, s, np.zeros_like(b), gs, 4, "float32")
    assert not O.check_output(nob, ref, "float32")["ok"]


def test_tolerance_rejects_planted_mistakes():
    """Plausible kernel mistakes must fail the contract (mistakes planted in the
    oracle's inputs, on the CPU)."""
    rng = np.random.default_rng(9)
    M, N, K, gs = 2, 256, 5120, 64
    wq, s, b = O.quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02, gs, 4)
    x = O.from_f32(rng.standard_normal((M, K)).astype(np.float32), "bfloat16")
    ref = O.quantized_matmul_ref(x, wq, s, b, gs, 4)
    xf = O.bf16_to_f32(x).astype(np.float64)

    def as_out(v):
        return O.bf16_to_f32(O.bf16_bits(np.asarray(v, np.float32)))

    # 1. un-rounded (fold) weights: MLX qmv's arithmetic, misses by ~1.5e-3
    fold = xf @ O.dequantize_f32(wq, s, b, gs, 4, "bfloat16").astype(np.float64).T
    assert not O.check_output(as_out(fold), ref)["ok"]
    # 2. dropped bias term
    nob = O.quantized_matmul_ref(x, wq, s, np.zeros_like(b), gs, 4)
    assert not O.check_output(as_out(nob), ref)["ok"]
    # 3. codes unpacked high nibble first
    codes = O.unpack(wq, 4).reshape(N, K // 8, 8)[:, :, ::-1].reshape(N, K)
    swapped = O.quantized_matmul_ref(x, O.pack(codes, 4), s, b, gs, 4)
    assert not O.check_output(as_out(swapped), ref)["ok"]
    # 4. scale of the neighbouring group
    s_shift = np.roll(s, 1, axis=1)
    wrong_g = O.quantized_matmul_ref(x, wq, s_shift, b, gs, 4)
    assert not O.check_output(as_out(wrong_g), ref)["ok"]
    # 5. one k-block (256 codes) lost
    x_drop = O.bf16_to_f32(x).copy()
    x_drop[:, 256:512] = 0
    lost = O.quantized_matmul_ref(O.from_f32(x_drop, "bfloat16"), wq, s, b, gs, 4)
    assert not O.check_output(as_out(lost), ref)["ok"]


# --------------------------------------------------------------- moe combine

def _combine_loop(y_f32, inv, w, rows, top_k):
    """Pure-Python restatement, element by element, with struct-rounded
    float32 accumulation (independent of numpy's vector casts)."""
    def f32(v):
        return struct.unpack("f", struct.pack("f", v))[0]
    N = y_f32.shape[1]
    out = np.zeros((rows, N), np.float32)
    for t in range(rows):
        for n in range(N):
            acc = 0.0
            for k in range(top_k):
                r = t * top_k + k if inv is None else int(inv[t * top_k + k])
                acc = f32(float(np.float32(w[t * top_k + k])) * float(y_f32[r, n]) + acc)
            out[t, n] = acc
    return out


def test_moe_combine_matches_loop():
    rng = np.random.default_rng(3)
    rows, top_k, N = 5, 3, 16
    y = O.from_f32(rng.standard_normal((rows * top_k, N)).astype(np.float32), "bfloat16")
    inv = rng.permutation(rows * top_k)
    w = rng.random(rows * top_k).astype(np.float32)
    got = O.moe_combine_ref(y, inv, w, rows, top_k)
    want = _combine_loop(O.to_f32(y, "bfloat16"), inv, w, rows, top_k)
    np.testing.assert_array_equal(got, want)


def test_moe_combine_invariants():
    rng = np.random.default_rng(4)
    rows, top_k, N = 7, 4, 24
    y = O.from_f32(rng.standard_normal((rows * top_k, N)).astype(np.float32), "bfloat16")
    yf = O.to_f32(y, "bfloat16")
    order = rng.permutation(rows * top_k)
    inv = np.argsort(order)
    # one-hot weights copy exactly the selected rows
    w = np.zeros(rows * top_k, np.float32)
    w[np.arange(rows) * top_k + 2] = 1.0
    got = O.moe_combine_ref(y, inv, w, rows, top_k)
    np.testing.assert_array_equal(got, yf[inv[np.arange(rows) * top_k + 2]])
    # identity inv == the unsorted layout; a sorted copy with inv == the original
    w = rng.random(rows * top_k).astype(np.float32)
    plain = O.moe_combine_ref(y, None, w, rows, top_k)
    np.testing.assert_array_equal(O.moe_combine_ref(y, np.arange(rows * top_k), w, rows, top_k),
                                  plain)
    y_sorted = y[order]                     # row j of y_sorted = row order[j] of y
    np.testing.assert_array_equal(O.moe_combine_ref(y_sorted, inv, w, rows, top_k), plain)
    # linear in w (up to float32 rounding)
    np.testing.assert_allclose(O.moe_combine_ref(y, None, 2 * w, rows, top_k), 2 * plain,
                               rtol=1e-6, atol=1e-6)
    # a planted mistake (dropping the last expert) is caught by the loop check
    bad = O.moe_combine_ref(y, None, np.where(np.arange(rows * top_k) % top_k == top_k - 1, 0, w)
                            .astype(np.float32), rows, top_k)
    assert not np.array_equal(bad, _combine_loop(yf, None, w, rows, top_k))
