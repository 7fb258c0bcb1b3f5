"""Pins the oracle's MoE routing and shared-expert merge (CPU only).

``moe_route_ref`` is checked by brute force over expert subsets, against
torch.topk / torch.softmax on distinct logits, on ties, on large logits (the
max subtraction), and by planted mistakes; ``sigmoid_t`` by closed-form
points and a float64 sigmoid; the shared merge of ``moe_combine_ref`` by the
cases where its roundings are known exactly.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _distinct_logits(rng, rows, E):
    return rng.permutation(rows * E).reshape(rows, E).astype(np.float32) / 7.0 - 3.0


def test_route_brute_force_subsets():
    rng = np.random.default_rng(1)
    E, k = 7, 3
    L = _distinct_logits(rng, 5, E)
    idx, w, _ = O.moe_route_ref(L, k)
    for r in range(L.shape[0]):
        best = max(itertools.combinations(range(E), k), key=lambda c: sum(L[r, list(c)]))
        assert set(idx[r]) == set(best)
        assert np.all(np.diff(L[r, idx[r]]) < 0)             # descending


def test_route_matches_torch_topk_softmax():
    rng = np.random.default_rng(2)
    L = _distinct_logits(rng, 4, 64)
    idx, w, _ = O.moe_route_ref(L, 8)
    tv, ti = torch.topk(torch.from_numpy(L), 8, dim=-1)
    np.testing.assert_array_equal(idx, ti.numpy())
    np.testing.assert_allclose(w, torch.softmax(tv.double(), -1).numpy(), rtol=2e-7, atol=0)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)


def test_route_ties_take_the_smaller_index():
    L = np.array([[1.0, 2.0, 2.0, 0.0, 2.0], [0.0, -0.0, 0.0, -1.0, 5.0]], np.float32)
    idx, w, _ = O.moe_route_ref(L, 3)
    np.testing.assert_array_equal(idx[0], [1, 2, 4])
    np.testing.assert_array_equal(idx[1], [4, 0, 1])
    np.testing.assert_array_equal(w[0], np.float32(1.0) / np.float32(3.0))


def test_route_large_logits_stay_finite():
    L = np.array([[200.0, 199.0, -50.0, 198.5]], np.float32)
    idx, w, _ = O.moe_route_ref(L, 3)
    np.testing.assert_array_equal(idx[0], [0, 1, 3])
    assert np.all(np.isfinite(w))
    np.testing.assert_allclose(w[0], np.exp([0.0, -1.0, -1.5]) / np.exp([0.0, -1.0, -1.5]).sum(),
                               rtol=1e-6)


def _planted_route(L, k, mistake):
    rows, E = L.shape
    idx = np.zeros((rows, k), np.int32)
    w = np.zeros((rows, k), np.float32)
    for r in range(rows):
        if mistake == "ties_larger":
            order = sorted(range(E), key=lambda e: (-float(L[r, e]), -e))[:k]
        else:
            order = sorted(range(E), key=lambda e: (-float(L[r, e]), e))[:k]
        v = L[r, order].astype(np.float32)
        ex = np.exp(v) if mistake == "no_max" else np.exp(v - v[0])
        w[r] = ex / ex.sum()
        idx[r] = order
    return idx, w


@pytest.mark.parametrize("mistake", ["ties_larger", "no_max"])
def test_route_checks_reject_planted_mistakes(mistake):
    L = np.array([[1.0, 2.0, 2.0, 0.0, 2.0]], np.float32)
    big = np.array([[200.0, 199.0, -50.0, 198.5]], np.float32)
    ref_t, _, _ = O.moe_route_ref(L, 3)
    ref_b, ref_wb, _ = O.moe_route_ref(big, 3)
    got_t, _ = _planted_route(L, 3, mistake)
    got_b, got_wb = _planted_route(big, 3, mistake)
    with np.errstate(all="ignore"):
        same = (np.array_equal(got_t, ref_t) and np.array_equal(got_b, ref_b)
                and np.allclose(got_wb, ref_wb, rtol=1e-6))
    assert not same


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_sigmoid_t_points(dtype):
    s = O.sigmoid_t(np.array([0.0, 30.0, -30.0], np.float32), dtype)
    assert s[0] == 0.5 and s[1] == 1.0 and s[2] < 1e-10
    x = O.to_f32(O.from_f32(np.linspace(-8, 8, 257).astype(np.float32), dtype), dtype)
    got = O.sigmoid_t(x, dtype)
    exact = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = O.ulp_bf16(exact.astype(np.float32)) if dtype == "bfloat16" else O.ulp_f16(exact.astype(np.float32))
    assert np.all(np.abs(got - exact) <= 2 * ulp)
    sym = O.sigmoid_t(-x, dtype)
    big = np.maximum(sym, got).astype(np.float32)   # the one >= 1/2 sets the rounding
    ulp2 = O.ulp_bf16(big) if dtype == "bfloat16" else O.ulp_f16(big)
    assert np.all(np.abs(sym - (1.0 - got)) <= 2 * ulp2)


def test_sigmoid_t_per_operation_rounding_known_answers():
    """Known answers worked by hand, where rounding every operation to T (the
    reference's form, moe_route_decode.py:141-146) and rounding the exact
    sigmoid once give different T values.

    bf16 (8 significant bits), x = -5: exp(5) = 148.41 -> 148; 1 + 148 =
    149 exactly; 1/149 = 219.92 * 2^-15 -> 220 * 2^-15.  The exact
    sigmoid(-5) = 0.0066929 = 219.31 * 2^-15 rounds to 219 * 2^-15.
    bf16, x = -5.75: exp(5.75) = 314.19 -> 314 (ulp 2 above 256); 1 + 314 =
    315, halfway between 314 and 316 -> 316 (even mantissa); 1/316 = 207.39
    * 2^-16 -> 207 * 2^-16.  Once: 0.0031727 = 207.92 * 2^-16 -> 208.
    fp16 (11 bits), x = -7.75: exp(7.75) = 2321.57 -> 2322 (ulp 2 above
    2048); 1 + 2322 = 2323 -> 2324 (tie, even); 1/2324 = 1804.78 * 2^-22 ->
    1805 * 2^-22.  Once: 0.00043056 = 1805.91 * 2^-22 -> 1806."""
    got = O.sigmoid_t(np.array([-5.0, -5.75], np.float32), "bfloat16")
    assert got[0] == np.float32(220 * 2.0 ** -15)
    assert got[1] == np.float32(207 * 2.0 ** -16)
    got16 = O.sigmoid_t(np.array([-7.75], np.float32), "float16")
    assert got16[0] == np.float32(1805 * 2.0 ** -22)

    # the plausible mistake (the sigmoid in float, rounded to T once) differs
    def once(x, dtype):
        f = (1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))).astype(np.float32)
        return O.to_f32(O.from_f32(f, dtype), dtype)

    assert once([-5.0, -5.75], "bfloat16").tolist() == [219 * 2.0 ** -15, 208 * 2.0 ** -16]
    assert once([-7.75], "float16")[0] == np.float32(1806 * 2.0 ** -22)


def test_route_shared_gate_is_sigmoid_of_rounded_dot():
    rng = np.random.default_rng(3)
    H = 64
    x = O.from_f32((rng.integers(-4, 5, (2, H)) / 8.0).astype(np.float32), "bfloat16")
    g = O.from_f32((rng.integers(-4, 5, H) / 4.0).astype(np.float32), "bfloat16")
    _, _, sg = O.moe_route_ref(np.zeros((2, 4), np.float32), 1, x, g)
    dot = O.to_f32(x, "bfloat16").astype(np.float64) @ O.to_f32(g, "bfloat16").astype(np.float64)
    np.testing.assert_array_equal(sg, O.sigmoid_t(dot.astype(np.float32), "bfloat16"))


def test_combine_shared_merge_known_roundings():
    rng = np.random.default_rng(4)
    rows, k, N = 3, 2, 16
    y = O.from_f32((rng.integers(-8, 8, (rows * k, N)) / 4.0).astype(np.float32), "bfloat16")
    w = np.array([0.5, 0.25, 1.0, 0.0, 2.0, -1.0], np.float32)
    base = O.moe_combine_ref(y, None, w, rows, k)                # exact sums of quarters
    zero = O.moe_combine_ref(y, None, w, rows, k, sgate=O.from_f32(np.zeros(rows, np.float32), "bfloat16"),
                             shared=O.from_f32(rng.standard_normal((rows, N)).astype(np.float32), "bfloat16"))
    np.testing.assert_array_equal(zero, O.to_f32(O.from_f32(base, "bfloat16"), "bfloat16"))
    sh = (rng.integers(-8, 8, (rows, N)) / 2.0).astype(np.float32)
    one = O.moe_combine_ref(y, None, w, rows, k, sgate=O.from_f32(np.ones(rows, np.float32), "bfloat16"),
                            shared=O.from_f32(sh, "bfloat16"))
    np.testing.assert_array_equal(one, base + sh)
