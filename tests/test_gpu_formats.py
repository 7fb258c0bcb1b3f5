"""GPU parity of the format definers and of the composed routes.

* ``quantize`` (mq_quantize) bit-exact against ``oracle.quantize`` for every
  width, group size and dtype, including zero, constant, below-floor,
  |min|-dominant, large, NaN and inf groups;
* ``dequantize`` of the 2/3/5/6-bit widths bit-exact against the oracle;
* configurations without a matmul kernel (2/3/5/6 bits, ``transpose=False``,
  float32 and mixed-dtype activations) and gathers routed around the kernels'
  limits (more than 16 rows per pair, more experts than the prep tables)
  against the oracle's fp32 reference, to the same tolerance;
* moe_combine skipping out-of-range rows; the rebit flow (requantize).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import rebit
from mlxturbo_amd.nn import QuantizedLinear
from oracle import oracle as O
from qmm_helpers import TORCH_DTYPE, act, bits16, from_dev, quantized, to_dev

pytestmark = pytest.mark.gpu


def _dev_float(a32: np.ndarray, dtype: str) -> torch.Tensor:
    """float32 values (exactly representable in dtype) -> tensor of dtype."""
    if dtype == "float32":
        return torch.from_numpy(np.ascontiguousarray(a32, dtype=np.float32)).cuda()
    return to_dev(O.from_f32(a32, dtype), dtype)


def _param_bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


def _oracle_param_bits(a: np.ndarray, dtype: str) -> np.ndarray:
    return a.view(np.uint32) if dtype == "float32" else a


def _special_rows(rng, K, gs, dtype):
    """Rows exercising every branch of the quantizer."""
    G = K // gs
    rows = [(rng.standard_normal((8, K)) * 0.02).astype(np.float32)]
    z = np.zeros((1, K), np.float32)                               # all-zero groups
    c = np.full((1, K), 0.3, np.float32)                           # constant groups
    t = np.full((1, K), 3e-8, np.float32)                          # below the 1e-7 floor
    neg = (rng.standard_normal((1, K)) * 0.02).astype(np.float32)
    neg[0, ::gs] = -0.5                                            # |min| dominant
    big = (rng.standard_normal((1, K)) * (300.0 if dtype != "float16" else 30.0)).astype(np.float32)
    rows += [z, c, t, neg, big]
    if dtype != "float16":
        huge = (rng.standard_normal((1, K)) * 1e30).astype(np.float32)
        rows.append(huge)
    w = np.concatenate(rows)
    w = O.to_f32(O.from_f32(w, dtype), dtype)                      # exact in dtype
    return w


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_quantize_bit_exact(bits, dtype):
    for gs in (32, 64, 128):
        rng = np.random.default_rng(100 * bits + gs)
        K = gs * 5
        w = _special_rows(rng, K, gs, dtype)
        wq, s, b = mq.quantize(_dev_float(w, dtype), group_size=gs, bits=bits)
        ewq, es, eb = O.quantize(w, gs, bits, dtype)
        np.testing.assert_array_equal(from_dev(wq), ewq, err_msg=f"codes gs={gs}")
        np.testing.assert_array_equal(_param_bits(s), _oracle_param_bits(es, dtype),
                                      err_msg=f"scales gs={gs}")
        np.testing.assert_array_equal(_param_bits(b), _oracle_param_bits(eb, dtype),
                                      err_msg=f"biases gs={gs}")
        assert s.dtype == TORCH_DTYPE[dtype] and wq.shape == (w.shape[0], K * bits // 32)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_quantize_nonfinite_groups(dtype):
    """NaN propagates through a group's min/max (codes 0, NaN scale and
    bias); an inf value makes the group's scale NaN.  NaN signs are the
    generating hardware's, so NaN-ness is compared, not bits."""
    rng = np.random.default_rng(3)
    K, gs = 256, 64
    w = (rng.standard_normal((4, K)) * 0.02).astype(np.float32)
    w[0, 5] = np.nan
    w[1, 70] = np.inf
    w[2, 130] = -np.inf
    w = O.to_f32(O.from_f32(w, dtype), dtype)
    wq, s, b = mq.quantize(_dev_float(w, dtype), group_size=gs, bits=4)
    ewq, es, eb = O.quantize(w, gs, 4, dtype)
    np.testing.assert_array_equal(from_dev(wq), ewq)
    for got, want in ((s, es), (b, eb)):
        g = from_dev(got) if dtype == "float32" else O.to_f32(_param_bits(got), dtype)
        e = O.to_f32(want, dtype)
        np.testing.assert_array_equal(np.isnan(g), np.isnan(e))
        ok = ~np.isnan(e)
        np.testing.assert_array_equal(g[ok], e[ok])


def test_quantize_round_trips_exact_grids():
    """Values on an affine grid come back unchanged through quantize +
    dequantize on the GPU (both scale orientations)."""
    gs, bits = 64, 4
    s = 2.0 ** -7
    codes = np.random.default_rng(1).integers(0, 16, size=(4, 256))
    codes[:, ::64] = 0
    codes[:, 1::64] = 15
    w = np.concatenate([(-12 + codes[:2]) * s, (9 - codes[2:]) * s]).astype(np.float32)
    wd = _dev_float(w, "bfloat16")
    wq, sc, bi = mq.quantize(wd, group_size=gs, bits=bits)
    back = mq.dequantize(wq, sc, bi, group_size=gs, bits=bits)
    np.testing.assert_array_equal(bits16(back), bits16(wd))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("bits", [2, 3, 5, 6])
def test_dequantize_other_widths_bit_exact(bits, dtype):
    for gs in (32, 64, 128):
        rng = np.random.default_rng(7 * bits + gs)
        N, K = 19, gs * 6
        w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
        s = O.from_f32((rng.random((N, K // gs)) * 0.02 - 0.01).astype(np.float32), dtype)
        b = O.from_f32((rng.random((N, K // gs)) * 0.2 - 0.1).astype(np.float32), dtype)
        sd = _dev_float(O.to_f32(s, dtype), dtype)
        bd = _dev_float(O.to_f32(b, dtype), dtype)
        got = mq.dequantize(to_dev(w), sd, bd, group_size=gs, bits=bits)
        want = O.dequantize(w, s, b, gs, bits, dtype)
        np.testing.assert_array_equal(_param_bits(got), _oracle_param_bits(want, dtype),
                                      err_msg=f"gs={gs}")


# ------------------------------------------------------------ composed routes

def _chk(out, ref, dtype="bfloat16"):
    res = O.check_output(from_dev(out), ref, dtype)
    assert res["ok"], res


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
@pytest.mark.parametrize("M", [1, 7, 40])
def test_qmm_other_widths(bits, M):
    rng = np.random.default_rng(bits * 10 + M)
    N, K, gs = 200, 640, 64
    w, s, b = quantized(rng, N, K, gs, bits)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"), group_size=gs, bits=bits)
    assert out.dtype == torch.bfloat16
    _chk(out, O.quantized_matmul_ref(x, w, s, b, gs, bits))


@pytest.mark.parametrize("bits", [4, 8, 3])
def test_qmm_transpose_false(bits):
    """x @ dequantize(w) with w [K, N*bits/32] quantized along N."""
    rng = np.random.default_rng(bits)
    K, N, gs, M = 384, 256, 64, 5
    w, s, b = quantized(rng, K, N, gs, bits)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"), transpose=False, group_size=gs, bits=bits)
    assert out.shape == (M, N)
    _chk(out, O.quantized_matmul_ref(x, w, s, b, gs, bits, transpose=False))


def test_qmm_float32_and_mixed_activations():
    rng = np.random.default_rng(5)
    N, K, gs, bits, M = 96, 512, 64, 4, 3
    w, s16, b16 = quantized(rng, N, K, gs, bits)
    # float32 scales and activations: everything in float32
    s32, b32 = O.to_f32(s16, "bfloat16"), O.to_f32(b16, "bfloat16")
    x32 = (rng.standard_normal((M, K))).astype(np.float32)
    out = mq.quantized_matmul(torch.from_numpy(x32).cuda(), to_dev(w), torch.from_numpy(s32).cuda(),
                              torch.from_numpy(b32).cuda(), group_size=gs, bits=bits)
    assert out.dtype == torch.float32
    _chk(out, O.quantized_matmul_ref(x32, w, s32, b32, gs, bits, "float32"), "float32")
    # float16 activations over bfloat16 scales: MLX promotes both to float32
    xh = O.from_f32(x32, "float16")
    out = mq.quantized_matmul(to_dev(xh, "float16"), to_dev(w), to_dev(s16, "bfloat16"),
                              to_dev(b16, "bfloat16"), group_size=gs, bits=bits)
    assert out.dtype == torch.float32
    ref = O.quantized_matmul_ref(O.to_f32(xh, "float16"), w, s32, b32, gs, bits, "float32")
    _chk(out, ref, "float32")


def _bank(rng, E, N, K, gs=64, bits=4):
    parts = [quantized(rng, N, K, gs, bits) for _ in range(E)]
    return tuple(np.stack([p[i] for p in parts]) for i in range(3))


def test_gather_more_than_16_rows_per_pair():
    rng = np.random.default_rng(8)
    E, N, K, T, top, M = 6, 96, 256, 5, 3, 24
    w, s, b = _bank(rng, E, N, K)
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    x = act(rng, (T, 1, M, K))
    out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                        to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda())
    assert out.shape == (T, top, M, N)
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, np.repeat(np.arange(T), top),
                           idx.reshape(-1))
    _chk(out.reshape(T * top, M, N), ref)


def test_gather_more_experts_than_prep_tables():
    """4100 experts, 700 pairs (prep path): the bank runs in 2048-expert
    slices; invalid indices still give zero rows."""
    rng = np.random.default_rng(9)
    E, N, K, P = 4100, 32, 64, 700
    w = rng.integers(0, 2**32, size=(E, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = O.from_f32((rng.random((E, N, 1)) * 0.01).astype(np.float32), "bfloat16")
    b = O.from_f32((rng.random((E, N, 1)) * 0.02 - 0.04).astype(np.float32), "bfloat16")
    idx = rng.integers(0, E, P).astype(np.int32)
    idx[[3, 50]] = [-1, E + 7]
    x = act(rng, (P, 1, K))
    out = from_dev(mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                                 to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda()))
    assert np.all(out[[3, 50]] == 0)
    ok = np.setdiff1d(np.arange(P), [3, 50])
    ref = O.gather_qmm_ref(x, w, s, b, ok, idx[ok])
    res = O.check_output(out[ok], ref)
    assert res["ok"], res


@pytest.mark.parametrize("case", ["bits3", "transpose", "float32"])
def test_gather_composed(case):
    rng = np.random.default_rng(10)
    E, T, top = 5, 7, 2
    N, K, gs = 64, 128, 64
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    lhs, rhs = np.repeat(np.arange(T), top), idx.reshape(-1)
    if case == "bits3":
        w, s, b = _bank(rng, E, N, K, gs, 3)
        x = act(rng, (T, 1, 1, K))
        out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                            to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda(), bits=3)
        _chk(out.reshape(T * top, 1, N), O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, lhs, rhs,
                                                          gs, 3))
    elif case == "transpose":
        w, s, b = _bank(rng, E, K, N, gs, 4)                  # [E, K, N*bits/32]
        x = act(rng, (T, 1, 1, K))
        out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                            to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda(),
                            transpose=False)
        assert out.shape == (T, top, 1, N)
        ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, lhs, rhs, gs, 4, transpose=False)
        _chk(out.reshape(T * top, 1, N), ref)
    else:
        w, s, b = _bank(rng, E, N, K, gs, 4)
        s32, b32 = O.to_f32(s, "bfloat16"), O.to_f32(b, "bfloat16")
        x = rng.standard_normal((T, 1, 1, K)).astype(np.float32)
        out = mq.gather_qmm(torch.from_numpy(x).cuda(), to_dev(w), torch.from_numpy(s32).cuda(),
                            torch.from_numpy(b32).cuda(), rhs_indices=torch.from_numpy(idx).cuda())
        assert out.dtype == torch.float32
        ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s32, b32, lhs, rhs, gs, 4, "float32")
        _chk(out.reshape(T * top, 1, N), ref, "float32")


def test_gather_glu_composed_for_other_widths():
    rng = np.random.default_rng(11)
    E, T, top, N, K, gs = 4, 3, 2, 64, 128, 64
    gate, up = _bank(rng, E, N, K, gs, 5), _bank(rng, E, N, K, gs, 5)
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    x = act(rng, (T, 1, 1, K))
    dev = lambda bk: (to_dev(bk[0]), to_dev(bk[1], "bfloat16"), to_dev(bk[2], "bfloat16"))
    out = mq.gather_glu(to_dev(x, "bfloat16"), *dev(gate), *dev(up),
                        rhs_indices=torch.from_numpy(idx).cuda(), bits=5)
    lhs, rhs = np.repeat(np.arange(T), top), idx.reshape(-1)
    g = O.from_f32(O.gather_qmm_ref(x.reshape(T, 1, K), *gate, lhs, rhs, gs, 5), "bfloat16")
    u = O.from_f32(O.gather_qmm_ref(x.reshape(T, 1, K), *up, lhs, rhs, gs, 5), "bfloat16")
    gf = O.to_f32(g, "bfloat16").astype(np.float64)
    ref = (gf / (1 + np.exp(-gf)) * O.to_f32(u, "bfloat16")).astype(np.float32)
    _chk(out.reshape(T * top, 1, N), ref)


def test_moe_combine_skips_out_of_range_rows():
    rng = np.random.default_rng(12)
    rows, top_k, N = 6, 4, 128
    y_rows = rows * top_k - 3                                # y holds fewer rows than pairs
    y = O.from_f32(rng.standard_normal((y_rows, N)).astype(np.float32), "bfloat16")
    inv = rng.integers(0, y_rows, rows * top_k).astype(np.int32)
    inv[[1, 6, 11]] = [-1, y_rows, 1 << 30]
    w = rng.random(rows * top_k).astype(np.float32)
    out = mq.moe_combine(to_dev(y, "bfloat16"), torch.from_numpy(inv).cuda(),
                         torch.from_numpy(w).cuda(), rows, top_k)
    w0 = w.copy()
    w0[[1, 6, 11]] = 0.0
    inv0 = np.where((inv >= 0) & (inv < y_rows), inv, 0)
    ref = O.moe_combine_ref(y, inv0, w0, rows, top_k)
    _chk(out, ref)


def test_rebit_requantize_and_apply():
    """rebit flow: a float layer quantized to 8 bits, re-quantized to 4
    (dequantize + quantize on the GPU) equals the oracle's double
    quantization bit for bit, and runs."""
    rng = np.random.default_rng(13)
    N, K = 128, 512
    wf = O.to_f32(O.from_f32((rng.standard_normal((N, K)) * 0.02).astype(np.float32),
                             "bfloat16"), "bfloat16")
    lin = torch.nn.Linear(K, N, bias=False).to(torch.bfloat16).cuda()
    with torch.no_grad():
        lin.weight.copy_(_dev_float(wf, "bfloat16"))
    q8 = rebit.requantize(lin, 8, 64)
    q4 = rebit.requantize(q8, 4, 32)
    w8, s8, b8 = O.quantize(wf, 64, 8, "bfloat16")
    d8 = O.to_f32(O.dequantize(w8, s8, b8, 64, 8, "bfloat16"), "bfloat16")
    w4, s4, b4 = O.quantize(d8, 32, 4, "bfloat16")
    np.testing.assert_array_equal(from_dev(q4.weight), w4)
    np.testing.assert_array_equal(bits16(q4.scales), s4)
    np.testing.assert_array_equal(bits16(q4.biases), b4)
    model = torch.nn.Module()
    model.lm_head = q8
    model.layers = torch.nn.ModuleList([torch.nn.Module()])
    model.layers[0].self_attn = torch.nn.Module()
    model.layers[0].self_attn.q_proj = QuantizedLinear.from_linear(_dev_float(wf, "bfloat16"),
                                                                   bits=4)
    counts = rebit.apply(model, "head=4:32,attn=4")
    assert counts == {"head": 1, "attn": 0}                  # attn already 4-bit g64
    assert model.lm_head.bits == 4 and model.lm_head.group_size == 32
    x = act(rng, (2, K))
    out = model.lm_head(to_dev(x, "bfloat16"))
    _chk(out, O.quantized_matmul_ref(x, w4, s4, b4, 32, 4))
