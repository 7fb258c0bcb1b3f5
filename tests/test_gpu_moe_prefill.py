"""The MoE layer at prefill widths as the reference runs it (fused.py:3283-3316):
one table build per routing shared by the gate, up and down gathers, x read
through each pair's token, the gate and up gathers with the SwiGLU in one
launch, one combine.

Checked: the SwiGLU kernel against its torch composition bit for bit (bf16,
fp16, ragged lengths, unaligned views); gathers over shared tables against
the same gathers building their own, bit for bit, with hot experts (the
two-row-class tables, whose 128-pair segments the down bank's 4-wave kernel
runs as two 64-row tiles); the fused gate+up+SwiGLU launch against the two
gathers and the SwiGLU pass, bit for bit (8- and 4-wave kernels, ragged
column counts, fp16, 8-bit, out-of-range experts); the whole layer against
the sort path (sorted gathers, torch SwiGLU, unsort or combine) bit for bit,
at config-4 size (2048 tokens x top-8 over 512 experts, hidden 2048,
intermediate 512) and small banks, zipf and uniform routing; each gather of
the layer against the oracle on sampled pairs; launch counts (two table
kernels per layer).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import ops
from mlxturbo_amd.nn import QuantizedSwitchLinear, SwitchGLU
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, quantized, random_packed, to_dev, zipf_routing

pytestmark = pytest.mark.gpu


def _check(out_t, ref, dtype="bfloat16"):
    res = O.check_output(from_dev(out_t), ref, dtype)
    assert res["ok"], res
    return res


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [8, 1000, 4099, 65536 + 5])
def test_swiglu_matches_torch_composition(dtype, n):
    g = torch.randn(n, device="cuda").mul(4).to(dtype)
    u = torch.randn(n, device="cuda").to(dtype)
    want = (torch.nn.functional.silu(g.float()).to(dtype).float() * u.float()).to(dtype)
    np.testing.assert_array_equal(bits16(ops.swiglu(g, u)), bits16(want))
    # unaligned views take the scalar path
    gv, uv = g[1:], u[1:]
    np.testing.assert_array_equal(bits16(ops.swiglu(gv, uv)), bits16(want[1:]))


def test_swiglu_special_values():
    """silu(0) = 0, silu of large negatives -> -0, silu(inf) = inf, and NaN
    where torch gives NaN (silu(-inf) = -inf / inf, a NaN whose sign bit
    differs: 0xFFC0 here, 0x7FC0 from torch; NaN positions must agree and
    every other value bit for bit)."""
    g = torch.tensor([0.0, -100.0, 100.0, float("inf"), float("-inf"), float("nan"), 1.0, -1.0],
                     device="cuda").to(torch.bfloat16)
    u = torch.tensor([3.0, 2.0, 0.5, 1.0, 1.0, 1.0, 0.0, -2.0], device="cuda").to(torch.bfloat16)
    want = (torch.nn.functional.silu(g.float()).to(torch.bfloat16).float() * u.float()).to(
        torch.bfloat16)
    got = ops.swiglu(g, u)
    nan = torch.isnan(want)
    assert torch.equal(torch.isnan(got), nan) and int(nan.sum()) == 2
    np.testing.assert_array_equal(bits16(got[~nan]), bits16(want[~nan]))


def _bank(rng, E, N, K, mlx=False):
    if mlx:
        parts = [quantized(rng, N, K) for _ in range(E)]
        w, s, b = [np.stack([p[i] for p in parts]) for i in range(3)]
    else:
        w, s, b = random_packed(rng, E * N, K)
        w, s, b = w.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    return (w, s, b), QuantizedSwitchLinear(to_dev(w), to_dev(s, "bfloat16"),
                                            to_dev(b, "bfloat16"))


@pytest.mark.parametrize("routing", ["zipf", "uniform"])
def test_gathers_over_shared_tables(routing):
    """gate (K=2048, 8-wave kernel, 128-row tiles for hot experts) and down
    (K=512, 4-wave kernel, 128-pair segments as two 64-row tiles) over one
    table build equal the gathers that build their own, bit for bit."""
    rng = np.random.default_rng(7 if routing == "zipf" else 8)
    E, T, top, H, I = 64, 512, 8, 2048, 512
    _, gate = _bank(rng, E, I, H)
    _, down = _bank(rng, E, H, I)
    idx = zipf_routing(rng, T, top, E) if routing == "zipf" else \
        np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    if routing == "zipf":
        assert counts.max() > 128                     # class-1 segments in both halves
    rhs = torch.from_numpy(idx).cuda()
    xe = to_dev(act(rng, (T, 1, 1, H), scale=0.5), "bfloat16")
    hx = to_dev(act(rng, (T, top, 1, I), scale=0.5), "bfloat16")
    before = mq.launch_count()
    tables = ops.gather_tables(rhs, E)
    assert tables is not None and mq.launch_count() == before + 2
    for mod, x in ((gate, xe), (down, hx)):
        before = mq.launch_count()
        got = mod(x, rhs, tables=tables)
        assert mq.launch_count() == before + 1        # no table build
        want = mod(x, rhs)
        np.testing.assert_array_equal(bits16(got), bits16(want))


@pytest.mark.parametrize("E, T, top, H, I, routing, dtype, bits", [
    (64, 512, 8, 2048, 512, "zipf", "bfloat16", 4),     # 8 waves, 128-row tiles
    (64, 512, 8, 1024, 256, "uniform", "bfloat16", 4),  # 4 waves, halves
    (48, 300, 4, 512, 200, "zipf", "bfloat16", 4),      # ragged column tile
    (64, 512, 8, 2048, 512, "zipf", "float16", 4),
    (64, 256, 8, 1024, 384, "uniform", "bfloat16", 8),
])
def test_gather_swiglu_matches_three_calls(E, T, top, H, I, routing, dtype, bits):
    """mq_gather_swiglu_tables equals the gate and up gathers over the same
    tables followed by the SwiGLU pass, bit for bit, in one launch."""
    rng = np.random.default_rng(E + T + I + bits)
    banks = []
    for _ in range(2):
        w, s, b = random_packed(rng, E * I, H, bits=bits, dtype=dtype)
        banks.append((to_dev(w).view(E, I, -1), to_dev(s, dtype).view(E, I, -1),
                      to_dev(b, dtype).view(E, I, -1)))
    idx = zipf_routing(rng, T, top, E) if routing == "zipf" else \
        np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    rhs = torch.from_numpy(idx).cuda()
    xe = to_dev(act(rng, (T, 1, 1, H), dtype, scale=0.5), dtype)
    tables = ops.gather_tables(rhs, E)
    assert tables is not None
    kw = dict(group_size=64, bits=bits)
    before = mq.launch_count()
    got = ops.gather_swiglu(xe, banks[0], banks[1], rhs, tables, **kw)
    assert mq.launch_count() == before + 1
    want = ops.swiglu(ops.gather_qmm(xe, *banks[0], rhs_indices=rhs, tables=tables, **kw),
                      ops.gather_qmm(xe, *banks[1], rhs_indices=rhs, tables=tables, **kw))
    assert got.shape == (T, top, 1, I)
    np.testing.assert_array_equal(bits16(got), bits16(want))


def test_gather_swiglu_rows_per_pair():
    """Four x rows per pair (tables of 16-pair segments): the fused launch
    equals the two gathers and the SwiGLU pass, bit for bit."""
    rng = np.random.default_rng(21)
    E, T, top, H, I, Mi = 32, 128, 4, 1024, 256, 4
    banks = []
    for _ in range(2):
        w, s, b = random_packed(rng, E * I, H)
        banks.append((to_dev(w).view(E, I, -1), to_dev(s, "bfloat16").view(E, I, -1),
                      to_dev(b, "bfloat16").view(E, I, -1)))
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    rhs = torch.from_numpy(idx).cuda()
    xe = to_dev(act(rng, (T, 1, Mi, H), scale=0.5), "bfloat16")
    tables = ops.gather_tables(rhs, E, rows=Mi)
    assert tables is not None
    got = ops.gather_swiglu(xe, banks[0], banks[1], rhs, tables)
    want = ops.swiglu(ops.gather_qmm(xe, *banks[0], rhs_indices=rhs, tables=tables),
                      ops.gather_qmm(xe, *banks[1], rhs_indices=rhs, tables=tables))
    assert got.shape == (T, top, Mi, I)
    np.testing.assert_array_equal(bits16(got), bits16(want))


def test_gather_swiglu_out_of_range_experts():
    """Pairs whose expert is outside the bank get zero rows from the fused
    launch, as from the gathers and the SwiGLU."""
    rng = np.random.default_rng(3)
    E, T, top, H, I = 32, 256, 4, 1024, 256
    banks = []
    for _ in range(2):
        w, s, b = random_packed(rng, E * I, H)
        banks.append((to_dev(w).view(E, I, -1), to_dev(s, "bfloat16").view(E, I, -1),
                      to_dev(b, "bfloat16").view(E, I, -1)))
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    idx[::7, 1] = E + 3
    idx[::11, 2] = -1
    rhs = torch.from_numpy(idx).cuda()
    xe = to_dev(act(rng, (T, 1, 1, H), scale=0.5), "bfloat16")
    tables = ops.gather_tables(rhs, E)
    got = ops.gather_swiglu(xe, banks[0], banks[1], rhs, tables)
    want = ops.swiglu(ops.gather_qmm(xe, *banks[0], rhs_indices=rhs, tables=tables),
                      ops.gather_qmm(xe, *banks[1], rhs_indices=rhs, tables=tables))
    np.testing.assert_array_equal(bits16(got), bits16(want))
    assert not bits16(got)[::7, 1].any() and not bits16(got)[::11, 2].any()


def _layer(rng, E, H, I, mlx=False):
    banks = [_bank(rng, E, I, H, mlx), _bank(rng, E, I, H, mlx), _bank(rng, E, H, I, mlx)]
    return [b[0] for b in banks], [b[1] for b in banks]


@pytest.mark.parametrize("E, T, top, H, I, routing, mlx", [
    (64, 512, 8, 1024, 256, "zipf", False),
    (64, 300, 4, 512, 512, "uniform", False),
    (512, 2048, 8, 2048, 512, "zipf", True),
])
def test_prefill_layer_matches_sort_path(E, T, top, H, I, routing, mlx):
    """SwitchGLU over shared tables (4 launches + combine) equals the sort
    path (argsorts, gathered x, sorted gathers with their own tables, torch
    SwiGLU, unsort / combine) bit for bit, with and without router scores;
    the gate gather and the down gather of the layer meet the oracle on
    sampled pairs."""
    rng = np.random.default_rng(E + T + H)
    raw, mods = _layer(rng, E, H, I, mlx)
    new, old = SwitchGLU(*mods), SwitchGLU(*mods, prefill_tables=False)
    idx = zipf_routing(rng, T, top, E) if routing == "zipf" else \
        np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    rhs = torch.from_numpy(idx).cuda()
    xh = act(rng, (T, H))
    x = to_dev(xh, "bfloat16")
    scores = torch.from_numpy(rng.random((T, top)).astype(np.float32)).cuda()
    before = mq.launch_count()
    y = new(x, rhs)
    assert mq.launch_count() == before + 4            # tables (2), gate+up+swiglu, down
    assert y.shape == (T, top, H)
    np.testing.assert_array_equal(bits16(y), bits16(old(x, rhs)))
    before = mq.launch_count()
    ys = new(x, rhs, scores)
    assert mq.launch_count() == before + 5
    np.testing.assert_array_equal(bits16(ys), bits16(old(x, rhs, scores)))
    # the layer's gathers against the oracle on sampled pairs
    pairs = np.unique(rng.choice(T * top, 48, replace=False))
    xe = x.reshape(T, 1, 1, H)
    gk = mods[0](xe, rhs)
    lhs = np.repeat(np.arange(T), top)
    ref = O.gather_qmm_ref(xh.reshape(T, 1, H), *raw[0], lhs[pairs], idx.reshape(-1)[pairs])
    _check(gk.reshape(T * top, 1, I)[torch.from_numpy(pairs).cuda()], ref)
    h = ops.swiglu(gk, mods[1](xe, rhs))
    hp = bits16(h).reshape(T * top, 1, I)[pairs]
    ref = O.gather_qmm_ref(hp, *raw[2], np.arange(len(pairs)), idx.reshape(-1)[pairs])
    _check(y.reshape(T * top, 1, H)[torch.from_numpy(pairs).cuda()], ref)


def test_prefill_layer_falls_back_off_the_thin_kernel():
    """Few experts (more than 96 rows each): the gathers do not run on the
    tables' kernel; the layer still equals the sort path."""
    rng = np.random.default_rng(31)
    E, T, top, H, I = 8, 512, 2, 512, 256
    _, mods = _layer(rng, E, H, I)
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    rhs = torch.from_numpy(idx).cuda()
    x = to_dev(act(rng, (T, H)), "bfloat16")
    new, old = SwitchGLU(*mods), SwitchGLU(*mods, prefill_tables=False)
    np.testing.assert_array_equal(bits16(new(x, rhs)), bits16(old(x, rhs)))
