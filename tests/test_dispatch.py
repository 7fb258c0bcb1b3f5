"""Module-level drop-in: route table, per-instance class swap, dispatch scope,
class-level patch (reference: mlxturbo/kernels/dispatch.py:59-466,
fast_qmm.py:395-472), and the torch QuantizedLinear / SwitchGLU modules.

Routing logic runs on the CPU (module tensors stay on the CPU and nothing is
computed); the forward passes are GPU tests against the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import dispatch
from mlxturbo_amd.nn import QuantizedLinear, QuantizedSwitchLinear, SwitchGLU
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, quantized, to_dev, zipf_routing


def _layer(N=64, K=128, device="cpu", bias=False):
    rng = np.random.default_rng(0)
    w, s, b = quantized(rng, N, K)
    return QuantizedLinear(to_dev(w, device=device), to_dev(s, "bfloat16", device),
                           to_dev(b, "bfloat16", device),
                           bias=(torch.zeros(N, dtype=torch.bfloat16, device=device)
                                 if bias else None))


def test_select_route_table():
    # measured geometries: skinny at every verify width, wide past 16 rows
    assert dispatch.select_route(5120, 17408, 1) == dispatch.SKINNY
    assert dispatch.select_route(5120, 17408, 16) == dispatch.SKINNY
    assert dispatch.select_route(5120, 17408, 17) == dispatch.WIDE
    assert dispatch.select_route(17408, 5120, 8) == dispatch.SKINNY
    # unknown geometry, M = 0 and negative widths: stock
    assert dispatch.select_route(1000, 1000, 4) == dispatch.STOCK
    assert dispatch.select_route(5120, 17408, 0) == dispatch.STOCK
    assert dispatch.select_route(5120, 17408, -1) == dispatch.STOCK
    # caller tables override; invalid route names are rejected
    assert dispatch.select_route(8, 8, 2, {(8, 8): ("stock", "wide", "skinny")}) == "skinny"
    with pytest.raises(ValueError):
        dispatch.select_route(8, 8, 1, {(8, 8): ("stock", "bogus")})


def test_enable_swaps_class_in_place():
    model = torch.nn.Sequential(_layer(), torch.nn.ReLU(), _layer(bias=True))
    first = model[0]
    w = first.weight
    keys = sorted(model.state_dict().keys())
    dispatch.enable(model)
    assert model[0] is first and model[0].weight is w
    assert type(model[0]) is dispatch.DispatchedQuantizedLinear
    assert type(model[2]) is dispatch.DispatchedQuantizedLinear
    assert sorted(model.state_dict().keys()) == keys
    assert model[0]._mq_dispatch_always is True
    dispatch.enable(model, active=False)                 # idempotent, flips the flag
    assert type(model[0]) is dispatch.DispatchedQuantizedLinear
    assert model[0]._mq_dispatch_always is False
    dispatch.disable(model)
    assert type(model[0]) is QuantizedLinear and model[0] is first


def test_dispatch_scope_flag():
    assert not dispatch._DISPATCH_ACTIVE.get()
    with dispatch.dispatch_scope():
        assert dispatch._DISPATCH_ACTIVE.get()
        with dispatch.dispatch_scope():
            assert dispatch._DISPATCH_ACTIVE.get()
        assert dispatch._DISPATCH_ACTIVE.get()
    assert not dispatch._DISPATCH_ACTIVE.get()


def test_class_patch_is_reversible():
    orig = QuantizedLinear.forward
    dispatch.enable_class()
    assert QuantizedLinear.forward is not orig
    dispatch.enable_class()                               # idempotent
    dispatch.disable_class()
    assert QuantizedLinear.forward is orig


def test_module_validation():
    rng = np.random.default_rng(1)
    w, s, b = quantized(rng, 32, 128)
    with pytest.raises(ValueError):
        QuantizedLinear(torch.from_numpy(w.view(np.int32)).float(), to_dev(s, "bfloat16", "cpu"),
                        to_dev(b, "bfloat16", "cpu"))
    with pytest.raises(ValueError):
        QuantizedLinear(to_dev(w, device="cpu"), to_dev(s, "bfloat16", "cpu"),
                        to_dev(b, "bfloat16", "cpu"), group_size=32)
    with pytest.raises(ValueError):
        QuantizedSwitchLinear(to_dev(w, device="cpu"), to_dev(s, "bfloat16", "cpu"),
                              to_dev(b, "bfloat16", "cpu"))


def test_forward_without_gpu_fails_loudly():
    layer = _layer()
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU fallback"):
        layer(x)


# ------------------------------------------------------------------ GPU


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_dispatched_forward_matches_operator(M):
    rng = np.random.default_rng(40 + M)
    N, K = 192, 512
    w, s, b = quantized(rng, N, K)
    bias = act(rng, (N,))
    layer = QuantizedLinear(to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"),
                            bias=to_dev(bias, "bfloat16"))
    x = to_dev(act(rng, (2, M, K)), "bfloat16")
    want = bits16(mq.quantized_matmul(x, layer.weight, layer.scales, layer.biases) + layer.bias)
    base = bits16(layer(x))
    np.testing.assert_array_equal(base, want)
    dispatch.enable(layer, active=False)
    np.testing.assert_array_equal(bits16(layer(x)), want)          # outside the scope
    with dispatch.dispatch_scope():
        np.testing.assert_array_equal(bits16(layer(x)), want)
    # a table routing wide inputs through 16-row skinny launches: each row is
    # bit-identical to the two-row result (the skinny kernel's property)
    table = {(K, N): tuple(["stock"] + ["skinny"] * 64)}
    got = bits16(dispatch.quantized_matmul(x, layer.weight, layer.scales, layer.biases,
                                           group_size=64, bits=4, table=table))
    two = bits16(mq.quantized_matmul(x[:1, :2], layer.weight, layer.scales, layer.biases))
    np.testing.assert_array_equal(got[0, :2], two[0])
    assert got.shape == (2, M, N)
    dispatch.disable(layer)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [3, 40])
def test_switch_glu_matches_composition(T):
    """SwitchGLU = down(silu(gate(x)) * up(x)) per (token, expert), unsorted
    below 64 pairs and through the sort/unsort path above.  Each gather is
    checked against the oracle at the full contract, the SwiGLU step is
    rebuilt from the gathers' own outputs with the module's torch ops, and
    the module's output must equal the down gather of that, bit for bit."""
    rng = np.random.default_rng(50 + T)
    E, H, I, top = 8, 256, 128, 4
    def bank(N, K):
        parts = [quantized(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    g, u, d = bank(I, H), bank(I, H), bank(H, I)
    mods = [QuantizedSwitchLinear(to_dev(t[0]), to_dev(t[1], "bfloat16"), to_dev(t[2], "bfloat16"))
            for t in (g, u, d)]
    glu = SwitchGLU(*mods)
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, H))
    rhs = torch.from_numpy(idx).cuda()
    y = glu(to_dev(x, "bfloat16"), rhs)
    assert y.shape == (T, top, H)
    xe = to_dev(x, "bfloat16").reshape(T, 1, 1, H)
    gk, uk = mods[0](xe, rhs), mods[1](xe, rhs)                   # (T, top, 1, I)
    lhs = np.repeat(np.arange(T), top)
    for out, bk in ((gk, g), (uk, u)):
        ref = O.gather_qmm_ref(x.reshape(T, 1, H), *bk, lhs, idx.reshape(-1))
        res = O.check_output(from_dev(out).reshape(T * top, 1, I), ref)
        assert res["ok"], res
    act_ = torch.nn.functional.silu(gk.float()).to(gk.dtype)
    h = (act_.float() * uk.float()).to(gk.dtype)
    want = mods[2](h, rhs)
    np.testing.assert_array_equal(bits16(y), bits16(want.reshape(T, top, H)))
    ref = O.gather_qmm_ref(bits16(h).reshape(T * top, 1, I), *d, np.arange(T * top),
                           idx.reshape(-1))
    res = O.check_output(from_dev(y).reshape(T * top, 1, H), ref)
    assert res["ok"], res


@pytest.mark.gpu
@pytest.mark.parametrize("T", [3, 40])
def test_switch_glu_router_combine(T):
    """scores fold into one combine pass (sorted path above 64 pairs)."""
    rng = np.random.default_rng(60 + T)
    E, H, I, top = 8, 256, 128, 4
    def bank(N, K):
        parts = [quantized(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    mods = [QuantizedSwitchLinear(to_dev(t[0]), to_dev(t[1], "bfloat16"), to_dev(t[2], "bfloat16"))
            for t in (bank(I, H), bank(I, H), bank(H, I))]
    glu = SwitchGLU(*mods)
    idx = torch.from_numpy(zipf_routing(rng, T, top, E)).cuda()
    x = to_dev(act(rng, (T, H)), "bfloat16")
    scores = torch.from_numpy(rng.random((T, top)).astype(np.float32)).cuda()
    per = glu(x, idx).float()                           # (T, top, H) bf16 outputs
    want = (per * scores[..., None]).sum(-2)            # fp32 sum of the same rows
    got = glu(x, idx, scores)
    assert got.shape == (T, H)
    res = O.check_output(from_dev(got), want.cpu().numpy())
    assert res["ok"], res


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 6])
def test_switch_glu_fused_gate_up(T):
    """fuse_gate_up: one gate+up+SiLU kernel (float sums, one rounding), no
    sort, then the down gather; with scores the combine epilogue."""
    rng = np.random.default_rng(80 + T)
    E, H, I, top = 8, 256, 128, 4
    def bank(N, K):
        parts = [quantized(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    g, u, d = bank(I, H), bank(I, H), bank(H, I)
    mods = [QuantizedSwitchLinear(to_dev(t[0]), to_dev(t[1], "bfloat16"), to_dev(t[2], "bfloat16"))
            for t in (g, u, d)]
    glu = SwitchGLU(*mods, fuse_gate_up=True)
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, H))
    n0 = mq.launch_count()
    y = glu(to_dev(x, "bfloat16"), torch.from_numpy(idx).cuda())
    assert mq.launch_count() - n0 == 2                      # gate+up, down
    assert y.shape == (T, top, H)
    lhs, rhs = np.repeat(np.arange(T), top), idx.reshape(-1)
    h = O.from_f32(O.gather_glu_ref(x.reshape(T, 1, H), g, u, lhs, rhs), "bfloat16")
    ref = O.gather_qmm_ref(h.reshape(T * top, 1, I), *d, np.arange(T * top), rhs)
    res = O.check_output(from_dev(y).reshape(T * top, 1, H), ref)
    assert res["ok"], res
    scores = torch.from_numpy(rng.random((T, top)).astype(np.float32)).cuda()
    got = glu(to_dev(x, "bfloat16"), torch.from_numpy(idx).cuda(), scores)
    want = (y.float() * scores[..., None]).sum(-2)
    assert O.check_output(from_dev(got), want.cpu().numpy())["ok"]


@pytest.mark.gpu
def test_prepared_weights_follow_buffer_changes():
    """QuantizedLinear validates its weights once; replacing a buffer (new
    tensor) or loading new values in place both reach the kernel."""
    rng = np.random.default_rng(90)
    N, K = 96, 256
    w1, s1, b1 = quantized(rng, N, K)
    w2, s2, b2 = quantized(rng, N, K)
    layer = QuantizedLinear(to_dev(w1), to_dev(s1, "bfloat16"), to_dev(b1, "bfloat16"))
    x = to_dev(act(rng, (3, K)), "bfloat16")
    first = bits16(layer(x))
    layer.weight = to_dev(w2)
    layer.scales = to_dev(s2, "bfloat16")
    layer.biases = to_dev(b2, "bfloat16")
    want = bits16(mq.quantized_matmul(x, layer.weight, layer.scales, layer.biases))
    np.testing.assert_array_equal(bits16(layer(x)), want)
    layer.weight.copy_(to_dev(w1))
    layer.scales.copy_(to_dev(s1, "bfloat16"))
    layer.biases.copy_(to_dev(b1, "bfloat16"))
    np.testing.assert_array_equal(bits16(layer(x)), first)
    # another activation dtype takes the operator's composed route (MLX
    # promotes fp16 x over bf16 scales to float32)
    out = layer(x.half())
    assert out.dtype == torch.float32 and out.shape == (3, N)
    ref = O.quantized_matmul_ref(O.to_f32(bits16(x.half()), "float16"), w1,
                                 O.to_f32(s1, "bfloat16"), O.to_f32(b1, "bfloat16"), 64, 4,
                                 "float32")
    res = O.check_output(from_dev(out), ref, "float32")
    assert res["ok"], res


@pytest.mark.gpu
def test_prepared_weights_see_in_place_writes_to_copied_buffers():
    """A weight buffer the prepared path has to copy (misaligned view) and
    that is then written in place: the next forward uses the new values."""
    rng = np.random.default_rng(91)
    N, K = 64, 256
    w1, s1, b1 = quantized(rng, N, K)
    w2, _, _ = quantized(rng, N, K)
    base = torch.zeros(N * K // 8 + 1, dtype=torch.int32, device="cuda")
    base[1:].copy_(to_dev(w1).view(torch.int32).reshape(-1))
    wview = base[1:].view(N, K // 8).view(torch.uint32)        # 4 bytes off 16-byte alignment
    assert wview.data_ptr() % 16
    layer = QuantizedLinear(wview, to_dev(s1, "bfloat16"), to_dev(b1, "bfloat16"))
    x = to_dev(act(rng, (2, K)), "bfloat16")
    first = bits16(layer(x))
    base[1:].copy_(to_dev(w2).view(torch.int32).reshape(-1))   # in place, same storage
    second = bits16(layer(x))
    want = bits16(mq.quantized_matmul(x, to_dev(w2), to_dev(s1, "bfloat16"), to_dev(b1, "bfloat16")))
    np.testing.assert_array_equal(second, want)
    assert not np.array_equal(first, second)
