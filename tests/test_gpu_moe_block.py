"""The decode MoE block after its router matmul as one unit (ops.moe_block):
routing (top-k, softmax, the shared expert's gate), the fused gate+up+SiLU
gather, the down projection with the combine and the shared-expert merge
folded in -- the reference's decode route and combine around its fused
decode gathers (kernels/moe_route_decode.py:151-327, 353-398;
kernels/moe_decode_fused.py:331-397).

Checked at config-4 size (512 experts, top-8, hidden 2048, intermediate
512) on MLX-quantized banks, T = 1, 4, 8 tokens: the block equals the three
steps called one by one, bit for bit; the routing equals the oracle's
exactly; each step meets the oracle on the previous step's GPU output (the
GLU and the down projection at the matmul tolerance, the combine with the
shared merge bit for bit); the routing inside the gate+up launch gives the
routing kernel's and the GLU gather's bits; the one-launch block of one
token (mq_moe_block) gives the two launches' bits on fresh routings, in
graph replays and across calls of other shapes, and so does the one-launch
block of 2-8 tokens over the gather launches' tile configurations; launch
counts (1 launch up to 8 tokens).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import _lib, ops
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, quantized, to_dev

pytestmark = pytest.mark.gpu

E, TOP, H, I = 512, 8, 2048, 512


@pytest.fixture(scope="module")
def banks():
    rng = np.random.default_rng(77)

    def bank(N, K):
        parts = [quantized(rng, N, K) for _ in range(E)]
        raw = [np.stack([p[i] for p in parts]) for i in range(3)]
        return raw, (to_dev(raw[0]), to_dev(raw[1], "bfloat16"), to_dev(raw[2], "bfloat16"))

    return bank(I, H), bank(I, H), bank(H, I)


@pytest.mark.parametrize("T", [1, 4, 8])
@pytest.mark.parametrize("with_shared", [True, False])
def test_moe_block(banks, T, with_shared):
    (graw, gate), (uraw, up), (draw, down) = banks
    rng = np.random.default_rng(T + 10 * with_shared)
    xh = act(rng, (T, H))
    x = to_dev(xh, "bfloat16")
    logits_np = rng.standard_normal((T, E)).astype(np.float32)
    logits = torch.from_numpy(logits_np).cuda()
    sgw_np = act(rng, (H,), scale=0.02)
    sgw = to_dev(sgw_np, "bfloat16") if with_shared else None
    sh_np = act(rng, (T, H), scale=0.1)
    shared = to_dev(sh_np, "bfloat16") if with_shared else None

    before = mq.launch_count()
    out = ops.moe_block(x, logits, TOP, gate, up, down, sgw=sgw, shared=shared)
    launches = mq.launch_count() - before
    # up to 8 tokens: the whole block in one launch
    assert launches == 1
    assert out.shape == (T, H)

    # the three steps one by one
    idx, w, sg = ops.moe_route(logits, TOP, x, sgw) if with_shared else ops.moe_route(logits, TOP)
    h = ops.gather_glu(x.reshape(T, 1, 1, H), *gate, *up, rhs_indices=idx)
    want = ops.gather_qmm_combine(h, *down, idx, w, sgate=sg, shared=shared)
    np.testing.assert_array_equal(bits16(out), bits16(want))
    # the routed launch's own outputs are the two launches' bits
    h2, idx2, w2, sg2 = ops._glu_routed(x, logits, TOP, gate, up, sgw, 64, 4)
    assert torch.equal(idx2, idx) and torch.equal(w2, w)
    np.testing.assert_array_equal(bits16(h2), bits16(h))
    if with_shared:
        np.testing.assert_array_equal(bits16(sg2), bits16(sg))
    else:
        assert sg2 is None

    # against the oracle, each step from the previous step's GPU output
    ridx, rw, rsg = O.moe_route_ref(logits_np, TOP, xh if with_shared else None,
                                    sgw_np if with_shared else None)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-7, atol=0)
    lhs = np.repeat(np.arange(T), TOP)
    href = O.gather_glu_ref(xh.reshape(T, 1, H), graw, uraw, lhs, ridx.reshape(-1))
    res = O.check_output(from_dev(h).reshape(T * TOP, 1, I), href)
    assert res["ok"], res
    # the down projection (the folded kernel equals gather_qmm + combine bit
    # for bit, tests/test_gpu_fold.py) at the matmul tolerance, then the
    # combine and shared merge on its rows, exactly
    y = ops.gather_qmm(h, *down, rhs_indices=idx).reshape(T * TOP, H)
    yref = O.gather_qmm_ref(bits16(h).reshape(T * TOP, 1, I), *draw, np.arange(T * TOP),
                            ridx.reshape(-1))
    res = O.check_output(from_dev(y), yref.reshape(T * TOP, H))
    assert res["ok"], res
    ref = O.moe_combine_ref(bits16(y), None, rw.reshape(-1), T, TOP,
                            sgate=bits16(sg).reshape(-1) if with_shared else None,
                            shared=sh_np if with_shared else None)
    np.testing.assert_array_equal(bits16(out), O.from_f32(ref, "bfloat16"))


@pytest.mark.parametrize("E_, top, T", [(64, 4, 16), (512, 8, 8), (100, 2, 3), (512, 1, 1)])
def test_routed_glu_matches_route_then_glu(E_, top, T):
    """Other expert counts, top-k widths and token counts (up to 64 pairs),
    logits with ties (quantized to quarters): mq_moe_glu_route equals
    mq_moe_route then mq_gather_glu, bit for bit, routing and output."""
    rng = np.random.default_rng(E_ + top + T)
    K, N = 512, 256
    def bank():
        w, s, b = quantized(rng, E_ * N, K)
        return (to_dev(w).view(E_, N, -1), to_dev(s, "bfloat16").view(E_, N, -1),
                to_dev(b, "bfloat16").view(E_, N, -1))
    gate, up = bank(), bank()
    x = to_dev(act(rng, (T, K)), "bfloat16")
    logits = torch.from_numpy((np.round(rng.standard_normal((T, E_)) * 4) / 4)
                              .astype(np.float32)).cuda()
    sgw = to_dev(act(rng, (K,), scale=0.02), "bfloat16")
    got = ops._glu_routed(x, logits, top, gate, up, sgw, 64, 4)
    assert got is not None
    h2, idx2, w2, sg2 = got
    idx, w, sg = ops.moe_route(logits, top, x, sgw)
    h = ops.gather_glu(x.reshape(T, 1, 1, K), *gate, *up, rhs_indices=idx)
    assert torch.equal(idx2, idx) and torch.equal(w2, w)
    np.testing.assert_array_equal(bits16(sg2), bits16(sg))
    np.testing.assert_array_equal(bits16(h2), bits16(h))


@pytest.mark.parametrize("T", [1, 4])
def test_routed_glu_rounds_without_expert(T):
    """Logits whose order key is 0 (the all-ones NaN pattern) are never
    chosen: with only 3 other experts, top-8 rounds 3..7 find none and
    route to -1.  The routed launch gives those pairs zero rows, as the
    GLU gather does for an out-of-range expert, and otherwise the same bits
    as the routing kernel and the GLU gather."""
    rng = np.random.default_rng(40 + T)
    E_, top, K, N = 64, 8, 512, 256
    def bank():
        w, s, b = quantized(rng, E_ * N, K)
        return (to_dev(w).view(E_, N, -1), to_dev(s, "bfloat16").view(E_, N, -1),
                to_dev(b, "bfloat16").view(E_, N, -1))
    gate, up = bank(), bank()
    x = to_dev(act(rng, (T, K)), "bfloat16")
    bits = np.full((T, E_), -1, dtype=np.int32)               # 0xffffffff: key 0
    for t in range(T):
        keep = rng.choice(E_, 3, replace=False)
        bits[t, keep] = rng.standard_normal(3).astype(np.float32).view(np.int32)
    logits = torch.from_numpy(bits.view(np.float32)).cuda()
    got = ops._glu_routed(x, logits, top, gate, up, None, 64, 4)
    assert got is not None
    h2, idx2, w2, _ = got
    idx, w, _ = ops.moe_route(logits, top)
    assert torch.equal(idx2, idx)
    assert (idx.cpu().numpy()[:, 3:] == -1).all() and (idx.cpu().numpy()[:, :3] >= 0).all()
    assert torch.equal(w2.view(torch.int32), w.view(torch.int32))
    h = ops.gather_glu(x.reshape(T, 1, 1, K), *gate, *up, rhs_indices=idx)
    np.testing.assert_array_equal(bits16(h2), bits16(h))
    assert not bits16(h2).reshape(T, top, N)[:, 3:].any()


def test_routed_glu_declines_beyond_its_range():
    """More than 64 pairs or 512 experts: the block composes the launches."""
    rng = np.random.default_rng(5)
    E_, K, N = 600, 256, 128
    w, s, b = quantized(rng, E_ * N, K)
    bank = (to_dev(w).view(E_, N, -1), to_dev(s, "bfloat16").view(E_, N, -1),
            to_dev(b, "bfloat16").view(E_, N, -1))
    x = to_dev(act(rng, (2, K)), "bfloat16")
    logits = torch.from_numpy(rng.standard_normal((2, E_)).astype(np.float32)).cuda()
    assert ops._glu_routed(x, logits, 8, bank, bank, None, 64, 4) is None


def _two_launch_block(x, logits, top, gate, up, down, sgw, shared, gs=64, bits=4):
    """The block of one token as the routed gate+up launch and the folded
    down launch (what mq_moe_block fuses)."""
    h, idx, w, sg = ops._glu_routed(x, logits, top, gate, up, sgw, gs, bits)
    return ops.gather_qmm_combine(h, *down, idx, w, group_size=gs, bits=bits, sgate=sg,
                                  shared=shared), idx, w, sg, h


def _block_launch(x, logits, top, gate, up, down, sgw, shared, bits=4, gs=64):
    before = mq.launch_count()
    out = ops.moe_block(x, logits, top, gate, up, down, sgw=sgw, shared=shared, bits=bits,
                        group_size=gs)
    assert mq.launch_count() - before == 1
    return out


def test_block_one_launch_fresh_routings(banks):
    """One token, 24 calls in a row with fresh logits (normal, zipf-skewed,
    and quantized to quarters so that ties occur), with and without the
    shared expert: the one-launch block equals the two launches bit for
    bit every time (each call's arrival flags follow the last call's)."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(2024)
    for i in range(24):
        with_shared = i % 2 == 0
        x = to_dev(act(rng, (1, H)), "bfloat16")
        lg = rng.standard_normal((1, E)).astype(np.float32)
        if i % 3 == 1:
            lg = lg - 0.5 * np.log(np.arange(1, E + 1, dtype=np.float32))
        elif i % 3 == 2:
            lg = np.round(lg * 4) / 4
        logits = torch.from_numpy(lg).cuda()
        sgw = to_dev(act(rng, (H,), scale=0.02), "bfloat16") if with_shared else None
        shared = to_dev(act(rng, (1, H), scale=0.1), "bfloat16") if with_shared else None
        out = _block_launch(x, logits, TOP, gate, up, down, sgw, shared)
        want = _two_launch_block(x, logits, TOP, gate, up, down, sgw, shared)[0]
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"call {i}")


def test_block_one_launch_outputs(banks):
    """The launch's routing, gate and h outputs are the two launches' bits."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(8)
    x = to_dev(act(rng, (1, H)), "bfloat16")
    logits = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
    sgw = to_dev(act(rng, (H,), scale=0.02), "bfloat16")
    shared = to_dev(act(rng, (1, H), scale=0.1), "bfloat16")
    want, idx, w, sg, h = _two_launch_block(x, logits, TOP, gate, up, down, sgw, shared)
    (wg, sg_, bg), (wu, su, bu), (wd, sd, bd) = gate, up, down
    idx2 = torch.empty_like(idx)
    w2 = torch.empty_like(w)
    sg2 = torch.empty_like(sg)
    h2 = torch.empty_like(h)
    out = torch.empty_like(want)
    lib = _lib.lib()
    rc = lib.mq_moe_block(x.data_ptr(), logits.data_ptr(),
                          *[t.data_ptr() for t in (wg, sg_, bg, wu, su, bu, wd, sd, bd)],
                          sgw.data_ptr(), shared.data_ptr(), idx2.data_ptr(), w2.data_ptr(),
                          sg2.data_ptr(), h2.data_ptr(), out.data_ptr(), 1, TOP, I, H, H, E,
                          64, 4, 0, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_block")
    torch.cuda.synchronize()
    assert torch.equal(idx2, idx) and torch.equal(w2, w)
    np.testing.assert_array_equal(bits16(sg2), bits16(sg))
    np.testing.assert_array_equal(bits16(h2), bits16(h))
    np.testing.assert_array_equal(bits16(out), bits16(want))


def test_block_one_launch_graph_replays(banks):
    """A captured one-token block replayed 6 times with new logits and x
    copied in between (eager two-launch blocks run between the replays):
    every replay equals the two launches on its inputs."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(99)
    x = to_dev(act(rng, (1, H)), "bfloat16")
    logits = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
    sgw = to_dev(act(rng, (H,), scale=0.02), "bfloat16")
    shared = to_dev(act(rng, (1, H), scale=0.1), "bfloat16")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            ops.moe_block(x, logits, TOP, gate, up, down, sgw=sgw, shared=shared)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.moe_block(x, logits, TOP, gate, up, down, sgw=sgw, shared=shared)
    for r in range(6):
        x.copy_(to_dev(act(rng, (1, H)), "bfloat16"))
        logits.copy_(torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda())
        g.replay()
        torch.cuda.synchronize()
        want = _two_launch_block(x, logits, TOP, gate, up, down, sgw, shared)[0]
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"replay {r}")


@pytest.mark.parametrize("dtype,bits,gs,E_,top,H_,I_", [
    ("float16", 4, 64, 128, 8, 1024, 512),
    ("bfloat16", 8, 64, 64, 4, 1024, 384),
    ("bfloat16", 4, 64, 96, 6, 1536, 320),
    ("bfloat16", 4, 128, 64, 4, 2048, 1024),
])
def test_block_one_launch_other_shapes(banks, dtype, bits, gs, E_, top, H_, I_):
    """Other dtypes, bit widths, group sizes, expert counts and widths
    (grids of 96-256 workgroups), each call followed by a call of the
    config-4 block (a grid of another size over the same arrival flags):
    both equal the two launches bit for bit."""
    (_, gate4), (_, up4), (_, down4) = banks
    rng = np.random.default_rng(E_ + top + bits)

    def bank(N, K):
        w, s_, b = quantized(rng, E_ * N, K, gs=gs, bits=bits, dtype=dtype)
        return (to_dev(w).view(E_, N, -1), to_dev(s_, dtype).view(E_, N, -1),
                to_dev(b, dtype).view(E_, N, -1))

    gate, up, down = bank(I_, H_), bank(I_, H_), bank(H_, I_)
    for i in range(3):
        x = to_dev(act(rng, (1, H_), dtype), dtype)
        logits = torch.from_numpy(rng.standard_normal((1, E_)).astype(np.float32)).cuda()
        sgw = to_dev(act(rng, (H_,), dtype, scale=0.02), dtype)
        shared = to_dev(act(rng, (1, H_), dtype, scale=0.1), dtype)
        out = _block_launch(x, logits, top, gate, up, down, sgw, shared, bits, gs)
        want = _two_launch_block(x, logits, top, gate, up, down, sgw, shared, gs, bits)[0]
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"call {i}")
        x4 = to_dev(act(rng, (1, H)), "bfloat16")
        lg4 = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
        out4 = _block_launch(x4, lg4, TOP, gate4, up4, down4, None, None)
        want4 = _two_launch_block(x4, lg4, TOP, gate4, up4, down4, None, None)[0]
        np.testing.assert_array_equal(bits16(out4), bits16(want4), err_msg=f"config-4 call {i}")


def test_block_one_launch_rounds_without_expert():
    """One token whose logits leave only 3 choosable experts: top-8 rounds
    3..7 route to -1, their pairs contribute zero rows, and the one-launch
    block equals the two launches bit for bit."""
    rng = np.random.default_rng(41)
    E_, top, H_, I_ = 64, 8, 1024, 512

    def bank(N, K):
        w, s_, b = quantized(rng, E_ * N, K)
        return (to_dev(w).view(E_, N, -1), to_dev(s_, "bfloat16").view(E_, N, -1),
                to_dev(b, "bfloat16").view(E_, N, -1))

    gate, up, down = bank(I_, H_), bank(I_, H_), bank(H_, I_)
    x = to_dev(act(rng, (1, H_)), "bfloat16")
    lb = np.full((1, E_), -1, dtype=np.int32)                # 0xffffffff: key 0
    keep = rng.choice(E_, 3, replace=False)
    lb[0, keep] = rng.standard_normal(3).astype(np.float32).view(np.int32)
    logits = torch.from_numpy(lb.view(np.float32)).cuda()
    out = _block_launch(x, logits, top, gate, up, down, None, None)
    want, idx, _, _, _ = _two_launch_block(x, logits, top, gate, up, down, None, None)
    assert (idx.cpu().numpy()[:, 3:] == -1).all()
    np.testing.assert_array_equal(bits16(out), bits16(want))


@pytest.mark.parametrize("E_,top,H_,I_,gs", [(32, 4, 512, 256, 64), (64, 8, 2048, 1024, 128)])
def test_block_one_launch_declines(E_, top, H_, I_, gs):
    """Shapes outside the one-launch kernel's tiles (gate/up K whose tiles
    split over fewer than 4 waves) or grid (more than 256 workgroups):
    moe_block runs the two launches."""
    rng = np.random.default_rng(6)

    def bank(N, K):
        w, s_, b = quantized(rng, E_ * N, K, gs=gs)
        return (to_dev(w).view(E_, N, -1), to_dev(s_, "bfloat16").view(E_, N, -1),
                to_dev(b, "bfloat16").view(E_, N, -1))

    gate, up, down = bank(I_, H_), bank(I_, H_), bank(H_, I_)
    x = to_dev(act(rng, (1, H_)), "bfloat16")
    logits = torch.from_numpy(rng.standard_normal((1, E_)).astype(np.float32)).cuda()
    before = mq.launch_count()
    out = ops.moe_block(x, logits, top, gate, up, down, group_size=gs)
    assert mq.launch_count() - before == 2
    want = _two_launch_block(x, logits, top, gate, up, down, None, None, gs)[0]
    np.testing.assert_array_equal(bits16(out), bits16(want))


def _two_launch_layer(x, idx, w, gate, up, down, gs=64, bits=4):
    h = ops.gather_glu(x.reshape(x.shape[0], 1, 1, -1), *gate, *up, rhs_indices=idx,
                       group_size=gs, bits=bits)
    return ops.gather_qmm_combine(h, *down, idx, w, group_size=gs, bits=bits)


def test_layer_one_launch(banks):
    """The decode layer of one token with its routing given (mq_moe_layer):
    24 calls with fresh experts (distinct, repeated, out of range) and
    router weights, interleaved with routed one-launch blocks (the same
    arrival flags): each equals gather_glu then gather_qmm_combine bit for
    bit, in one launch; nn.SwitchGLU(fuse_gate_up=True) takes it at T = 1."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(55)
    for i in range(24):
        x = to_dev(act(rng, (1, H)), "bfloat16")
        e = rng.choice(E, TOP, replace=False).astype(np.int32)
        if i % 4 == 1:
            e[3] = e[1]                                  # a repeated expert
        elif i % 4 == 2:
            e[5] = E + 7                                 # out of range: a zero row
        idx = torch.from_numpy(e.reshape(1, TOP)).cuda()
        w = torch.softmax(torch.from_numpy(rng.standard_normal((1, TOP)).astype(np.float32)),
                          -1).cuda()
        before = mq.launch_count()
        out = ops.moe_layer(x, idx, w, gate, up, down)
        assert mq.launch_count() - before == 1
        want = _two_launch_layer(x, idx, w, gate, up, down)
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"call {i}")
        if i % 3 == 0:
            lg = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
            ob = _block_launch(x, lg, TOP, gate, up, down, None, None)
            np.testing.assert_array_equal(
                bits16(ob), bits16(_two_launch_block(x, lg, TOP, gate, up, down, None, None)[0]))
    from mlxturbo_amd import nn as mqnn
    layer = mqnn.SwitchGLU(mqnn.QuantizedSwitchLinear(*gate), mqnn.QuantizedSwitchLinear(*up),
                           mqnn.QuantizedSwitchLinear(*down), fuse_gate_up=True)
    before = mq.launch_count()
    out = layer(x, idx, w)
    assert mq.launch_count() - before == 1
    np.testing.assert_array_equal(bits16(out), bits16(_two_launch_layer(x, idx, w, gate, up, down)))


def test_layer_one_launch_graph_replays(banks):
    """A captured one-token layer replayed 5 times with new experts,
    weights and x copied in between: every replay equals the two calls."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(7)
    x = to_dev(act(rng, (1, H)), "bfloat16")
    idx = torch.from_numpy(rng.choice(E, TOP, replace=False).astype(np.int32).reshape(1, TOP)).cuda()
    w = torch.full((1, TOP), 1.0 / TOP, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            ops.moe_layer(x, idx, w, gate, up, down)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.moe_layer(x, idx, w, gate, up, down)
    for r in range(5):
        x.copy_(to_dev(act(rng, (1, H)), "bfloat16"))
        idx.copy_(torch.from_numpy(rng.choice(E, TOP, replace=False).astype(np.int32)
                                   .reshape(1, TOP)).cuda())
        w.copy_(torch.softmax(torch.from_numpy(rng.standard_normal((1, TOP))
                                               .astype(np.float32)), -1).cuda())
        g.replay()
        torch.cuda.synchronize()
        want = _two_launch_layer(x, idx, w, gate, up, down)
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"replay {r}")


@pytest.mark.parametrize("T", [2, 3, 4, 5, 8])
def test_block_multi_token(banks, T):
    """2-8 tokens in one launch (segments of pairs sharing an expert, the
    gather launches' tile configurations: gate/up over 4 waves at T = 2, 2
    waves with the scale copy at T = 3-4, 1 wave at T = 5-8): 6 calls with
    fresh zipf-skewed and tied logits, with and without the shared expert,
    each equal to the routed gate+up launch then the down projection and the
    combine, bit for bit."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(300 + T)
    for i in range(6):
        with_shared = i % 2 == 0
        x = to_dev(act(rng, (T, H)), "bfloat16")
        lg = rng.standard_normal((T, E)).astype(np.float32)
        lg = lg - 0.5 * np.log(np.arange(1, E + 1, dtype=np.float32)) if i % 3 == 1 else lg
        lg = np.round(lg * 4) / 4 if i % 3 == 2 else lg
        logits = torch.from_numpy(lg).cuda()
        sgw = to_dev(act(rng, (H,), scale=0.02), "bfloat16") if with_shared else None
        shared = to_dev(act(rng, (T, H), scale=0.1), "bfloat16") if with_shared else None
        out = _block_launch(x, logits, TOP, gate, up, down, sgw, shared)
        want = _two_launch_block(x, logits, TOP, gate, up, down, sgw, shared)[0]
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"T={T} call {i}")


@pytest.mark.parametrize("T", [2, 4, 7])
def test_layer_multi_token(banks, T):
    """The layer of 2-8 tokens with the routing given, in one launch: repeated
    experts across tokens (shared segments), an out-of-range expert, equal to
    gather_glu then gather_qmm_combine bit for bit; interleaved with blocks
    of other token counts over the same arrival flags."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(400 + T)
    for i in range(5):
        x = to_dev(act(rng, (T, H)), "bfloat16")
        e = np.stack([rng.choice(E, TOP, replace=False) for _ in range(T)]).astype(np.int32)
        if i % 2 == 1:
            e[1:, 0] = e[0, 0]                           # one expert in every token
        if i == 3:
            e[0, 5] = E + 3                              # out of range: a zero row
        idx = torch.from_numpy(e).cuda()
        w = torch.softmax(torch.from_numpy(rng.standard_normal((T, TOP)).astype(np.float32)),
                          -1).cuda()
        before = mq.launch_count()
        out = ops.moe_layer(x, idx, w, gate, up, down)
        assert mq.launch_count() - before == 1
        np.testing.assert_array_equal(bits16(out),
                                      bits16(_two_launch_layer(x, idx, w, gate, up, down)),
                                      err_msg=f"T={T} call {i}")
        T2 = 1 + (T + i) % 8
        x2 = to_dev(act(rng, (T2, H)), "bfloat16")
        lg = torch.from_numpy(rng.standard_normal((T2, E)).astype(np.float32)).cuda()
        ob = _block_launch(x2, lg, TOP, gate, up, down, None, None)
        np.testing.assert_array_equal(
            bits16(ob), bits16(_two_launch_block(x2, lg, TOP, gate, up, down, None, None)[0]))


def test_block_multi_token_graph_replays(banks):
    """A captured 4-token block replayed 4 times with new logits and x."""
    (_, gate), (_, up), (_, down) = banks
    rng = np.random.default_rng(17)
    T = 4
    x = to_dev(act(rng, (T, H)), "bfloat16")
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    sgw = to_dev(act(rng, (H,), scale=0.02), "bfloat16")
    shared = to_dev(act(rng, (T, H), scale=0.1), "bfloat16")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            ops.moe_block(x, logits, TOP, gate, up, down, sgw=sgw, shared=shared)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.moe_block(x, logits, TOP, gate, up, down, sgw=sgw, shared=shared)
    for r in range(4):
        x.copy_(to_dev(act(rng, (T, H)), "bfloat16"))
        logits.copy_(torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda())
        g.replay()
        torch.cuda.synchronize()
        want = _two_launch_block(x, logits, TOP, gate, up, down, sgw, shared)[0]
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"replay {r}")


def test_block_multi_token_rounds_without_expert():
    """Three tokens whose logits leave 3 choosable experts each (rounds 3..7
    route to -1, zero rows), then two tokens (the 4-wave configuration), on
    a 64-expert bank: the one-launch blocks equal the two launches."""
    rng = np.random.default_rng(43)
    E_, top, H_, I_ = 64, 8, 2048, 512

    def bank(N, K):
        w, s_, b = quantized(rng, E_ * N, K)
        return (to_dev(w).view(E_, N, -1), to_dev(s_, "bfloat16").view(E_, N, -1),
                to_dev(b, "bfloat16").view(E_, N, -1))

    gate, up, down = bank(I_, H_), bank(I_, H_), bank(H_, I_)
    for T in (3, 2):
        x = to_dev(act(rng, (T, H_)), "bfloat16")
        lb = np.full((T, E_), -1, dtype=np.int32)
        for t in range(T):
            keep = rng.choice(E_, 3, replace=False)
            lb[t, keep] = rng.standard_normal(3).astype(np.float32).view(np.int32)
        logits = torch.from_numpy(lb.view(np.float32)).cuda()
        out = _block_launch(x, logits, top, gate, up, down, None, None)
        want, idx, _, _, _ = _two_launch_block(x, logits, top, gate, up, down, None, None)
        assert (idx.cpu().numpy()[:, 3:] == -1).all()
        np.testing.assert_array_equal(bits16(out), bits16(want), err_msg=f"T={T}")
