"""mq_gather_qmm_combine: the MoE down projection with the combine folded in
(one or two decode tokens, up to 16 pairs), against mq_gather_qmm followed by
mq_moe_combine bit for bit, and against the oracle (gather_qmm_ref rounded to
T, then moe_combine_ref) within the tolerance contract; the shared-expert
merge against mq_moe_combine_shared; the two-pass fallback beyond 64 pairs;
SwitchGLU's router-weighted output through the folded kernel."""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd.nn import QuantizedSwitchLinear, SwitchGLU
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, quantized, to_dev, uniform_routing, zipf_routing

pytestmark = pytest.mark.gpu


def _bank(rng, E, N, K, gs=64, bits=4, dtype="bfloat16"):
    parts = [quantized(rng, N, K, gs=gs, bits=bits, dtype=dtype) for _ in range(E)]
    host = [np.stack([p[i] for p in parts]) for i in range(3)]
    return host, (to_dev(host[0]), to_dev(host[1], dtype), to_dev(host[2], dtype))


def _two_pass(xd, dev, idx_d, w_d, T, top, sgate=None, shared=None):
    y = mq.gather_qmm(xd, *dev, rhs_indices=idx_d)
    return mq.moe_combine(y.reshape(T * top, -1), None, w_d, T, top, sgate=sgate, shared=shared)


@pytest.fixture(scope="module")
def down_bank():
    """configs[3]'s down projection shape (N=2048, K=512, 4-bit g64), 64 experts."""
    return _bank(np.random.default_rng(7), 64, 2048, 512)


@pytest.mark.parametrize("T,routing", [(1, "zipf"), (2, "zipf"), (4, "zipf"), (8, "zipf"),
                                       (1, "uniform"), (8, "uniform")])
def test_fold_matches_gather_then_combine(down_bank, T, routing):
    (w, s, b), dev = down_bank
    E, N, K, top = w.shape[0], w.shape[1], w.shape[2] * 8, 8
    rng = np.random.default_rng(100 + T + (routing == "zipf"))
    idx = (zipf_routing if routing == "zipf" else uniform_routing)(rng, T, top, E)
    x = act(rng, (T, top, 1, K))
    wts = rng.random((T, top)).astype(np.float32)
    xd, idx_d, w_d = to_dev(x, "bfloat16"), torch.from_numpy(idx).cuda(), torch.from_numpy(wts).cuda()
    print(f"fold T={T} routing={routing}", flush=True)
    n0 = mq.launch_count()
    one = mq.gather_qmm_combine(xd, *dev, idx_d, w_d)
    assert mq.launch_count() - n0 == (1 if T <= 2 else 2)    # folded, or gather + combine
    two = _two_pass(xd, dev, idx_d, w_d, T, top)
    torch.cuda.synchronize()
    assert one.shape == (T, N)
    np.testing.assert_array_equal(bits16(one), bits16(two))
    y_ref = O.from_f32(O.gather_qmm_ref(x.reshape(T * top, 1, K), w, s, b, np.arange(T * top),
                                        idx.reshape(-1)).reshape(T * top, N), "bfloat16")
    ref = O.moe_combine_ref(y_ref, None, wts, T, top)
    res = O.check_output(from_dev(one), ref)
    assert res["ok"], res


@pytest.mark.parametrize("bits,gs,dtype,N,K", [(4, 32, "float16", 200, 256), (8, 64, "bfloat16", 136, 512),
                                                (4, 128, "bfloat16", 264, 1024),
                                                (8, 32, "float16", 72, 768),
                                                (4, 64, "bfloat16", 512, 768)])
@pytest.mark.parametrize("layout", ["shared_and_invalid", "distinct"])
def test_fold_formats_ragged_and_invalid(bits, gs, dtype, N, K, layout):
    """Every format, ragged N (a last workgroup with fewer than 16 columns),
    K splits of 1-4 waves, scales copied to LDS or loaded per step (K / gs =
    12: rows that are not 16-byte multiples); two tokens sharing an expert
    (a segment of two pairs) next to out-of-range experts (their terms are
    zero), or one token's four distinct experts.  Four pairs fold at every
    K split."""
    rng = np.random.default_rng(bits + gs + N)
    E = 12
    (w, s, b), dev = _bank(rng, E, N, K, gs, bits, dtype)
    if layout == "shared_and_invalid":
        T, top = 2, 2
        idx = np.array([[7, -1], [E + 3, 7]], np.int32)
    else:
        T, top = 1, 4
        idx = rng.choice(E, size=(1, top), replace=False).astype(np.int32)
    x = act(rng, (T, top, 1, K), dtype)
    wts = rng.random((T, top)).astype(np.float32)
    xd, idx_d, w_d = to_dev(x, dtype), torch.from_numpy(idx).cuda(), torch.from_numpy(wts).cuda()
    print(f"fold bits={bits} gs={gs} dtype={dtype} N={N} K={K} {layout}", flush=True)
    n0 = mq.launch_count()
    one = mq.gather_qmm_combine(xd, *dev, idx_d, w_d, group_size=gs, bits=bits)
    assert mq.launch_count() - n0 == 1
    y = mq.gather_qmm(xd, *dev, rhs_indices=idx_d, group_size=gs, bits=bits)
    two = mq.moe_combine(y.reshape(T * top, N), None, w_d, T, top)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(one), bits16(two))
    flat = idx.reshape(-1)
    ok = (flat >= 0) & (flat < E)
    y_ref = np.zeros((T * top, N), np.uint16)
    rows = np.nonzero(ok)[0]
    y_ref[rows] = O.from_f32(O.gather_qmm_ref(x.reshape(T * top, 1, K), w, s, b, rows, flat[rows],
                                              gs, bits, dtype).reshape(-1, N), dtype)
    ref = O.moe_combine_ref(y_ref, None, wts, T, top, dtype)
    res = O.check_output(from_dev(one), ref, dtype)
    assert res["ok"], res


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_fold_shared_expert(down_bank, dtype):
    rng = np.random.default_rng(33)
    if dtype == "bfloat16":
        (w, s, b), dev = down_bank
    else:
        (w, s, b), dev = _bank(rng, 16, 2048, 512, dtype=dtype)
    E, N, K, T, top = w.shape[0], w.shape[1], w.shape[2] * 8, 2, 8
    idx = uniform_routing(rng, T, top, E)
    x = act(rng, (T, top, 1, K), dtype)
    wts = rng.random((T, top)).astype(np.float32)
    sg = O.from_f32(rng.random(T).astype(np.float32), dtype)
    sh = act(rng, (T, N), dtype)
    xd, idx_d, w_d = to_dev(x, dtype), torch.from_numpy(idx).cuda(), torch.from_numpy(wts).cuda()
    sg_d, sh_d = to_dev(sg, dtype), to_dev(sh, dtype)
    n0 = mq.launch_count()
    one = mq.gather_qmm_combine(xd, *dev, idx_d, w_d, sgate=sg_d, shared=sh_d)
    assert mq.launch_count() - n0 == 1
    two = _two_pass(xd, dev, idx_d, w_d, T, top, sgate=sg_d, shared=sh_d)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(one), bits16(two))


def test_fold_beyond_16_pairs_runs_two_passes(down_bank):
    (w, s, b), dev = down_bank
    E, N, K, T, top = w.shape[0], w.shape[1], w.shape[2] * 8, 12, 8
    rng = np.random.default_rng(44)
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, top, 1, K))
    wts = rng.random((T, top)).astype(np.float32)
    xd, idx_d, w_d = to_dev(x, "bfloat16"), torch.from_numpy(idx).cuda(), torch.from_numpy(wts).cuda()
    n0 = mq.launch_count()
    one = mq.gather_qmm_combine(xd, *dev, idx_d, w_d)
    assert mq.launch_count() - n0 == 2                       # gather + combine
    two = _two_pass(xd, dev, idx_d, w_d, T, top)
    np.testing.assert_array_equal(bits16(one), bits16(two))


@pytest.mark.parametrize("fuse", [False, True])
def test_switch_glu_scores_fold(fuse):
    """SwitchGLU with router scores at decode widths: the down projection
    and the combine run as one kernel, and the result equals the explicit
    gather + combine of the same h bit for bit."""
    rng = np.random.default_rng(55 + fuse)
    E, H, I, top, T = 16, 512, 256, 4, 3

    def bank(N, K):
        parts = [quantized(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    mods = [QuantizedSwitchLinear(to_dev(t[0]), to_dev(t[1], "bfloat16"), to_dev(t[2], "bfloat16"))
            for t in (bank(I, H), bank(I, H), bank(H, I))]
    glu = SwitchGLU(*mods, fuse_gate_up=fuse)
    idx = torch.from_numpy(zipf_routing(rng, T, top, E)).cuda()
    x = to_dev(act(rng, (T, H)), "bfloat16")
    scores = torch.from_numpy(rng.random((T, top)).astype(np.float32)).cuda()
    n0 = mq.launch_count()
    got = glu(x, idx, scores)
    # the fused gate+up launch, or the gate and up gathers and the SwiGLU
    # pass; then the fold
    assert mq.launch_count() - n0 == (2 if fuse else 4)
    y = glu(x, idx)                                           # (T, top, H) per-pair outputs
    want = mq.moe_combine(y.reshape(T * top, H), None, scores.reshape(-1), T, top)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits16(got), bits16(want))
