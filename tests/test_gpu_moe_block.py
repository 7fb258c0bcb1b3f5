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
shared merge bit for bit); launch counts (3 launches at T <= 2, 4 above).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import ops
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
    assert launches == (3 if T * TOP <= 16 else 4)
    assert out.shape == (T, H)

    # the three steps one by one
    idx, w, sg = ops.moe_route(logits, TOP, x, sgw) if with_shared else ops.moe_route(logits, TOP)
    h = ops.gather_glu(x.reshape(T, 1, 1, H), *gate, *up, rhs_indices=idx)
    want = ops.gather_qmm_combine(h, *down, idx, w, sgate=sg, shared=shared)
    np.testing.assert_array_equal(bits16(out), bits16(want))

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
