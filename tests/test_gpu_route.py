"""GPU parity of the MoE routing kernel and the shared-expert combine.

``moe_route`` (mq_moe_route) against ``oracle.moe_route_ref``: the expert
indices exactly (distinct logits, heavy ties, -0/+0, E not a multiple of 64,
top_k up to 64), the weights to a few float32 ulps (the kernel's exp is
not the oracle's correctly rounded one), the shared-expert gate exactly when
the dot product is exact in float32 and within one T ulp otherwise.
``moe_combine`` with the shared expert against ``oracle.moe_combine_ref``
bit for bit, with and without an unsort table.
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _check_route(logits, k, got_idx, got_w):
    ref_idx, ref_w, _ = O.moe_route_ref(logits, k)
    np.testing.assert_array_equal(got_idx, ref_idx)
    # expf is within 2 ulp of the correctly rounded exp; the sum and the
    # division carry it: 4 float32 ulps of relative error
    np.testing.assert_allclose(got_w, ref_w, rtol=4.8e-7, atol=1e-30)


@pytest.mark.parametrize("rows,E,k", [(1, 512, 8), (3, 512, 10), (8, 128, 8), (100, 64, 2),
                                      (5, 1000, 32), (2, 1024, 64), (4, 8, 8), (7, 37, 1)])
def test_route_distinct_logits(rows, E, k):
    rng = np.random.default_rng(rows * 1000 + E + k)
    logits = (rng.standard_normal((rows, E)) * 3).astype(np.float32)
    print(f"route rows={rows} E={E} k={k}", flush=True)
    idx, w, sg = mq.moe_route(torch.from_numpy(logits).cuda(), k)
    torch.cuda.synchronize()
    assert sg is None
    _check_route(logits, k, idx.cpu().numpy(), w.cpu().numpy())


def test_route_ties_and_signed_zero():
    rng = np.random.default_rng(9)
    rows, E, k = 6, 512, 16
    logits = rng.integers(-3, 4, (rows, E)).astype(np.float32) / 2   # many equal values
    logits[0, :] = 0.0
    logits[0, 1::3] = -0.0
    logits[1, 300] = 7.0
    logits[1, 5] = 7.0
    idx, w, _ = mq.moe_route(torch.from_numpy(logits).cuda(), k)
    torch.cuda.synchronize()
    _check_route(logits, k, idx.cpu().numpy(), w.cpu().numpy())


def test_route_batched_shape():
    rng = np.random.default_rng(10)
    logits = rng.standard_normal((2, 3, 256)).astype(np.float32)
    idx, w, _ = mq.moe_route(torch.from_numpy(logits).cuda(), 8)
    torch.cuda.synchronize()
    assert idx.shape == (2, 3, 8)
    _check_route(logits.reshape(6, 256), 8, idx.cpu().numpy().reshape(6, 8),
                 w.cpu().numpy().reshape(6, 8))


@pytest.mark.parametrize("dtype,H", [("bfloat16", 2560), ("float16", 2560), ("bfloat16", 1001)])
def test_route_shared_gate_exact_dot(dtype, H):
    # small dyadic values: every partial sum is exact in float32, so the
    # kernel's T(dot) is the oracle's and the sigmoid must match bit for bit
    # (H = 1001: rows neither a multiple of 8 long nor 16-byte aligned)
    rng = np.random.default_rng(11)
    rows, E = 8, 512
    x = O.from_f32((rng.integers(-8, 9, (rows, H)) / 64.0).astype(np.float32), dtype)
    g = O.from_f32((rng.integers(-8, 9, H) / 256.0).astype(np.float32), dtype)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    idx, w, sg = mq.moe_route(torch.from_numpy(logits).cuda(), 8, to_dev(x, dtype), to_dev(g, dtype))
    torch.cuda.synchronize()
    ref_idx, ref_w, ref_sg = O.moe_route_ref(logits, 8, x, g, dtype)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_array_equal(bits16(sg).reshape(-1), O.from_f32(ref_sg, dtype))


def test_route_shared_gate_random_dot():
    rng = np.random.default_rng(12)
    rows, E, H = 4, 512, 2560
    x = act(rng, (rows, H))
    g = act(rng, (H,), scale=0.02)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    _, _, sg = mq.moe_route(torch.from_numpy(logits).cuda(), 8, to_dev(x, "bfloat16"),
                            to_dev(g, "bfloat16"))
    torch.cuda.synchronize()
    _, _, ref_sg = O.moe_route_ref(logits, 8, x, g)
    got = from_dev(sg).reshape(-1)
    assert np.all(np.abs(got - ref_sg) <= O.ulp_bf16(ref_sg))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("with_inv", [False, True])
def test_combine_with_shared_expert(dtype, with_inv):
    rng = np.random.default_rng(13 + with_inv)
    rows, k, N = 8, 8, 2560
    y = act(rng, (rows * k, N), dtype)
    w = rng.random(rows * k).astype(np.float32)
    sg = O.from_f32(rng.random(rows).astype(np.float32), dtype)
    sh = act(rng, (rows, N), dtype)
    inv = rng.permutation(rows * k).astype(np.int32) if with_inv else None
    out = mq.moe_combine(to_dev(y, dtype), torch.from_numpy(inv).cuda() if with_inv else None,
                         torch.from_numpy(w).cuda(), rows, k, sgate=to_dev(sg, dtype),
                         shared=to_dev(sh, dtype))
    torch.cuda.synchronize()
    ref = O.moe_combine_ref(y, inv, w, rows, k, dtype, sgate=sg, shared=sh)
    np.testing.assert_array_equal(bits16(out), O.from_f32(ref, dtype))
