"""Gathers whose x batches repeat over consecutive pairs pass no index table.

Tokens ``(T, 1)`` broadcast against their expert indices ``(T, top_k)`` (mlx-lm's
SwitchGLU call) reach the C ABI with a NULL lhs, pair p reading x batch
p / (P / B).  Every kernel route must give exactly what the same call gives
with the explicit index table, and the oracle's answer.
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from oracle import oracle as O
from qmm_helpers import act, from_dev, quantized, to_dev

pytestmark = pytest.mark.gpu


def _bank(rng, E, N, K, gs=64, bits=4):
    parts = [quantized(rng, N, K, gs, bits) for _ in range(E)]
    return tuple(np.stack([p[i] for p in parts]) for i in range(3))


# (T, top_k, M): wave-level segment discovery (P <= 64), LDS discovery
# (P <= 256), prep kernel + decode tiles, prep kernel + grouped MFMA tiles
ROUTES = [(4, 8, 1), (24, 8, 1), (100, 8, 1), (300, 8, 1), (6, 4, 3), (90, 4, 3)]


@pytest.mark.parametrize("T,top,M", ROUTES)
def test_repeated_batches_match_explicit_table(T, top, M):
    rng = np.random.default_rng(T * 10 + M)
    E, N, K = 40, 128, 256
    bank = _bank(rng, E, N, K)
    w, s, b = (to_dev(a, d) for a, d in zip(bank, (None, "bfloat16", "bfloat16")))
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    idx[1, 2] = -1                                              # an invalid pair: zero rows
    x_np = act(rng, (T, 1, M, K))
    x = to_dev(x_np, "bfloat16")
    rhs = torch.from_numpy(idx).cuda()
    lhs = torch.arange(T, device="cuda", dtype=torch.int32)[:, None].expand(T, top)
    print(f"repeat broadcast T={T} top={top} M={M}", flush=True)
    got = mq.gather_qmm(x, w, s, b, rhs_indices=rhs)
    want = mq.gather_qmm(x, w, s, b, lhs_indices=lhs.contiguous(), rhs_indices=rhs)
    torch.cuda.synchronize()
    assert got.shape == (T, top, M, N)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    out = from_dev(got).reshape(T * top, M, N)
    assert np.all(out[1 * top + 2] == 0)
    ok = np.flatnonzero(idx.reshape(-1) >= 0)
    ref = O.gather_qmm_ref(x_np.reshape(T, M, K), *bank, ok // top, idx.reshape(-1)[ok])
    res = O.check_output(out[ok], ref)
    assert res["ok"], res


def test_single_batch_serves_every_pair():
    # x (1, M, K) against indices (T, top_k): B = 1, every pair reads batch 0
    rng = np.random.default_rng(3)
    E, N, K, T, top = 16, 64, 128, 9, 4
    bank = _bank(rng, E, N, K)
    w, s, b = (to_dev(a, d) for a, d in zip(bank, (None, "bfloat16", "bfloat16")))
    idx = rng.integers(0, E, (T, top)).astype(np.int32)
    x_np = act(rng, (1, 2, K))
    got = mq.gather_qmm(to_dev(x_np, "bfloat16"), w, s, b,
                        rhs_indices=torch.from_numpy(idx).cuda())
    assert got.shape == (T, top, 2, N)
    ref = O.gather_qmm_ref(x_np, *bank, np.zeros(T * top, np.int64), idx.reshape(-1))
    res = O.check_output(from_dev(got).reshape(T * top, 2, N), ref)
    assert res["ok"], res


@pytest.mark.parametrize("T", [3, 20, 60])
def test_glu_repeated_batches_match_explicit_table(T):
    rng = np.random.default_rng(50 + T)
    E, N, K, top = 24, 64, 256, 8
    gate = [to_dev(a, d) for a, d in zip(_bank(rng, E, N, K), (None, "bfloat16", "bfloat16"))]
    up = [to_dev(a, d) for a, d in zip(_bank(rng, E, N, K), (None, "bfloat16", "bfloat16"))]
    idx = np.stack([rng.choice(E, top, replace=False) for _ in range(T)]).astype(np.int32)
    x = to_dev(act(rng, (T, 1, 1, K)), "bfloat16")
    rhs = torch.from_numpy(idx).cuda()
    lhs = torch.arange(T, device="cuda", dtype=torch.int32)[:, None].expand(T, top).contiguous()
    got = mq.gather_glu(x, *gate, *up, rhs_indices=rhs)
    want = mq.gather_glu(x, *gate, *up, lhs_indices=lhs, rhs_indices=rhs)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
