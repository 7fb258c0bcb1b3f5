"""Scales with |s| >= 2^100 through every matmul kernel.

The kernels dequantize with s * 2^24 folded into one fma (exact while
|s| < 2^100); larger scales must take the plain float route and still give
MLX's values.  The skinny and thin kernels choose per step, the wide tile
runs the fast route and recomputes a tile that met such a scale.  Rows with
huge scales and ordinary rows are checked against the oracle separately (the
tolerance scales with each set's own magnitude).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from oracle import oracle as O
from qmm_helpers import act, from_dev, quantized, to_dev

pytestmark = pytest.mark.gpu


def _huge(s, rows, group):
    s_f = O.to_f32(s, "bfloat16")
    s_f[rows, group] = 2.0 ** 110
    return O.from_f32(s_f, "bfloat16")


def _check_split(out, ref, huge_rows):
    rest = np.setdiff1d(np.arange(ref.shape[-1]), huge_rows)
    for cols in (huge_rows, rest):
        res = O.check_output(out[..., cols], ref[..., cols])
        assert res["ok"], res


@pytest.mark.parametrize("M", [1, 8, 40, 300])
def test_qmm_huge_scales(M):
    rng = np.random.default_rng(M)
    N, K, gs = 512, 1024, 64
    w, s, b = quantized(rng, N, K, gs)
    huge_rows = np.array([3, 260, 511])
    s = _huge(s, huge_rows, 5)
    x = act(rng, (M, K))
    out = from_dev(mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                                       to_dev(b, "bfloat16"), group_size=gs))
    ref = O.quantized_matmul_ref(x, w, s, b, gs)
    assert np.all(np.isfinite(out))
    _check_split(out, ref, huge_rows)


@pytest.mark.parametrize("M", [6, 16, 24])
def test_qmm_huge_scales_shared_x(M):
    """5-32 rows on a matrix of 48+ rows per CU: one workgroup per CU of three
    wave groups (x resident in LDS for 6 rows, staged per step for 16, two
    16-row A tiles for 24)."""
    rng = np.random.default_rng(40 + M)
    N, K, gs = 12288, 1024, 64
    w, s, b = quantized(rng, N, K, gs)
    huge_rows = np.array([3, 6000, 12287])
    s = _huge(s, huge_rows, 5)
    x = act(rng, (M, K))
    out = from_dev(mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                                       to_dev(b, "bfloat16"), group_size=gs))
    ref = O.quantized_matmul_ref(x, w, s, b, gs)
    assert np.all(np.isfinite(out))
    _check_split(out, ref, huge_rows)


def test_grouped_gather_huge_scales():
    # prefill-width gather (grouped MFMA tiles) with one expert's scales huge
    rng = np.random.default_rng(5)
    E, N, K, P = 6, 256, 512, 1200
    parts = [quantized(rng, N, K, 64) for _ in range(E)]
    w, s, b = (np.stack([p[i] for p in parts]) for i in range(3))
    huge_rows = np.array([0, 100, 255])
    s[2] = _huge(s[2], huge_rows, 1)
    idx = np.sort(rng.integers(0, E, P)).astype(np.int32)
    x = act(rng, (P, 1, K))
    out = from_dev(mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                                 to_dev(b, "bfloat16"),
                                 rhs_indices=torch.from_numpy(idx).cuda(), sorted_indices=True))
    ref = O.gather_qmm_ref(x, w, s, b, np.arange(P), idx)
    assert np.all(np.isfinite(out))
    hot = idx == 2
    _check_split(out[hot], ref[hot], huge_rows)
    res = O.check_output(out[~hot], ref[~hot])
    assert res["ok"], res
