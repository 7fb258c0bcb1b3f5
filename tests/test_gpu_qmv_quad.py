"""GPU parity of the one-row quad kernel (csrc/qmv_quad.cuh) against the oracle.

One-row calls (decode, M = 1: the reference's mx.quantized_matmul -> MLX qmv,
dispatch.py:317-327) run a kernel of their own: a wave per quad of 4 weight
rows reading 256 contiguous bytes of each per load instruction, the x slab
of the instruction coalesced, 4x4x4 MFMAs with each lane's own x piece as A.
Covered here: every format (4/8 bits, group 32/64/128, bf16/fp16), rows not
a multiple of 4, K not a multiple of the 256-byte instruction (the scale copy
zeroes groups past the row, the x slab reads zeros past K), rows shorter than
one instruction, every K split (1-8 waves per quad), scales that need the
plain float route, NaN/inf propagation, and operands that make the kernel
decline (the 16-row family then runs, bit-identical to its two-row calls).
Tolerance: oracle.check_output (relL2 <= 1e-3, 2 ulp at the rms floor).
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import _lib
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, quantized, random_packed, to_dev

pytestmark = pytest.mark.gpu


def _check(out_t, ref, dtype="bfloat16"):
    res = O.check_output(from_dev(out_t), ref, dtype)
    assert res["ok"], res
    return res


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N, K", [(37, 384), (1001, 4224), (258, 5120), (6, 256)])
def test_quad_formats_and_ragged_shapes(N, K, bits, gs, dtype):
    """N = 37, 1001, 258, 6: partial last quads; K = 384 / 4224 at 4 bits
    (192 / 2112 bytes per row: less than one instruction, and 8.25 of
    them), K = 256: one short instruction; every case against the oracle."""
    if K % gs:
        pytest.skip("K must be a multiple of the group size")
    rng = np.random.default_rng(N * 7 + K + bits * 3 + gs)
    w, s, b = quantized(rng, N, K, gs, bits, dtype)
    x = act(rng, (1, K), dtype)
    out = mq.quantized_matmul(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                              group_size=gs, bits=bits)
    _check(out, O.quantized_matmul_ref(x, w, s, b, gs, bits, dtype), dtype)


@pytest.mark.parametrize("N, K", [(8, 17408), (40, 8192), (200, 4096), (1200, 2048),
                                  (5120, 17408)])
@pytest.mark.parametrize("bits", [4, 8])
def test_quad_k_splits(N, K, bits):
    """Few quads split K over 2-8 waves of a workgroup (partials summed in
    LDS in wave order): N = 8 and 40 take 8 waves, 200 four or two, 1200 two,
    and the down-proj shape K=17408 N=5120 four; sampled columns against the
    oracle, and the result is the same on a second call (fixed order)."""
    rng = np.random.default_rng(N + K + bits)
    w, s, b = random_packed(rng, N, K, 64, bits)
    x = act(rng, (1, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    out = mq.quantized_matmul(xd, *args, bits=bits)
    again = mq.quantized_matmul(xd, *args, bits=bits)
    np.testing.assert_array_equal(bits16(out), bits16(again))
    cols = np.unique(np.concatenate([np.arange(0, min(N, 40)), np.arange(max(0, N - 40), N),
                                     rng.choice(N, min(N, 80), False)]))
    ref = O.quantized_matmul_ref(x, w[cols], s[cols], b[cols], 64, bits)
    _check(out[:, torch.from_numpy(cols).cuda()], ref)


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("extra, K, bits", [(64, 4096, 4), (64, 2048, 8), (300, 4096, 4),
                                            (3, 1024, 4)])
@pytest.mark.parametrize("ragged", [0, 2])
def test_quad_tail_split(extra, K, bits, ragged):
    """One wave per quad over 4 x CUs SIMDs and `extra` quads more: those
    leftover quads run split over 4 waves (extra <= CUs; K = 1024 at 4 bits
    has 2 instructions, so 2 waves there) or 2 (300 on 256 CUs), the full
    quads 4 or 2 to a workgroup, one wave each.  Rows of both kinds, a
    partial last quad (ragged), the whole output against the oracle; the
    same result on a second call; one launch."""
    N = 4 * (4 * _cus() + extra) - ragged
    rng = np.random.default_rng(extra + K + bits + ragged)
    w, s, b = quantized(rng, N, K, 64, bits)
    x = act(rng, (1, K))
    args = (to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    before = mq.launch_count()
    out = mq.quantized_matmul(*args, bits=bits)
    assert mq.launch_count() == before + 1
    again = mq.quantized_matmul(*args, bits=bits)
    np.testing.assert_array_equal(bits16(out), bits16(again))
    _check(out, O.quantized_matmul_ref(x, w, s, b, 64, bits))


@pytest.mark.parametrize("bits", [4, 8])
def test_quad_plain_route(bits):
    """Scales of 2^100 and beyond overflow the fast dequant's s * 2^24; a wave
    whose scale copy holds one runs the plain float route.  Rows with huge
    scales and their neighbours (same wave) against the oracle."""
    rng = np.random.default_rng(90 + bits)
    N, K, gs = 333, 1024, 64
    w, s, b = quantized(rng, N, K, gs, bits)
    sf = O.bf16_to_f32(s).copy()
    for r in (2, 130, 331):
        sf[r, ::3] = np.float32(2.0 ** 110) * np.sign(sf[r, ::3] + 1e-30)
    s = O.from_f32(sf, "bfloat16")
    x = act(rng, (1, K), scale=2.0 ** -100)
    out = from_dev(mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                                       to_dev(b, "bfloat16"), group_size=gs, bits=bits))
    ref = O.quantized_matmul_ref(x, w, s, b, gs, bits)
    assert np.all(np.isfinite(out))
    for cols in (np.array([0, 1, 2, 3, 128, 129, 130, 131, 328, 329, 330, 331, 332]),
                 np.setdiff1d(np.arange(N), [2, 130, 331])):
        res = O.check_output(out[..., cols], ref[..., cols])
        assert res["ok"], res


def test_quad_nan_inf_propagate():
    """A NaN scale makes its row NaN (0 * NaN and q * NaN are NaN in MLX's
    float arithmetic too); an inf x element makes every row with a nonzero
    dequantized weight there inf or NaN; other rows are unaffected."""
    rng = np.random.default_rng(5)
    N, K = 64, 1024
    w, s, b = quantized(rng, N, K)
    x = act(rng, (1, K))
    s_nan = s.copy()
    s_nan[9, 3] = 0x7FC0                 # bf16 NaN
    out = from_dev(mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s_nan, "bfloat16"),
                                       to_dev(b, "bfloat16")))
    assert np.isnan(out[0, 9])
    keep = np.setdiff1d(np.arange(N), [9])
    ref = O.quantized_matmul_ref(x, w, s, b)
    res = O.check_output(out[:, keep], ref[:, keep])
    assert res["ok"], res
    x_inf = x.copy()
    x_inf[0, 700] = 0x7F80               # bf16 +inf
    out = from_dev(mq.quantized_matmul(to_dev(x_inf, "bfloat16"), to_dev(w),
                                       to_dev(s, "bfloat16"), to_dev(b, "bfloat16")))
    deq = O.bf16_to_f32(O.dequantize(w, s, b))[:, 700]
    assert np.all(~np.isfinite(out[0, deq != 0]))


def test_quad_declines_unaligned_to_skinny():
    """Scale and bias pointers off a 16-byte boundary (possible through the C
    ABI only: the Python layer aligns its operands) make the quad kernel
    decline; the 16-row kernel's one-row launch then runs and is bit-identical
    to the two-row call's first row."""
    rng = np.random.default_rng(12)
    N, K = 1000, 2048
    w, s, b = random_packed(rng, N, K)
    x = act(rng, (2, K), scale=0.1)
    xd, wd = to_dev(x, "bfloat16"), to_dev(w)
    sd, bd = to_dev(s, "bfloat16"), to_dev(b, "bfloat16")

    def unaligned(t):
        buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
        v = buf[1:1 + t.numel()].view(t.shape)
        v.copy_(t)
        return v

    su, bu = unaligned(sd), unaligned(bd)
    out = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    before = mq.launch_count()
    rc = _lib.lib().mq_quantized_matmul(xd.data_ptr(), wd.data_ptr(), su.data_ptr(),
                                        bu.data_ptr(), out.data_ptr(), 1, N, K, 64, 4, 0, 1,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert mq.launch_count() == before + 1
    two = bits16(mq.quantized_matmul(xd, wd, sd, bd))
    np.testing.assert_array_equal(bits16(out)[0], two[0])
    _check(out, O.quantized_matmul_ref(x[:1], w, s, b))


def test_quad_config2_full():
    """Config 2's M = 1 (K=5120 N=17408, the north-star shape) in full against
    the oracle on MLX-quantized N(0, 0.02) weights."""
    rng = np.random.default_rng(1)
    N, K = 17408, 5120
    w, s, b = quantized(rng, N, K)
    x = act(rng, (1, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"))
    _check(out, O.quantized_matmul_ref(x, w, s, b))
