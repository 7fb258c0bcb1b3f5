"""GPU parity tests: HIP kernels (through the C ABI) against the CPU oracle.

Contract (tolerance in oracle.check_output): dequantize bit-exact; matmul
outputs within relL2 <= 1e-3 of round(ref) and <= 2 ulp of the fp32-
accumulated reference over dtype-rounded dequantized weights.  Full
BASELINE sizes are checked exactly where the oracle is cheap, and through
a sampled column subset plus size-independent properties (row independence
across M, sort invariance of gather) where it is not.
"""

import ctypes

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import _lib
from oracle import oracle as O
from qmm_helpers import (act, bits16, from_dev, quantized, random_packed, to_dev, uniform_routing,
                         zipf_routing)

pytestmark = pytest.mark.gpu


def _check(out_t, ref, dtype="bfloat16"):
    res = O.check_output(from_dev(out_t), ref, dtype)
    assert res["ok"], res
    return res


# ---------------------------------------------------------------- dequantize

@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_bit_exact(bits, gs, dtype):
    rng = np.random.default_rng(1000 + bits * 10 + gs)
    N, K = 67, 1024
    w, s, b = random_packed(rng, N, K, gs, bits, dtype)
    s_f = O.to_f32(s, dtype)
    s_f[0] = 0.0                                     # s = 0 -> b
    s_f[1] = -s_f[1]                                 # negative scales
    if dtype == "bfloat16":
        s_f[2] = 2.0 ** 110                          # plain-path scales (|s| >= 2^100)
        s_f[3, ::2] = 2.0 ** 101
    s = O.from_f32(s_f, dtype)
    w[4] = 0xFFFFFFFF                                # max codes
    got = mq.dequantize(to_dev(w), to_dev(s, dtype), to_dev(b, dtype), gs, bits)
    torch.cuda.synchronize()
    want = O.dequantize(w, s, b, gs, bits, dtype)
    np.testing.assert_array_equal(bits16(got), want)


def test_dequantize_nonfinite_scales():
    rng = np.random.default_rng(7)
    N, K, gs, bits = 4, 256, 64, 4
    w, s, b = random_packed(rng, N, K, gs, bits)
    s_f = O.to_f32(s, "bfloat16")
    s_f[0, 0] = np.inf
    s_f[1, 1] = np.nan
    s = O.from_f32(s_f, "bfloat16")
    got = from_dev(mq.dequantize(to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"), gs, bits))
    want = O.bf16_to_f32(O.dequantize(w, s, b, gs, bits))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    np.testing.assert_array_equal(got[fin], want[fin])


@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_float32(bits):
    rng = np.random.default_rng(11)
    N, K, gs = 33, 512, 64
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = (rng.standard_normal((N, K // gs)) * 0.01).astype(np.float32)
    b = (rng.standard_normal((N, K // gs)) * 0.01).astype(np.float32)
    got = mq.dequantize(to_dev(w), torch.from_numpy(s).cuda(), torch.from_numpy(b).cuda(), gs, bits)
    want = O.dequantize(w, s, b, gs, bits, "float32")
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_dequantize_golden_fixture():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "dequant.npz"))
    for key in sorted({k.rsplit("_", 1)[0] for k in d.files}):
        bits, gs, dtype = int(key.split("_")[0][1:]), int(key.split("_")[1][1:]), key.split("_")[2]
        got = mq.dequantize(to_dev(d[key + "_w"]), to_dev(d[key + "_s"], dtype),
                            to_dev(d[key + "_b"], dtype), gs, bits)
        np.testing.assert_array_equal(bits16(got), d[key + "_deq"])


# ------------------------------------------------------------ skinny matmul

def test_qmm_golden_fixture():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "qmm.npz"))
    for key in sorted({k.rsplit("_", 1)[0] for k in d.files}):
        M, N, K, gs, bits, dt = (int(v) for v in d[key + "_meta"])
        dtype = "bfloat16" if dt == 0 else "float16"
        out = mq.quantized_matmul(to_dev(d[key + "_x"], dtype), to_dev(d[key + "_w"]),
                                  to_dev(d[key + "_s"], dtype), to_dev(d[key + "_b"], dtype),
                                  group_size=gs, bits=bits)
        _check(out, d[key + "_ref"], dtype)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 33])
@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_vs_oracle_ragged(M, bits):
    """N not a multiple of 16 and K not a multiple of the k-block."""
    rng = np.random.default_rng(M * 10 + bits)
    N, K, gs = 1000, 4160, 64
    w, s, b = quantized(rng, N, K, gs, bits)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"), group_size=gs, bits=bits)
    _check(out, O.quantized_matmul_ref(x, w, s, b, gs, bits))


@pytest.mark.parametrize("M", [6, 12])
@pytest.mark.parametrize("gs", [32, 128])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_qmm_group_sizes_and_dtypes(M, gs, dtype):
    # M=12: 16 streamed x rows with two tiles per workgroup (gs 32), global
    # x fragments (4-bit gs 128, whose steps are 512 codes long)
    rng = np.random.default_rng(gs + M)
    N, K = 300, 2048
    for bits in (4, 8):
        w, s, b = quantized(rng, N, K, gs, bits, dtype)
        x = act(rng, (M, K), dtype)
        out = mq.quantized_matmul(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                                  group_size=gs, bits=bits)
        _check(out, O.quantized_matmul_ref(x, w, s, b, gs, bits, dtype), dtype)


def test_qmm_leading_dims():
    rng = np.random.default_rng(5)
    N, K = 256, 1024
    w, s, b = quantized(rng, N, K)
    x = act(rng, (2, 3, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"))
    assert out.shape == (2, 3, N)
    ref = O.quantized_matmul_ref(x.reshape(6, K), w, s, b).reshape(2, 3, N)
    _check(out, ref)


def test_qmm_rows_bit_identical_across_widths():
    """Each row's answer does not depend on the verify width M (the property
    the reference's qmv_small_m test pins: bench/test_qmm_smallm.py:70-85)
    for every M >= 2, which run the 16-row skinny family.  One-row calls run
    the quad kernel, which sums the same products in its own order: they
    meet the oracle and stay within the tolerance of the M >= 2 rows."""
    rng = np.random.default_rng(6)
    N, K = 2048, 5120
    w, s, b = random_packed(rng, N, K)
    x = act(rng, (16, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    full = bits16(mq.quantized_matmul(xd, *args))
    for M in (2, 3, 5, 9, 16):
        part = bits16(mq.quantized_matmul(xd[:M], *args))
        np.testing.assert_array_equal(part, full[:M])
    for v in (0, 7, 14):
        pair = bits16(mq.quantized_matmul(xd[v:v + 2], *args))
        np.testing.assert_array_equal(pair, full[v:v + 2])
    ref = O.quantized_matmul_ref(x, w, s, b)
    for v in (0, 15):
        one = mq.quantized_matmul(xd[v:v + 1], *args)
        _check(one, ref[v:v + 1])
    _check(mq.quantized_matmul(xd, *args), ref)


@pytest.mark.parametrize("N, K, bits", [(17408, 5120, 4), (5120, 17408, 4), (2048, 4096, 8),
                                        (1001, 4224, 4)])
def test_row_identity_switch(N, K, bits):
    """With mq.row_identity() one-row calls run the 2..32-row family: every
    row of a 1-, 2-, 5- or 16-row call is then bit-identical (decode equal to
    verify bit for bit, the reference's opt-in small-M guarantee,
    kernels/qmv_small_m.py:289-307).  Outside the block one-row calls are back
    on their own kernel (still within the oracle's tolerance) and the
    setting is restored."""
    rng = np.random.default_rng(N + K + bits)
    w, s, b = random_packed(rng, N, K, 64, bits)
    x = act(rng, (16, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    full = bits16(mq.quantized_matmul(xd, *args, bits=bits))
    with mq.row_identity():
        for v in (0, 5, 15):
            one = bits16(mq.quantized_matmul(xd[v:v + 1], *args, bits=bits))
            np.testing.assert_array_equal(one, full[v:v + 1])
        for M in (2, 5):
            np.testing.assert_array_equal(bits16(mq.quantized_matmul(xd[:M], *args, bits=bits)),
                                          full[:M])
    assert mq.set_row_identity(False) is False
    cols = np.unique(np.concatenate([np.arange(min(N, 64)), rng.choice(N, min(N, 64), False)]))
    one = mq.quantized_matmul(xd[3:4], *args, bits=bits)
    _check(one[:, torch.from_numpy(cols).cuda()],
           O.quantized_matmul_ref(x[3:4], w[cols], s[cols], b[cols], 64, bits))


def _qmm_abi(xd, wd, sd, bd, M, N, K, gs=64, bits=4):
    """One mq_quantized_matmul call through the C ABI (operand pointers as
    given, so a caller can pass unaligned scale views)."""
    out = torch.empty((M, N), dtype=xd.dtype, device="cuda")
    rc = _lib.lib().mq_quantized_matmul(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(),
                                        bd.data_ptr(), out.data_ptr(), M, N, K, gs, bits,
                                        0 if xd.dtype == torch.bfloat16 else 1, 1,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _lib.lib().mq_last_error()
    return out


def _unaligned(t):
    """The same values at a base 2 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    v = buf[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 == 2
    return v


@pytest.mark.parametrize("N, K", [(3500, 1024), (17408, 5120), (5120, 17408)])
def test_qmv_balanced_rows_match_tiles(N, K):
    """Launches of the 16-row skinny kernel spread the rows evenly over the
    CUs when the workgroups do not divide over them: one-row calls (N=17408
    on 256 CUs: 1280 workgroups of 13-14 rows; N=3500: 256 of 13-14; one-row
    calls take that kernel when the quad kernel declines, here scales and
    biases that are not 16-byte aligned) and two-tile calls of 9 rows
    (N=5120: 256 workgroups of 20; N=17408: one workgroup of three wave
    groups per CU).  Every row must be bit-identical to the tiled launch of a
    two-row call; the aligned one-row call (quad kernel) meets the oracle."""
    rng = np.random.default_rng(11)
    w, s, b = random_packed(rng, N, K)
    x = act(rng, (9, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    two = bits16(mq.quantized_matmul(xd[:2], *args))
    sk = _qmm_abi(xd[:1], args[0], _unaligned(args[1]), _unaligned(args[2]), 1, N, K)
    np.testing.assert_array_equal(bits16(sk)[0], two[0])
    one = mq.quantized_matmul(xd[:1], *args)
    nine = bits16(mq.quantized_matmul(xd, *args))
    np.testing.assert_array_equal(nine[:2], two)
    cols = np.concatenate([np.arange(0, 40), np.arange(N - 40, N), rng.choice(N, 80, False)])
    _check(one[:, torch.from_numpy(cols).cuda()],
           O.quantized_matmul_ref(x[:1], w[cols], s[cols], b[cols]))
    if N * K <= 4 << 20:
        _check(one, O.quantized_matmul_ref(x[:1], w, s, b))
        _check(mq.quantized_matmul(xd, *args), O.quantized_matmul_ref(x, w, s, b))


@pytest.mark.parametrize("bits, gs, dtype, N, K", [
    (4, 64, "bfloat16", 12300, 1024),    # uneven rows over the workgroups and groups
    (4, 64, "bfloat16", 12300, 1088),    # 17 groups: no scale copy, the one-group launch
    (4, 32, "float16", 13000, 2048),
    (8, 64, "bfloat16", 12288, 4096),
    (4, 128, "bfloat16", 12500, 1536),   # 8 streamed rows (longer steps stream no 16)
    (4, 64, "bfloat16", 17408, 5120),
])
def test_qmv_shared_x_groups(bits, gs, dtype, N, K):
    """5-16 rows on matrices of >= 48 rows per CU run one workgroup per CU of
    three wave groups that read x once for all of them (5-8 rows: all of x
    resident in LDS; 9-16: each step's slice staged once).  Every row must be
    bit-identical to the two-row launches (the same K split) and
    match the oracle on a column sample."""
    rng = np.random.default_rng(N + K + bits + gs)
    w, s, b = random_packed(rng, N, K, gs, bits, dtype)
    x = act(rng, (16, K), dtype, scale=0.1)
    args = (to_dev(w), to_dev(s, dtype), to_dev(b, dtype))
    xd = to_dev(x, dtype)
    two = bits16(mq.quantized_matmul(xd[:2], *args, group_size=gs, bits=bits))
    cols = np.concatenate([np.arange(0, 40), np.arange(N - 40, N), rng.choice(N, 80, False)])
    colt = torch.from_numpy(cols).cuda()
    for M in (5, 7, 8, 11, 16):
        out = mq.quantized_matmul(xd[:M], *args, group_size=gs, bits=bits)
        ob = bits16(out)
        np.testing.assert_array_equal(ob[:2], two)
        ref = O.quantized_matmul_ref(x[:M], w[cols], s[cols], b[cols], gs, bits, dtype)
        _check(out[:, colt], ref, dtype)
    pair = bits16(mq.quantized_matmul(xd[14:16], *args, group_size=gs, bits=bits))
    np.testing.assert_array_equal(ob[14:16], pair)


@pytest.mark.parametrize("bits, gs, dtype, N, K", [
    (4, 64, "bfloat16", 5120, 17408),    # the down-proj shape: 320 tiles, 8 K slices
    (4, 32, "float16", 1000, 4096),      # ragged last tile
    (8, 64, "bfloat16", 2056, 4096),
    (8, 32, "bfloat16", 640, 2048),
])
def test_qmv_split_k_slices(bits, gs, dtype, N, K):
    """5-16 rows on matrices of fewer than 640 16-row tiles, given the
    workspace (the operator passes one), run the K slices of the
    one-workgroup launch on separate workgroups and add the float planes in
    slice order in a second kernel: the bits of the plain entry point (no
    workspace, one workgroup per tile group) and of the two-row launches,
    and the oracle on a column sample."""
    rng = np.random.default_rng(N + K + bits + gs + 7)
    w, s, b = random_packed(rng, N, K, gs, bits, dtype)
    x = act(rng, (64, K), dtype, scale=0.1)
    args = (to_dev(w), to_dev(s, dtype), to_dev(b, dtype))
    xd = to_dev(x, dtype)
    lib = _lib.lib()
    two = bits16(mq.quantized_matmul(xd[:2], *args, group_size=gs, bits=bits))
    cols = np.concatenate([np.arange(0, 24), np.arange(N - 24, N), rng.choice(N, 64, False)])
    colt = torch.from_numpy(cols).cuda()
    assert lib.mq_quantized_matmul_workspace_size(4, N, K, gs, bits) == 0
    for M in (5, 8, 9, 12, 16) + ((20, 32, 40, 64) if N == 5120 else ()):
        assert lib.mq_quantized_matmul_workspace_size(M, N, K, gs, bits) == M * N * 32
        n0 = mq.launch_count()
        out = mq.quantized_matmul(xd[:M], *args, group_size=gs, bits=bits)
        assert mq.launch_count() - n0 == 2
        ob = bits16(out)
        np.testing.assert_array_equal(ob[:2], two)
        if M > 16:
            # 2 or 4 16-row A tiles: each the arithmetic of its 16-row launch
            for m0 in range(0, M, 16):
                blk = bits16(mq.quantized_matmul(xd[m0:min(M, m0 + 16)], *args, group_size=gs,
                                                 bits=bits))
                np.testing.assert_array_equal(ob[m0:m0 + 16], blk)
            M_ = 16
        else:
            M_ = M
        plain = bits16(_qmm_abi(xd[:M_], *args, M_, N, K, gs, bits))
        np.testing.assert_array_equal(ob[:M_], plain)
        ref = O.quantized_matmul_ref(x[:M], w[cols], s[cols], b[cols], gs, bits, dtype)
        _check(out[:, colt], ref, dtype)


@pytest.mark.parametrize("bits", [4, 8])
def test_qmv_two_tiles_tall_matrix(bits):
    """3-4 rows on matrices of 256+ rows per CU run two tiles per x slice;
    each row stays bit-identical to the two-row launches."""
    rng = np.random.default_rng(77 + bits)
    N, K = 65600, 1024
    w, s, b = random_packed(rng, N, K, 64, bits)
    x = act(rng, (4, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    two = bits16(mq.quantized_matmul(xd[:2], *args, bits=bits))
    pair = bits16(mq.quantized_matmul(xd[2:4], *args, bits=bits))
    cols = np.concatenate([np.arange(0, 40), np.arange(N - 40, N), rng.choice(N, 80, False)])
    for M in (3, 4):
        out = mq.quantized_matmul(xd[:M], *args, bits=bits)
        ob = bits16(out)
        np.testing.assert_array_equal(ob[:2], two)
        ref = O.quantized_matmul_ref(x[:M], w[cols], s[cols], b[cols], 64, bits)
        _check(out[:, torch.from_numpy(cols).cuda()], ref)
    np.testing.assert_array_equal(ob[2:4], pair)


@pytest.mark.parametrize("bits, gs, dtype, N, K", [
    (4, 64, "bfloat16", 12300, 1024),    # uneven rows over the workgroups and groups
    (4, 32, "float16", 13000, 2048),
    (8, 64, "bfloat16", 12288, 4096),
])
def test_qmv_two_a_tiles(bits, gs, dtype, N, K):
    """17-32 rows in one shared-x launch (two 16-row A tiles per weight
    fragment): rows bit-identical to the 16-row launches of the same rows,
    and the oracle on a column sample.  (Shapes without that launch, such as
    group size 128 or K / group_size not a multiple of 8, price 17-32 rows
    on the wide tile.)"""
    rng = np.random.default_rng(N + K + bits + gs + 1)
    w, s, b = random_packed(rng, N, K, gs, bits, dtype)
    x = act(rng, (32, K), dtype, scale=0.1)
    args = (to_dev(w), to_dev(s, dtype), to_dev(b, dtype))
    xd = to_dev(x, dtype)
    lo = bits16(mq.quantized_matmul(xd[:16], *args, group_size=gs, bits=bits))
    cols = np.concatenate([np.arange(0, 40), np.arange(N - 40, N), rng.choice(N, 80, False)])
    for M in (17, 25, 32):
        out = mq.quantized_matmul(xd[:M], *args, group_size=gs, bits=bits)
        ob = bits16(out)
        np.testing.assert_array_equal(ob[:16], lo)
        # (a block of one row is compared through a two-row call: one-row
        # calls run the quad kernel)
        lo_row = 15 if M == 17 else 16
        hi = bits16(mq.quantized_matmul(xd[lo_row:M], *args, group_size=gs, bits=bits))
        np.testing.assert_array_equal(ob[16:], hi[16 - lo_row:])
        ref = O.quantized_matmul_ref(x[:M], w[cols], s[cols], b[cols], gs, bits, dtype)
        _check(out[:, torch.from_numpy(cols).cuda()], ref, dtype)


def test_qmm_writes_every_element():
    """Output poisoned with NaN before the call; no element may stay NaN."""
    rng = np.random.default_rng(8)
    M, N, K, gs, bits = 5, 1000, 1024, 64, 4
    w, s, b = quantized(rng, N, K, gs, bits)
    x = act(rng, (M, K))
    xd, wd, sd, bd = to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16")
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    rc = _lib.lib().mq_quantized_matmul(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                                        out.data_ptr(), M, N, K, gs, bits, 0, 1,
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    np.testing.assert_array_equal(bits16(out), bits16(mq.quantized_matmul(xd, wd, sd, bd)))


def test_launch_counter_moves():
    rng = np.random.default_rng(9)
    w, s, b = quantized(rng, 64, 512)
    x = act(rng, (1, 512))
    before = mq.launch_count()
    mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    assert mq.launch_count() == before + 1


# ------------------------------------------------------ BASELINE configs 1-2

@pytest.fixture(scope="module")
def cfg2_weights():
    """K=5120 N=17408 and the transposed down-proj shape, MLX affine 4-bit g64."""
    out = {}
    for seed, (K, N) in ((1, (5120, 17408)), (2, (17408, 5120))):
        rng = np.random.default_rng(seed)
        w, s, b = quantized(rng, N, K)
        deq = O.bf16_to_f32(O.dequantize(w, s, b, 64, 4)).astype(np.float64)
        out[(K, N)] = (w, s, b, deq, (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16")))
    return out


def test_config1_qmv_4096():
    rng = np.random.default_rng(0)
    K = N = 4096
    w, s, b = quantized(rng, N, K)
    x = act(rng, (1, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                              to_dev(b, "bfloat16"))
    _check(out, O.quantized_matmul_ref(x, w, s, b))


@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120)])
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_config2_skinny(cfg2_weights, shape, M):
    K, N = shape
    w, s, b, deq, dev = cfg2_weights[shape]
    rng = np.random.default_rng(100 + M)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), *dev)
    ref = (O.bf16_to_f32(x).astype(np.float64) @ deq.T).astype(np.float32)
    _check(out, ref)


@pytest.mark.parametrize("M", [8, 13])
def test_skinny_long_k_many_rows(M):
    """K=17408 with N >= 10240 (four waves per tile): the two-tile scale copy
    would not fit, so these widths run one tile per workgroup; checked on a
    column sample and against the two-row results."""
    rng = np.random.default_rng(300 + M)
    N, K = 10256, 17408
    w, s, b = random_packed(rng, N, K)
    x = act(rng, (M, K), scale=0.1)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    xd = to_dev(x, "bfloat16")
    out = mq.quantized_matmul(xd, *args)
    cols = np.concatenate([np.arange(0, 48), np.arange(N - 40, N), rng.choice(N, 64, False)])
    ref = O.quantized_matmul_ref(x, w[cols], s[cols], b[cols])
    _check(out[:, torch.from_numpy(cols).cuda()], ref)
    pair = bits16(mq.quantized_matmul(xd[M - 2:], *args))
    np.testing.assert_array_equal(bits16(out)[M - 2:], pair)


@pytest.mark.parametrize("shape, M", [((5120, 17408), 20), ((5120, 17408), 32),
                                      ((5120, 17408), 40), ((5120, 17408), 64),
                                      ((17408, 5120), 17), ((17408, 5120), 24)])
def test_skinny_launches_above_16_rows(cfg2_weights, shape, M):
    """Widths where the wide tile would stream its weights at ~0.9 TB/s run
    as skinny launches: on the tall matrix (48+ rows per CU) up to 32 rows in
    one launch whose wave groups multiply each weight fragment with two
    16-row A tiles, on the narrow one 16 rows per launch.  Each block of 16
    rows is bit-identical to a call of those rows alone (the same K split),
    and the whole matches the oracle on sampled columns."""
    K, N = shape
    w, s, b, deq, dev = cfg2_weights[shape]
    rng = np.random.default_rng(500 + M)
    x = act(rng, (M, K))
    xd = to_dev(x, "bfloat16")
    n0 = mq.launch_count()
    out = mq.quantized_matmul(xd, *dev)
    launches, m0 = 0, 0
    while m0 < M:
        if N == 5120 and min(64, M - m0) >= 5:
            # the narrow matrix: up to 64 rows with the K slices on separate
            # workgroups, then the sum kernel
            step, n = min(64, M - m0), 2
        else:
            step, n = (32 if N == 17408 and M - m0 > 16 else 16), 1
        launches += n
        m0 += step
    assert mq.launch_count() - n0 == launches
    ob = bits16(out)
    for m0 in range(0, M, 16):
        # a block of one row through a two-row call (one-row calls: quad kernel)
        lo_row = m0 - 1 if M - m0 == 1 else m0
        part = bits16(mq.quantized_matmul(xd[lo_row:m0 + 16], *dev))
        np.testing.assert_array_equal(ob[m0:m0 + 16], part[m0 - lo_row:])
    cols = np.sort(rng.choice(N, size=512, replace=False))
    ref = (O.bf16_to_f32(x).astype(np.float64) @ deq[cols].T).astype(np.float32)
    _check(out[:, torch.from_numpy(cols).cuda()], ref)


@pytest.mark.parametrize("M", [40, 256, 512, 1000])
def test_wide_split_k_narrow_matrix(cfg2_weights, M):
    """The down-proj shape (K=17408, N=5120) at prefill widths: 20 column
    tiles, so the wide kernel splits K over workgroups into the workspace
    (float partials, reduce kernel).  Checked on sampled rows and columns
    against the oracle, and against the unsplit launch of the plain entry
    point (no workspace) to the same tolerance."""
    K, N = 17408, 5120
    w, s, b, deq, dev = cfg2_weights[(K, N)]
    lib = _lib.lib()
    assert M < 256 or lib.mq_quantized_matmul_workspace_size(M, N, K, 64, 4) > 0
    rng = np.random.default_rng(400 + M)
    x = act(rng, (M, K))
    xd = to_dev(x, "bfloat16")
    n0 = mq.launch_count()
    out = mq.quantized_matmul(xd, *dev)
    assert mq.launch_count() > n0
    rows = np.sort(rng.choice(M, size=min(M, 48), replace=False))
    cols = np.sort(rng.choice(N, size=384, replace=False))
    ref = (O.bf16_to_f32(x[rows]).astype(np.float64) @ deq[cols].T).astype(np.float32)
    sel = lambda t: t[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()]  # noqa: E731
    _check(sel(out), ref)
    plain = torch.empty_like(out)
    rc = lib.mq_quantized_matmul(xd.data_ptr(), dev[0].data_ptr(), dev[1].data_ptr(),
                                 dev[2].data_ptr(), plain.data_ptr(), M, N, K, 64, 4, 0, 1,
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    _check(sel(plain), ref)


# ------------------------------------------------- BASELINE config 3 (wide)

@pytest.mark.parametrize("M", [40, 100, 300, 600, 512, 1100, 2048, 8192])
def test_config3_wide(cfg2_weights, M):
    """Prefill widths through the MFMA tile kernel, full size; the oracle checks
    64 sampled rows x 512 sampled columns.  M=40 runs as 16-row skinny
    launches; on 256 CUs 100 / 300 / 600 / 8192 pick tile heights 64 / 128 /
    256 / 256 and 512 / 1100 / 2048 pick 192, all but 8192 with a ragged last
    row tile."""
    K, N = 5120, 17408
    w, s, b, deq, dev = cfg2_weights[(K, N)]
    rng = np.random.default_rng(300 + M)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), *dev)
    assert out.shape == (M, N) and torch.isfinite(out).all()
    rows = np.sort(rng.choice(M, size=min(M, 64), replace=False))
    cols = np.sort(rng.choice(N, size=512, replace=False))
    ref = (O.bf16_to_f32(x[rows]).astype(np.float64) @ deq[cols].T).astype(np.float32)
    got = out[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()]
    _check(got, ref)


@pytest.mark.parametrize("bits,gs,dtype,M", [(8, 64, "bfloat16", 2500), (4, 32, "float16", 2500),
                                             (8, 128, "float16", 1600)])
def test_wide_heights_other_formats(bits, gs, dtype, M):
    """8-bit codes, fp16 and other group sizes at widths whose plan takes the
    taller tiles (K=1024 N=8192, 32 column tiles: on 256 CUs M=2500 runs 14
    rows of 192, M=1600 seven rows of 256); 96 sampled rows, all columns."""
    rng = np.random.default_rng(70 + bits + gs + M)
    N, K = 8192, 1024
    w, s, b = quantized(rng, N, K, gs, bits, dtype)
    x = act(rng, (M, K), dtype)
    out = mq.quantized_matmul(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                              group_size=gs, bits=bits)
    rows = np.sort(np.concatenate([rng.choice(M, size=88, replace=False), np.arange(M - 8, M)]))
    rows = np.unique(rows)
    ref = O.quantized_matmul_ref(x[rows], w, s, b, gs, bits, dtype)
    _check(out[torch.from_numpy(rows).cuda()], ref, dtype)


@pytest.mark.parametrize("bits,gs,dtype", [(4, 64, "bfloat16"), (8, 64, "bfloat16"),
                                           (4, 32, "float16"), (8, 128, "bfloat16")])
def test_wide_ragged(bits, gs, dtype):
    """M and N not multiples of the 256 x 128 tile, full oracle."""
    rng = np.random.default_rng(31 + bits + gs)
    M, N, K = 300, 200, 1024
    w, s, b = quantized(rng, N, K, gs, bits, dtype)
    x = act(rng, (M, K), dtype)
    out = mq.quantized_matmul(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                              group_size=gs, bits=bits)
    _check(out, O.quantized_matmul_ref(x, w, s, b, gs, bits, dtype), dtype)


# ------------------------------------------------------ BASELINE config 5

@pytest.fixture(scope="module")
def lm_head_8bit():
    rng = np.random.default_rng(5)
    N, K, gs = 248320, 5120, 64
    w = rng.integers(0, 2**32, size=(N, K // 4), dtype=np.uint64).astype(np.uint32)
    s = O.from_f32((rng.random((N, K // gs)) * 0.002).astype(np.float32), "bfloat16")
    b = O.from_f32((rng.random((N, K // gs)) * 0.02 - 0.25).astype(np.float32), "bfloat16")
    return w, s, b, (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))


@pytest.mark.parametrize("M", [1, 2, 4])
def test_config5_lm_head_8bit(lm_head_8bit, M):
    """8-bit K=5120 N=248320 (1.35 GB): full-size kernel run, oracle on 3000
    sampled output columns, and the row-independence property."""
    w, s, b, dev = lm_head_8bit
    N, K, gs, bits = 248320, 5120, 64, 8
    rng = np.random.default_rng(50 + M)
    x = act(rng, (M, K))
    out = mq.quantized_matmul(to_dev(x, "bfloat16"), *dev, group_size=gs, bits=bits)
    assert out.shape == (M, N) and torch.isfinite(out).all()
    cols = np.sort(rng.choice(N, size=3000, replace=False))
    ref = O.quantized_matmul_ref(x, w[cols], s[cols], b[cols], gs, bits)
    _check(out[:, torch.from_numpy(cols).cuda()], ref)
    if M >= 2:   # rows of 2+ row calls do not depend on M (one-row calls: quad kernel)
        pair = bits16(mq.quantized_matmul(to_dev(x[-2:], "bfloat16"), *dev, group_size=gs,
                                          bits=bits))
        np.testing.assert_array_equal(pair, bits16(out)[-2:])


# ---------------------------------------------------------------- gather_qmm

def test_gather_golden_fixture():
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "gather.npz"))
    E, N, K, gs, bits = (int(v) for v in d["meta"])
    x = to_dev(d["x"], "bfloat16")                      # (T, 1, K)
    out = mq.gather_qmm(x[:, None], to_dev(d["w"]), to_dev(d["s"], "bfloat16"),
                        to_dev(d["b"], "bfloat16"), rhs_indices=torch.from_numpy(d["rhs"]).cuda(),
                        group_size=gs, bits=bits)
    T, top = d["rhs"].shape
    assert out.shape == (T, top, 1, N)
    _check(out.reshape(T * top, 1, N), d["ref"])


@pytest.fixture(scope="module")
def moe_banks():
    """Config 4: E=512, gate/up [512,1024,2048] and down [512,2048,512], 4-bit g64."""
    rng = np.random.default_rng(4)
    E = 512
    banks = {}
    for name, (N, K) in (("gate_up", (1024, 2048)), ("down", (2048, 512))):
        w = rng.integers(0, 2**32, size=(E, N, K // 8), dtype=np.uint64).astype(np.uint32)
        s = O.from_f32((rng.random((E, N, K // 64)) * 0.004).astype(np.float32), "bfloat16")
        b = O.from_f32((rng.random((E, N, K // 64)) * 0.01 - 0.03).astype(np.float32), "bfloat16")
        banks[name] = (w, s, b, (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16")))
    return banks


@pytest.mark.parametrize("routing", ["zipf", "uniform"])
@pytest.mark.parametrize("T", [1, 4, 8])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_config4_gather(moe_banks, proj, T, routing):
    w, s, b, dev = moe_banks[proj]
    E, N, Kw = w.shape
    K = Kw * 8
    rng = np.random.default_rng(40 + T)
    idx = (zipf_routing if routing == "zipf" else uniform_routing)(rng, T, 8, E)
    x = act(rng, (T, 1, 1, K))
    out = mq.gather_qmm(to_dev(x, "bfloat16"), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    assert out.shape == (T, 8, 1, N)
    lhs = np.repeat(np.arange(T), 8)
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, lhs, idx.reshape(-1))
    _check(out.reshape(T * 8, 1, N), ref)


def test_gather_sorted_matches_unsorted(moe_banks):
    """mlx-lm's _gather_sort path (rows sorted by expert, sorted_indices=True)
    gives bit-identical per-pair results (fused.py:2626-2628)."""
    w, s, b, dev = moe_banks["gate_up"]
    E, N, Kw = w.shape
    K = Kw * 8
    rng = np.random.default_rng(77)
    T = 8
    idx = zipf_routing(rng, T, 8, E)
    x = act(rng, (T, 1, 1, K))
    xd = to_dev(x, "bfloat16")
    out = bits16(mq.gather_qmm(xd, *dev, rhs_indices=torch.from_numpy(idx).cuda()))
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    xs = xd.reshape(T, 1, K)[torch.from_numpy(order // 8).cuda()]      # (P, 1, K)
    out_s = bits16(mq.gather_qmm(xs, *dev, rhs_indices=torch.from_numpy(flat[order]).cuda(),
                                 sorted_indices=True))
    np.testing.assert_array_equal(out_s.reshape(T * 8, N), out.reshape(T * 8, N)[order])


def test_gather_adversarial_and_invalid():
    rng = np.random.default_rng(12)
    E, N, K = 8, 80, 512
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    dev = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    # 40 pairs all on one expert (more than 16 pairs -> several segments)
    x = act(rng, (40, 1, K))
    idx = np.full(40, 3, np.int32)
    out = mq.gather_qmm(to_dev(x, "bfloat16"), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    _check(out, O.gather_qmm_ref(x, w, s, b, np.arange(40), idx))
    # out-of-range experts produce zero rows, the rest are unaffected
    idx2 = np.array([1, -1, 8, 2], np.int32)
    x2 = act(rng, (4, 1, K))
    out2 = from_dev(mq.gather_qmm(to_dev(x2, "bfloat16"), *dev,
                                  rhs_indices=torch.from_numpy(idx2).cuda()))
    assert np.all(out2[1] == 0) and np.all(out2[2] == 0)
    ok = np.array([0, 3])
    ref = O.gather_qmm_ref(x2, w, s, b, ok, idx2[ok])
    assert O.check_output(out2[ok], ref)["ok"]


@pytest.mark.parametrize("M,bits,gs", [(9, 4, 64), (12, 4, 32), (16, 8, 64), (16, 4, 128)])
def test_gather_many_rows_per_pair(M, bits, gs):
    """9..16 rows per pair: one pair per segment, A fragments read from
    global memory (more rows than the streamed-x capacity of a segment)."""
    rng = np.random.default_rng(50 + M + bits + gs)
    E, N, K, T, top = 8, 72, 512, 5, 3
    banks = [quantized(rng, N, K, gs=gs, bits=bits) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, 1, M, K))
    out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                        to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda(),
                        group_size=gs, bits=bits)
    assert out.shape == (T, top, M, N)
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, np.repeat(np.arange(T), top),
                           idx.reshape(-1), gs, bits)
    _check(out.reshape(T * top, M, N), ref)


@pytest.mark.parametrize("M", [1, 3])
def test_gather_large_batch_prep_path(M):
    """P > 256 pairs: segment tables built by the counting-sort prep kernel."""
    rng = np.random.default_rng(13)
    E, N, K, T, top = 16, 48, 256, 80, 4
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, 1, M, K))
    out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                        to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda())
    assert out.shape == (T, top, M, N)
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, np.repeat(np.arange(T), top), idx.reshape(-1))
    _check(out.reshape(T * top, M, N), ref)


@pytest.mark.parametrize("M,bits,gs", [(1, 4, 64), (2, 4, 64), (1, 8, 64), (3, 4, 32)])
def test_gather_prefill_grouped(M, bits, gs):
    """P * M >= 1024 rows: the expert-grouped MFMA tile kernel (prefill
    gather_qmm, moe_grouped_gemm.qmm_segmented's role); ragged N, zipf
    routing so experts get from one to hundreds of rows."""
    rng = np.random.default_rng(21 + M + bits)
    E, N, K, T, top = 16, 320, 1024, 300, 4
    banks = [quantized(rng, N, K, gs=gs, bits=bits) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, 1, M, K))
    n0 = mq.launch_count()
    out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                        to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda(),
                        group_size=gs, bits=bits)
    assert mq.launch_count() > n0
    assert out.shape == (T, top, M, N)
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, np.repeat(np.arange(T), top),
                           idx.reshape(-1), group_size=gs, bits=bits)
    _check(out.reshape(T * top, M, N), ref)


@pytest.mark.parametrize("M,bits,gs,sort", [(1, 4, 64, True), (1, 4, 64, False),
                                             (2, 8, 64, True), (2, 4, 32, False)])
def test_gather_prefill_size_classes(M, bits, gs, sort):
    """K past 2048 with few rows per expert on average: the prep tables cut
    each expert by its own row count (256-row tiles from 192 rows, 128-row
    tiles from 96, 64-row tiles below) and one grouped launch runs all classes.
    Zipf routing over 48 experts gives all three classes (43 or 85 rows per
    expert on average: below 96, where one tile height would serve all);
    expert-sorted pairs (mlx-lm's _gather_sort) and shuffled ones; ragged N."""
    rng = np.random.default_rng(90 + M + bits + gs)
    E, N, K, T, top = 48, 300, 2176, 512, 4
    banks = [quantized(rng, N, K, gs=gs, bits=bits) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E).reshape(-1).astype(np.int32)
    counts = np.bincount(idx, minlength=E) * M
    assert counts.max() >= 192 and ((counts >= 96) & (counts < 192)).any() and counts.min() < 96
    x = act(rng, (T, 1, M, K))
    xb = np.repeat(np.arange(T), top)
    order = np.argsort(idx, kind="stable") if sort else rng.permutation(idx.size)
    rhs, lhs = idx[order], xb[order]
    n0 = mq.launch_count()
    out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                        to_dev(b, "bfloat16"), lhs_indices=torch.from_numpy(lhs.astype(np.int32)).cuda(),
                        rhs_indices=torch.from_numpy(rhs).cuda(), group_size=gs, bits=bits,
                        sorted_indices=sort)
    assert mq.launch_count() - n0 == 3                 # two prep kernels + the grouped kernel
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, lhs, rhs, gs, bits)
    _check(out.reshape(idx.size, M, N), ref)


@pytest.mark.parametrize("bits,gs,dtype,K", [(4, 32, "float16", 2560), (8, 64, "bfloat16", 2560),
                                             (8, 32, "bfloat16", 2560), (4, 128, "bfloat16", 2560),
                                             (4, 32, "float16", 2048), (8, 64, "bfloat16", 2048),
                                             (4, 64, "bfloat16", 512), (8, 32, "float16", 512)])
def test_gather_prefill_scale_blocks(bits, gs, dtype, K):
    """K / gs a multiple of 8: the grouped tiles (64/128-row wide tiles past
    K=2048, the thin kernel with 8 waves at K=2048 and 4 at K=512) read
    scales and biases in 16-byte blocks of 8 groups, one load per block
    (group 32: two groups per step, the group index differs across a row's
    chunks; group 128: per-step loads, the block would span 16 steps).
    Ragged N, zipf routing, full oracle."""
    rng = np.random.default_rng(90 + bits + gs + K)
    E, N, T, top = 32, 264, 384, 4
    banks = [quantized(rng, N, K, gs=gs, bits=bits, dtype=dtype) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E).astype(np.int32)
    x = act(rng, (T, 1, 1, K), dtype)
    n0 = mq.launch_count()
    out = mq.gather_qmm(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                        rhs_indices=torch.from_numpy(idx).cuda(), group_size=gs, bits=bits)
    assert mq.launch_count() - n0 == 3                 # two prep kernels + the grouped kernel
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, np.repeat(np.arange(T), top),
                           idx.reshape(-1), gs, bits, dtype)
    res = O.check_output(from_dev(out).reshape(T * top, 1, N), ref, dtype)
    assert res["ok"], res


@pytest.mark.parametrize("M,bits,gs,dtype", [(1, 4, 64, "bfloat16"), (2, 4, 32, "float16"),
                                              (3, 8, 64, "bfloat16"), (1, 8, 128, "float16"),
                                              (5, 4, 128, "bfloat16")])
def test_gather_prefill_thin_experts(M, bits, gs, dtype):
    """Prefill widths with few rows per expert (< 96): the register-B grouped
    kernel.  Zipf routing gives experts from 1 row to several 64-row
    segments; ragged N; two invalid pairs write zero rows."""
    rng = np.random.default_rng(40 + M + bits + gs)
    E, N, K, T, top = 64, 200, 768, 256, 4
    banks = [quantized(rng, N, K, gs=gs, bits=bits, dtype=dtype) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    idx = zipf_routing(rng, T, top, E).astype(np.int32)
    idx[3, 2] = -1
    idx[T - 1, 0] = E + 5
    x = act(rng, (T, 1, M, K), dtype)
    n0 = mq.launch_count()
    out = mq.gather_qmm(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                        rhs_indices=torch.from_numpy(idx).cuda(), group_size=gs, bits=bits)
    assert mq.launch_count() - n0 == 3                 # two prep kernels + grouped kernel
    o = from_dev(out).reshape(T * top, M, N)
    flat = idx.reshape(-1)
    bad = (flat < 0) | (flat >= E)
    assert np.all(o[bad] == 0)
    ok = np.nonzero(~bad)[0]
    ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, ok // top, flat[ok], gs, bits, dtype)
    res = O.check_output(o[ok], ref, dtype)
    assert res["ok"], res


@pytest.mark.parametrize("T,top,M,K", [(150, 4, 1, 512), (300, 4, 1, 1024), (300, 4, 1, 2048),
                                        (300, 4, 1, 2560), (200, 4, 2, 512)])
def test_gather_sorted_prep_matches_counting_sort(T, top, M, K):
    """Pairs already in expert order (mlx-lm's _gather_sort) take the prep
    kernel's scan path (identity order); the same pairs shuffled take the
    counting sort.  Per-pair rows must be bit-identical, and match the
    oracle.  Covers the streaming kernel with prep tables (P*M < 1024), the
    thin kernel with 4 and 8 waves and the wide grouped kernels, runs longer
    than a segment."""
    rng = np.random.default_rng(T + top + M + K)
    E, N = 24, 160
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    dev = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    flat = np.sort(zipf_routing(rng, T, top, E).reshape(-1)).astype(np.int32)
    P = flat.size
    x = act(rng, (P, M, K))
    xd = to_dev(x, "bfloat16")
    out_sorted = bits16(mq.gather_qmm(xd, *dev, rhs_indices=torch.from_numpy(flat).cuda(),
                                      sorted_indices=True))
    shuf = rng.permutation(P)
    out_shuf = bits16(mq.gather_qmm(xd[torch.from_numpy(shuf).cuda()], *dev,
                                    rhs_indices=torch.from_numpy(flat[shuf]).cuda()))
    np.testing.assert_array_equal(out_shuf, out_sorted[shuf])
    rows = rng.choice(P, 64, replace=False)
    ref = O.gather_qmm_ref(x, w, s, b, rows, flat[rows])
    res = O.check_output(O.to_f32(out_sorted[rows].view(np.uint16), "bfloat16"), ref)
    assert res["ok"], res


def _sorted_cases(rng, E):
    """Expert lists for the prep kernels' chunk logic (chunks of 256 pairs)."""
    z = np.sort(rng.integers(0, E, 3000)).astype(np.int32)          # runs cross chunks
    halves = np.concatenate([np.sort(rng.integers(0, E, 2048)),
                             np.sort(rng.integers(0, E, 2048))]).astype(np.int32)
    one = np.concatenate([np.full(2000, 3), np.full(5, E - 1)]).astype(np.int32)
    tail = np.concatenate([np.sort(rng.integers(0, E, 1022)), [E, E + 7, 99]]).astype(np.int32)
    return {"sorted": (z, True), "two_sorted_halves": (halves, False),
            "one_hot_expert": (one, True), "invalid_tail_1025": (tail, True)}


@pytest.mark.parametrize("case", ["sorted", "two_sorted_halves", "one_hot_expert",
                                  "invalid_tail_1025"])
def test_gather_prep_chunks(case):
    """The prep's run kernel checks key order per chunk of 256 pairs (the
    first pair of a chunk against the pair before it) and, where every chunk
    is in order, writes each expert's first pair once: sorted runs crossing
    chunks, two sorted halves (a descent exactly at a chunk boundary: the
    counting sort must take over), one expert holding almost every pair
    (long gaps of absent experts), out-of-range experts sorting last (key E)
    with a one-pair last chunk.  Rows must equal the same pairs shuffled
    (counting sort) bit for bit, zero where the expert is invalid, and the
    oracle on sampled rows."""
    rng = np.random.default_rng(["sorted", "two_sorted_halves", "one_hot_expert",
                                 "invalid_tail_1025"].index(case) + 700)
    E, N, K = 24, 160, 512
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    dev = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    flat, in_order = _sorted_cases(rng, E)[case]
    assert in_order == bool(np.all(np.diff(np.where((flat >= 0) & (flat < E), flat, E)) >= 0))
    P = flat.size
    x = act(rng, (P, 1, K))
    xd = to_dev(x, "bfloat16")
    print(f"prep chunks case={case} P={P}", flush=True)
    out = bits16(mq.gather_qmm(xd, *dev, rhs_indices=torch.from_numpy(flat).cuda(),
                               sorted_indices=in_order))
    shuf = rng.permutation(P)
    out_shuf = bits16(mq.gather_qmm(xd[torch.from_numpy(shuf).cuda()], *dev,
                                    rhs_indices=torch.from_numpy(flat[shuf]).cuda()))
    np.testing.assert_array_equal(out_shuf, out[shuf])
    bad = (flat < 0) | (flat >= E)
    assert np.all(out.reshape(P, N)[bad] == 0)
    ok = np.nonzero(~bad)[0]
    rows = rng.choice(ok, 64, replace=False)
    ref = O.gather_qmm_ref(x, w, s, b, rows, flat[rows])
    res = O.check_output(O.to_f32(out[rows].view(np.uint16), "bfloat16"), ref)
    assert res["ok"], res


def test_gather_prefill_grouped_invalid_and_sorted():
    """Grouped path: out-of-range experts give zero rows; sorted input (mlx-lm
    _gather_sort) gives bit-identical per-pair rows."""
    rng = np.random.default_rng(31)
    E, N, K, T, top = 8, 256, 512, 400, 4
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    dev = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    idx = zipf_routing(rng, T, top, E).astype(np.int32)
    idx[5, 1] = -1
    idx[17, 0] = E
    x = act(rng, (T, 1, 1, K))
    xd = to_dev(x, "bfloat16")
    out = mq.gather_qmm(xd, *dev, rhs_indices=torch.from_numpy(idx).cuda())
    o = from_dev(out).reshape(T * top, N)
    flat = idx.reshape(-1)
    bad = (flat < 0) | (flat >= E)
    assert np.all(o[bad] == 0)
    ok = np.nonzero(~bad)[0]
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, ok // top, flat[ok])
    _check(out.reshape(T * top, 1, N)[torch.from_numpy(ok).cuda()], ref)
    order = np.argsort(flat, kind="stable")
    xs = xd.reshape(T, 1, K)[torch.from_numpy(order // top).cuda()]
    out_s = bits16(mq.gather_qmm(xs, *dev, rhs_indices=torch.from_numpy(flat[order]).cuda(),
                                 sorted_indices=True))
    np.testing.assert_array_equal(out_s.reshape(T * top, N), bits16(out).reshape(T * top, N)[order])



@pytest.mark.parametrize("routing", ["zipf", "uniform"])
@pytest.mark.parametrize("T", [1, 4, 8])
def test_config4_gather_glu(moe_banks, T, routing):
    """Fused gate+up+SiLU (moe_glu.fused_glu / moe_decode_fused.gate_up) on
    config 4's gate/up bank split into its gate and up halves."""
    w, s, b, dev = moe_banks["gate_up"]
    E, N2, Kw = w.shape
    N, K = N2 // 2, Kw * 8
    gate = [t[:, :N] for t in (w, s, b)]
    up = [t[:, N:] for t in (w, s, b)]
    gate_d = [t[:, :N].contiguous() for t in dev]
    up_d = [t[:, N:].contiguous() for t in dev]
    rng = np.random.default_rng(60 + T)
    idx = (zipf_routing if routing == "zipf" else uniform_routing)(rng, T, 8, E)
    x = act(rng, (T, 1, 1, K))
    out = mq.gather_glu(to_dev(x, "bfloat16"), *gate_d, *up_d,
                        rhs_indices=torch.from_numpy(idx).cuda())
    assert out.shape == (T, 8, 1, N)
    lhs = np.repeat(np.arange(T), 8)
    ref = O.gather_glu_ref(x.reshape(T, 1, K), gate, up, lhs, idx.reshape(-1))
    _check(out.reshape(T * 8, 1, N), ref)


@pytest.mark.parametrize("M,bits,gs,dtype,T", [(1, 4, 64, "bfloat16", 5), (3, 4, 32, "bfloat16", 7),
                                              (2, 8, 64, "float16", 6), (1, 4, 128, "bfloat16", 200),
                                              (5, 8, 32, "float16", 40), (12, 4, 64, "bfloat16", 9),
                                              (16, 8, 128, "float16", 3)])
def test_gather_glu_formats_and_paths(M, bits, gs, dtype, T):
    """Ragged N, every format, M rows per pair, invalid experts (zero rows),
    and P > 256 pairs (counting-sort prep tables)."""
    rng = np.random.default_rng(70 + M + bits + T)
    E, N, K, top = 12, 88, 512, 4
    def bank():
        parts = [quantized(rng, N, K, gs=gs, bits=bits, dtype=dtype) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    gate, up = bank(), bank()
    dev = lambda bk: (to_dev(bk[0]), to_dev(bk[1], dtype), to_dev(bk[2], dtype))  # noqa: E731
    idx = zipf_routing(rng, T, top, E).astype(np.int32)
    idx[0, 1] = -1
    idx[T - 1, 0] = E
    x = act(rng, (T, 1, M, K))
    out = mq.gather_glu(to_dev(x, dtype), *dev(gate), *dev(up),
                        rhs_indices=torch.from_numpy(idx).cuda(), group_size=gs, bits=bits)
    assert out.shape == (T, top, M, N)
    o = from_dev(out).reshape(T * top, M, N)
    flat = idx.reshape(-1)
    bad = (flat < 0) | (flat >= E)
    assert np.all(o[bad] == 0)
    ok = np.nonzero(~bad)[0]
    ref = O.gather_glu_ref(x.reshape(T, M, K), gate, up, ok // top, flat[ok], gs, bits, dtype)
    res = O.check_output(o[ok], ref, dtype)
    assert res["ok"], res


def test_gather_glu_prefill_composition():
    """1024+ output rows: two grouped gather_qmm calls, then SiLU-multiply in
    float of their rounded outputs.  Each gather against the oracle at the
    full contract; the composition bit for bit from the gathers' outputs."""
    rng = np.random.default_rng(91)
    E, N, K, T, top = 8, 96, 512, 300, 4
    def bank():
        parts = [quantized(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]
    gate, up = bank(), bank()
    dev = lambda bk: (to_dev(bk[0]), to_dev(bk[1], "bfloat16"), to_dev(bk[2], "bfloat16"))  # noqa: E731
    idx = zipf_routing(rng, T, top, E)
    x = act(rng, (T, 1, 1, K))
    xd, rhs = to_dev(x, "bfloat16"), torch.from_numpy(idx).cuda()
    out = mq.gather_glu(xd, *dev(gate), *dev(up), rhs_indices=rhs)
    g = mq.gather_qmm(xd, *dev(gate), rhs_indices=rhs)
    u = mq.gather_qmm(xd, *dev(up), rhs_indices=rhs)
    lhs, flat = np.repeat(np.arange(T), top), idx.reshape(-1)
    for got, bk in ((g, gate), (u, up)):
        res = O.check_output(from_dev(got).reshape(T * top, 1, N),
                             O.gather_qmm_ref(x.reshape(T, 1, K), *bk, lhs, flat))
        assert res["ok"], res
    want = (torch.nn.functional.silu(g.float()) * u.float()).to(g.dtype)
    np.testing.assert_array_equal(bits16(out), bits16(want))
    # and the whole chain against the oracle's own gathers, rounded to bf16,
    # through a float64 SiLU-multiply: the full contract holds
    rb = lambda v: O.to_f32(O.from_f32(v, "bfloat16"), "bfloat16").astype(np.float64)  # noqa: E731
    gr = rb(O.gather_qmm_ref(x.reshape(T, 1, K), *gate, lhs, flat))
    ur = rb(O.gather_qmm_ref(x.reshape(T, 1, K), *up, lhs, flat))
    ref = (gr / (1 + np.exp(-gr)) * ur).astype(np.float32)
    res = O.check_output(from_dev(out).reshape(T * top, 1, N), ref)
    assert res["ok"], res


@pytest.mark.parametrize("rows,top_k,N,sorted_", [(1, 8, 2048, False), (7, 8, 2048, True),
                                                 (2048, 8, 2048, True), (33, 2, 64, True),
                                                 (5, 3, 264, False)])
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_moe_combine(rows, top_k, N, sorted_, dtype):
    """kernels/moe_combine.py's contract: unsort + router weight + top-k sum,
    float accumulation, one rounding."""
    rng = np.random.default_rng(rows + top_k + N)
    y = O.from_f32(rng.standard_normal((rows * top_k, N)).astype(np.float32), dtype)
    w = rng.random(rows * top_k).astype(np.float32)
    inv = np.argsort(rng.permutation(rows * top_k)).astype(np.int32) if sorted_ else None
    out = mq.moe_combine(to_dev(y, dtype), torch.from_numpy(inv).cuda() if sorted_ else None,
                         torch.from_numpy(w).cuda(), rows, top_k)
    ref = O.moe_combine_ref(y, inv, w, rows, top_k, dtype)
    res = O.check_output(from_dev(out), ref, dtype)
    assert res["ok"], res
    # the same fma order as the restatement: at most a last-bit difference
    assert res["max_ulp"] <= 1.0, res


def test_gather_two_streams_own_workspaces():
    """Calls on different streams do not share the prep workspace: both
    streams run the prep path at once and match their single-stream
    results bit for bit."""
    from mlxturbo_amd import ops
    rng = np.random.default_rng(99)
    E, N, K, T, top = 16, 64, 256, 100, 4
    banks = [quantized(rng, N, K) for _ in range(E)]
    w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
    b = np.stack([t[2] for t in banks])
    dev = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    cases = []
    for _ in range(2):
        idx = torch.from_numpy(zipf_routing(rng, T, top, E)).cuda()
        x = to_dev(act(rng, (T, 1, 1, K)), "bfloat16")
        cases.append((x, idx, bits16(mq.gather_qmm(x, *dev, rhs_indices=idx))))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = []
    for st, (x, idx, _) in zip(streams, cases):
        with torch.cuda.stream(st):
            outs.append(mq.gather_qmm(x, *dev, rhs_indices=idx))
    torch.cuda.synchronize()
    for o, (_, _, want) in zip(outs, cases):
        np.testing.assert_array_equal(bits16(o), want)
    with torch.cuda.stream(streams[0]):
        w0 = ops._workspace(torch.device("cuda"), 1024)
    with torch.cuda.stream(streams[1]):
        w1 = ops._workspace(torch.device("cuda"), 1024)
    assert w0.data_ptr() != w1.data_ptr()


def test_randomized_shapes_against_oracle():
    """Seeded random small problems across every route: M from 1 to 70
    (skinny, two-tile, wide, 16-row chunks when K is not whole 64-code
    steps), N from 1, K from one group, every format; gather with random
    M rows per pair and expert counts."""
    rng = np.random.default_rng(2024)
    for case in range(24):
        bits = int(rng.choice([4, 8]))
        gs = int(rng.choice([32, 64, 128]))
        dtype = str(rng.choice(["bfloat16", "float16"]))
        K = gs * int(rng.integers(1, 12))
        N = int(rng.integers(1, 300))
        M = int(rng.choice([1, 2, 3, 5, 8, 9, 13, 16, 17, 40, 70]))
        w, s, b = quantized(rng, N, K, gs, bits, dtype)
        x = act(rng, (M, K), dtype)
        print(f"case {case}: M={M} N={N} K={K} bits={bits} gs={gs} {dtype}", flush=True)
        out = mq.quantized_matmul(to_dev(x, dtype), to_dev(w), to_dev(s, dtype), to_dev(b, dtype),
                                  group_size=gs, bits=bits)
        res = O.check_output(from_dev(out), O.quantized_matmul_ref(x, w, s, b, gs, bits, dtype), dtype)
        assert res["ok"], (case, res)
    for case in range(12):
        bits = int(rng.choice([4, 8]))
        gs = int(rng.choice([32, 64, 128]))
        K = gs * int(rng.integers(1, 8))
        N = int(rng.integers(1, 200))
        E = int(rng.integers(1, 20))
        T = int(rng.integers(1, 40))
        top = int(rng.integers(1, min(E, 6) + 1))
        M = int(rng.choice([1, 2, 4, 7, 16]))
        banks = [quantized(rng, N, K, gs, bits) for _ in range(E)]
        w = np.stack([t[0] for t in banks]); s = np.stack([t[1] for t in banks])
        b = np.stack([t[2] for t in banks])
        idx = np.stack([rng.choice(E, size=top, replace=False) for _ in range(T)]).astype(np.int32)
        x = act(rng, (T, 1, M, K))
        print(f"gather {case}: T={T} top={top} E={E} M={M} N={N} K={K} bits={bits} gs={gs}",
              flush=True)
        out = mq.gather_qmm(to_dev(x, "bfloat16"), to_dev(w), to_dev(s, "bfloat16"),
                            to_dev(b, "bfloat16"), rhs_indices=torch.from_numpy(idx).cuda(),
                            group_size=gs, bits=bits)
        ref = O.gather_qmm_ref(x.reshape(T, M, K), w, s, b, np.repeat(np.arange(T), top),
                               idx.reshape(-1), gs, bits)
        res = O.check_output(from_dev(out).reshape(T * top, M, N), ref)
        assert res["ok"], (case, res)
