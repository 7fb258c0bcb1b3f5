"""GPU parity at the BASELINE.json configurations with the weights it names:
fp32 N(0, 0.02) cast to bf16 and quantized with MLX's affine quantizer
(this library's mq_quantize, itself checked bit for bit against
``oracle.quantize`` on sampled rows here and on every branch in
test_gpu_formats.py), as the reference builds its own test weights
(tools/qmm_wide_micro.py:160, kernels/moe_verify_gather.py:885-887).

Also the production-scale gather paths: prefill at 2048, 4096 and 8192
tokens x top-8 on the config-4 banks (16384 to 65536 pairs; above 24576 the
prep kernel reads keys from memory instead of LDS), sorted and shuffled,
fp16 8-bit, and a bank of 1024+ experts; the (K=21504, N=5376) geometry of
the reference's route table (dispatch.py:67); and a class-patched
QuantizedLinear (fast_qmm.py:395-472).  Full problems run on the GPU; the
oracle checks sampled rows or columns.
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import dispatch
from mlxturbo_amd.nn import QuantizedLinear
from oracle import oracle as O
from qmm_helpers import act, bits16, from_dev, to_dev, uniform_routing, zipf_routing

pytestmark = pytest.mark.gpu


def _gauss_bf16(shape, seed, sigma=0.02):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * sigma
            ).to(torch.bfloat16)


def _mlx_quantized(shape, seed, bits=4, gs=64, check_rows=32):
    """BASELINE weights on the GPU; the quantizer is checked bit for bit
    against the oracle on ``check_rows`` sampled rows."""
    wf = _gauss_bf16(shape, seed)
    wq, s, b = mq.quantize(wf, group_size=gs, bits=bits)
    flat = wf.reshape(-1, shape[-1])
    rows = torch.from_numpy(np.random.default_rng(seed).choice(flat.shape[0], check_rows,
                                                               replace=False)).cuda()
    wr = from_dev(flat[rows])                                 # bf16 values as float32
    ewq, es, eb = O.quantize(wr, gs, bits, "bfloat16")
    np.testing.assert_array_equal(from_dev(_take(wq.reshape(-1, wq.shape[-1]), rows)), ewq)
    np.testing.assert_array_equal(bits16(s.reshape(-1, s.shape[-1])[rows]), es)
    np.testing.assert_array_equal(bits16(b.reshape(-1, b.shape[-1])[rows]), eb)
    del wf
    return wq, s, b


def _host(t):
    return from_dev(t) if t.dtype == torch.uint32 else bits16(t)


def _take(t, idx):
    """t[idx] along dim 0 (uint32 through an int32 view: torch has no uint32
    indexing kernel)."""
    if t.dtype == torch.uint32:
        return t.view(torch.int32)[idx].view(torch.uint32)
    return t[idx]


def _cols(t, sl):
    """t[:, sl].contiguous(), uint32 through an int32 view."""
    if t.dtype == torch.uint32:
        return t.view(torch.int32)[:, sl].contiguous().view(torch.uint32)
    return t[:, sl].contiguous()


def _check(out, ref, dtype="bfloat16"):
    res = O.check_output(from_dev(out) if isinstance(out, torch.Tensor) else out, ref, dtype)
    assert res["ok"], res
    return res


# ------------------------------------------------------------ config 4 decode

@pytest.fixture(scope="module")
def mlx_banks():
    """Config 4: E=512 experts, gate/up [512, 1024, 2048], down [512, 2048, 512]."""
    banks = {}
    for i, (name, (N, K)) in enumerate((("gate_up", (1024, 2048)), ("down", (2048, 512)))):
        dev = _mlx_quantized((512, N, K), 400 + i)
        banks[name] = (tuple(_host(t) for t in dev), dev)
    return banks


@pytest.mark.parametrize("routing", ["zipf", "uniform"])
@pytest.mark.parametrize("T", [1, 4, 8])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_config4_on_mlx_quantized_banks(mlx_banks, proj, T, routing):
    (w, s, b), dev = mlx_banks[proj]
    E, N, Kw = w.shape
    K = Kw * 8
    rng = np.random.default_rng(440 + T)
    idx = (zipf_routing if routing == "zipf" else uniform_routing)(rng, T, 8, E)
    x = act(rng, (T, 1, 1, K))
    print(f"config4 {proj} T={T} {routing}", flush=True)
    out = mq.gather_qmm(to_dev(x, "bfloat16"), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), w, s, b, np.repeat(np.arange(T), 8),
                           idx.reshape(-1))
    _check(out.reshape(T * 8, 1, N), ref)


def test_config4_glu_on_mlx_quantized_banks(mlx_banks):
    """The fused gate+up+SiLU kernel on the same banks (gate = first half of
    the 1024 rows, up = second half)."""
    (w, s, b), dev = mlx_banks["gate_up"]
    T = 8
    rng = np.random.default_rng(45)
    idx = zipf_routing(rng, T, 8, 512)
    x = act(rng, (T, 1, 1, 2048))
    g = tuple(_cols(t, slice(0, 512)) for t in dev)
    u = tuple(_cols(t, slice(512, 1024)) for t in dev)
    out = mq.gather_glu(to_dev(x, "bfloat16"), *g, *u, rhs_indices=torch.from_numpy(idx).cuda())
    lhs, rhs = np.repeat(np.arange(T), 8), idx.reshape(-1)
    ref = O.gather_glu_ref(x.reshape(T, 1, 2048), (w[:, :512], s[:, :512], b[:, :512]),
                           (w[:, 512:], s[:, 512:], b[:, 512:]), lhs, rhs)
    _check(out.reshape(T * 8, 1, 512), ref)


# ------------------------------------------------------- prefill at scale

def _prefill_case(dev, host, T, top, seed, sort, dtype="bfloat16", sample=48):
    E, N, Kw = host[0].shape
    K = dev[1].shape[-1] * 64
    bits = Kw * 32 // K
    rng = np.random.default_rng(seed)
    idx = zipf_routing(rng, T, top, E) if E >= top else None
    x = act(rng, (T, 1, 1, K), dtype)
    xd = to_dev(x, dtype)
    flat = idx.reshape(-1)
    P = flat.size
    if sort:
        order = np.argsort(flat, kind="stable")
        lhs = order // top
        rhs = flat[order]
        xs = xd.reshape(T, 1, K)[torch.from_numpy(lhs).cuda()]            # (P, 1, K)
        print(f"prefill T={T} P={P} sorted {dtype}", flush=True)
        out = mq.gather_qmm(xs, *dev, rhs_indices=torch.from_numpy(rhs).cuda(),
                            sorted_indices=True, bits=bits)
    else:
        lhs = np.repeat(np.arange(T), top)
        rhs = flat
        print(f"prefill T={T} P={P} shuffled {dtype}", flush=True)
        out = mq.gather_qmm(xd, *dev, rhs_indices=torch.from_numpy(idx).cuda(), bits=bits)
    out = out.reshape(P, N)
    assert bool(torch.isfinite(out).all())
    sel = np.sort(rng.choice(P, size=sample, replace=False))
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), *host, lhs[sel], rhs[sel], 64, bits, dtype)
    _check(out[torch.from_numpy(sel).cuda()].reshape(sample, 1, N), ref, dtype)


@pytest.mark.parametrize("T,sort", [(2048, True), (2048, False), (4096, True), (4096, False),
                                    (8192, True)])
def test_prefill_gate_up_at_scale(mlx_banks, T, sort):
    host, dev = mlx_banks["gate_up"]
    _prefill_case(dev, host, T, 8, 500 + T + sort, sort)


@pytest.mark.parametrize("T", [2048, 8192])
def test_prefill_down_at_scale(mlx_banks, T):
    host, dev = mlx_banks["down"]
    _prefill_case(dev, host, T, 8, 600 + T, False)


def test_prefill_fp16_8bit_at_scale():
    """fp16 activations over an 8-bit bank (prep LDS above 64 KiB at E=512)."""
    E, N, K = 512, 512, 1024
    g = torch.Generator(device="cuda").manual_seed(77)
    wf = (torch.randn((E, N, K), generator=g, device="cuda") * 0.02).to(torch.float16)
    dev = mq.quantize(wf, group_size=64, bits=8)
    del wf
    host = tuple(_host(t) for t in dev)
    _prefill_case(dev, host, 2048, 8, 700, False, "float16")


def test_prefill_many_experts():
    """1100 experts (the prep kernel's per-thread key chunks hold more than
    one key), 4096 pairs."""
    E, N, K = 1100, 128, 256
    dev = _mlx_quantized((E, N, K), 800, check_rows=16)
    host = tuple(_host(t) for t in dev)
    rng = np.random.default_rng(801)
    T, top = 512, 8
    idx = uniform_routing(rng, T, top, E)
    x = act(rng, (T, 1, 1, K))
    out = mq.gather_qmm(to_dev(x, "bfloat16"), *dev, rhs_indices=torch.from_numpy(idx).cuda())
    out = out.reshape(T * top, N)
    sel = np.sort(rng.choice(T * top, 96, replace=False))
    lhs = np.repeat(np.arange(T), top)
    ref = O.gather_qmm_ref(x.reshape(T, 1, K), *host, lhs[sel], idx.reshape(-1)[sel])
    _check(out[torch.from_numpy(sel).cuda()].reshape(96, 1, N), ref)


# ------------------------------------------------------------ config 5

def test_config5_lm_head_on_mlx_quantized_weights():
    """8-bit K=5120 N=248320 from N(0, 0.02): quantized on the GPU (1.27 G
    values), M = 1, 2, 4 against the oracle on 2000 sampled columns."""
    N, K, gs = 248320, 5120, 64
    dev = _mlx_quantized((N, K), 900, bits=8, check_rows=16)
    rng = np.random.default_rng(901)
    cols = np.sort(rng.choice(N, 2000, replace=False))
    ci = torch.from_numpy(cols).cuda()
    host = tuple(_host(_take(t, ci)) for t in dev)
    for M in (1, 2, 4):
        x = act(rng, (M, K))
        print(f"config5 M={M}", flush=True)
        out = mq.quantized_matmul(to_dev(x, "bfloat16"), *dev, group_size=gs, bits=8)
        _check(out[:, ci], O.quantized_matmul_ref(x, *host, gs, 8))


# --------------------------------------------------- route-table geometry

@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_geometry_21504_5376(M):
    """(K=21504, N=5376): the reference routes its E120 kernel here at M=4
    (dispatch.py:67); this build runs its skinny kernel."""
    K, N = 21504, 5376
    dev = _mlx_quantized((N, K), 1000, check_rows=8)
    rng = np.random.default_rng(1001 + M)
    cols = np.sort(rng.choice(N, 400, replace=False))
    ci = torch.from_numpy(cols).cuda()
    host = tuple(_host(_take(t, ci)) for t in dev)
    x = act(rng, (M, K))
    out = dispatch.quantized_matmul(to_dev(x, "bfloat16"), *dev, group_size=64, bits=4)
    assert dispatch.select_route(K, N, M) == dispatch.SKINNY
    _check(out[:, ci], O.quantized_matmul_ref(x, *host, 64, 4))


# ------------------------------------------------------ class-level patch

def test_enable_class_forward_matches_oracle():
    """fast_qmm.enable's class patch: every QuantizedLinear (existing and new)
    routes through the dispatch table; results match the oracle and the
    unpatched forward bit for bit; disable restores the class."""
    rng = np.random.default_rng(1100)
    N, K = 17408, 5120
    dev = _mlx_quantized((N, K), 1101, check_rows=8)
    bias = _gauss_bf16((N,), 1102)
    plain, biased = QuantizedLinear(*dev), QuantizedLinear(*dev, bias=bias)
    cols = np.sort(rng.choice(N, 300, replace=False))
    ci = torch.from_numpy(cols).cuda()
    host = tuple(_host(_take(t, ci)) for t in dev)
    x = act(rng, (2, 3, K))
    xd = to_dev(x, "bfloat16")
    base_plain, base_biased = bits16(plain(xd)), bits16(biased(xd))
    orig = QuantizedLinear.forward
    dispatch.enable_class()
    try:
        assert QuantizedLinear.forward is not orig
        p_plain, p_biased = plain(xd), biased(xd)
        fresh = QuantizedLinear(*dev)(xd[:, :1])                # an instance made after patching
    finally:
        dispatch.disable_class()
    assert QuantizedLinear.forward is orig
    np.testing.assert_array_equal(bits16(p_plain), base_plain)
    np.testing.assert_array_equal(bits16(p_biased), base_biased)
    # the bias is one bf16 add on the rounded product (mlx's x @ W.T + b)
    np.testing.assert_array_equal(bits16(p_biased), bits16(p_plain + bias))
    ref = O.quantized_matmul_ref(x.reshape(6, K), *host, 64, 4)
    _check(from_dev(p_plain).reshape(6, N)[:, cols], ref)
    _check(from_dev(fresh).reshape(2, N)[:, cols], O.quantized_matmul_ref(x[:, 0], *host, 64, 4))
