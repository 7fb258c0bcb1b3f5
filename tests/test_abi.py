"""CPU tests of the C ABI and the host logic (no GPU compute).

Mirrors the reference's Metal-free static tests (bench/test_dispatch_static.py:
fake backend through the module's own seams, kwarg contract, leading-dim
flatten/restore) for the HIP boundary: the library loads, exports every
declared symbol, validates arguments before touching the GPU, and the Python
host logic passes the right sizes and indices to the ABI.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import mlxturbo_amd
from mlxturbo_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mlxturbo_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from mlxturbo_amd import build
        build.build()
    return _lib.lib()


def test_library_exports_every_declared_symbol(lib):
    declared = _declared()
    assert declared, "no mq_ declarations parsed from the header"
    assert set(declared) == set(_lib.EXPORTED)
    for name in declared:
        assert hasattr(lib, name), name


def test_version(lib):
    assert lib.mq_version() == 8


FAKE = 256  # aligned, never dereferenced: validation fails before any HIP call


def _qmm(lib, **kw):
    args = dict(x=FAKE, w=FAKE, s=FAKE, b=FAKE, out=FAKE, M=1, N=16, K=256, gs=64, bits=4,
                dtype=0, transpose=1)
    args.update(kw)
    return lib.mq_quantized_matmul(args["x"], args["w"], args["s"], args["b"], args["out"],
                                   args["M"], args["N"], args["K"], args["gs"], args["bits"],
                                   args["dtype"], args["transpose"], None)


@pytest.mark.parametrize("kw,code,needle", [
    (dict(b=None), -1, "requires biases"),
    (dict(w=None), -1, "non-null"),
    (dict(gs=48), -1, "group_size"),
    (dict(K=200), -1, "multiple of group_size"),
    (dict(bits=7), -1, "bits"),
    (dict(bits=3), -2, "no matmul kernel"),
    (dict(transpose=0), -2, "transpose"),
    (dict(dtype=2), -2, "float32"),
    (dict(dtype=9), -1, "dtype"),
    (dict(w=FAKE + 8), -1, "aligned"),
    (dict(x=FAKE + 4), -1, "aligned"),
    (dict(M=-1), -1, "M"),
])
def test_qmm_argument_validation(lib, kw, code, needle):
    rc = _qmm(lib, **kw)
    assert rc == code
    assert needle in lib.mq_last_error().decode()


def test_qmm_workspace_sizing(lib):
    # narrow matrix at a prefill width: K split over workgroups, float partials
    need = lib.mq_quantized_matmul_workspace_size(512, 5120, 17408, 64, 4)
    assert need > 0 and need % (512 * 5120 * 4) == 0
    # decode widths and the wide matrix at large M need none
    assert lib.mq_quantized_matmul_workspace_size(1, 5120, 17408, 64, 4) == 0
    assert lib.mq_quantized_matmul_workspace_size(8192, 17408, 5120, 64, 4) == 0
    assert lib.mq_quantized_matmul_workspace_size(0, 5120, 17408, 64, 4) == 0
    rc = lib.mq_quantized_matmul_ws(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 16, 256, 64, 4, 0, 1,
                                    FAKE + 4, 1024, None)
    assert rc == -1 and b"workspace" in lib.mq_last_error()


def test_qmm_route_by_workspace(lib):
    """The wide/skinny route model as the workspace sizing sees it (wide
    tiles that split K ask for float partials; skinny launches need none,
    but those of 5-64 rows on matrices of few tiles split their 8 K slices
    over workgroups into float planes, up to 64 rows per launch): on
    K=17408 N=5120 at least 48 rows run as one split skinny launch; on K=5120
    N=17408 up to ~70 rows as 32-row shared-x launches."""
    narrow = lambda M: lib.mq_quantized_matmul_workspace_size(M, 5120, 17408, 64, 4)  # noqa: E731
    tall = lambda M: lib.mq_quantized_matmul_workspace_size(M, 17408, 5120, 64, 4)  # noqa: E731
    planes = lambda m: m * 5120 * 8 * 4  # noqa: E731
    assert narrow(4) == 0 and narrow(5) == planes(5) and narrow(16) == planes(16)
    assert narrow(17) == planes(17) and narrow(32) == planes(32) and narrow(48) == planes(48)
    assert narrow(1024) > 0 and narrow(1024) != planes(64)
    assert tall(32) == 0 and tall(64) == 0 and tall(96) > 0


def test_empty_problem_is_a_noop(lib):
    assert _qmm(lib, M=0) == 0
    assert _qmm(lib, N=0) == 0


def test_route_and_shared_combine_validation(lib):
    r = lib.mq_moe_route
    def route(rows=2, E=64, k=8, x=None, g=None, sg=None, H=0, dtype=0, lg=FAKE):
        return r(lg, FAKE, FAKE, rows, E, k, x, g, sg, H, dtype, None)
    assert route(lg=None) == -1 and "non-null" in lib.mq_last_error().decode()
    assert route(k=65, E=64) == -1 and "exceeds" in lib.mq_last_error().decode()
    assert route(k=0) == -1
    assert route(E=2048) == -2 and "E <= 1024" in lib.mq_last_error().decode()
    assert route(E=1024, k=65) == -2
    assert route(x=FAKE) == -1 and "together" in lib.mq_last_error().decode()
    assert route(x=FAKE, g=FAKE, sg=FAKE, H=0) == -1 and "hidden size" in lib.mq_last_error().decode()
    assert route(x=FAKE, g=FAKE, sg=FAKE, H=64, dtype=2) == -2
    assert route(rows=0) == 0
    c = lib.mq_moe_combine_shared
    assert c(FAKE, 8, None, FAKE, None, FAKE, FAKE, 4, 2, 64, 0, None) == -1
    assert "sgate and shared" in lib.mq_last_error().decode()
    assert c(FAKE, 8, None, FAKE, FAKE, FAKE + 2, FAKE, 4, 2, 64, 0, None) == -1
    assert "shared must be 16-byte aligned" in lib.mq_last_error().decode()
    assert c(FAKE, 8, None, FAKE, FAKE, FAKE, FAKE, 4, 2, 60, 0, None) == -2
    assert c(FAKE, 8, None, FAKE, FAKE, FAKE, FAKE, 0, 2, 64, 0, None) == 0


def test_gather_argument_validation(lib):
    f = lib.mq_gather_qmm
    # lhs NULL needs B to divide P (pair p reads x batch p / (P / B))
    for P, B in ((4, 3), (4, 0), (6, 4), (4, 8)):
        rc = f(FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, P, B, 1, 16, 256, 8, 64, 4, 0, 0, None,
               0, None)
        assert rc == -1 and "B to divide P" in lib.mq_last_error().decode(), (P, B)
    # more than 16 rows per pair
    rc = f(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 4, 17, 16, 256, 8, 64, 4, 0, 0, None, 0, None)
    assert rc == -2
    assert lib.mq_gather_qmm_workspace_size(64, 1) == 0          # fused segment discovery
    assert lib.mq_gather_qmm_workspace_size(4096, 1) >= 4 * (1 + 4 * 4096)


def test_gather_combine_argument_validation(lib):
    f = lib.mq_gather_qmm_combine
    def call(weights=FAKE, sgate=None, shared=None, T=1, top_k=8, dtype=0, x=FAKE):
        return f(x, FAKE, FAKE, FAKE, FAKE, weights, sgate, shared, FAKE, T, top_k, 2048, 512,
                 64, 64, 4, dtype, None)
    assert call(weights=None) == -1 and "non-null" in lib.mq_last_error().decode()
    assert call(sgate=FAKE) == -1 and "together" in lib.mq_last_error().decode()
    assert call(top_k=0) == -1
    assert call(T=3) == -2 and "up to 16 pairs" in lib.mq_last_error().decode()
    assert call(dtype=2) == -2
    assert call(x=FAKE + 2) == -1 and "aligned" in lib.mq_last_error().decode()
    assert call(T=0) == 0


def test_dequant_argument_validation(lib):
    rc = lib.mq_dequantize(FAKE, FAKE, None, FAKE, 4, 256, 64, 4, 0, None)
    assert rc == -1
    rc = lib.mq_dequantize(FAKE, FAKE, FAKE, FAKE + 2, 4, 256, 64, 4, 0, None)
    assert rc == -1 and "aligned" in lib.mq_last_error().decode()
    # every MLX width validates (no rows: nothing is launched)
    for bits in (2, 3, 4, 5, 6, 8):
        assert lib.mq_dequantize(FAKE, FAKE, FAKE, FAKE, 0, 256, 64, bits, 0, None) == 0
    assert lib.mq_dequantize(FAKE, FAKE, FAKE, FAKE, 4, 256, 64, 7, 0, None) == -1


def test_quantize_argument_validation(lib):
    q = lib.mq_quantize
    assert q(FAKE, FAKE, FAKE, FAKE, 0, 256, 64, 3, 0, None) == 0
    assert q(FAKE, FAKE, FAKE, FAKE, 0, 256, 64, 6, 2, None) == 0
    rc = q(FAKE, FAKE, FAKE, FAKE, 4, 256, 64, 7, 0, None)
    assert rc == -1 and "bits" in lib.mq_last_error().decode()
    rc = q(FAKE, FAKE, FAKE, FAKE, 4, 200, 64, 4, 0, None)
    assert rc == -1 and "multiple of group_size" in lib.mq_last_error().decode()
    rc = q(FAKE, FAKE + 4, FAKE, FAKE, 4, 256, 64, 4, 0, None)
    assert rc == -1 and "aligned" in lib.mq_last_error().decode()
    rc = q(FAKE, None, FAKE, FAKE, 4, 256, 64, 4, 0, None)
    assert rc == -1
    rc = q(FAKE, FAKE, FAKE, None, 4, 256, 64, 4, 0, None)
    assert rc == -1 and "biases" in lib.mq_last_error().decode()


def test_combine_argument_validation(lib):
    rc = lib.mq_moe_combine(FAKE, 8, None, FAKE, FAKE, 4, 0, 64, 0, None)
    assert rc == -1 and "top_k" in lib.mq_last_error().decode()
    rc = lib.mq_moe_combine(FAKE, 8, None, FAKE, FAKE, 4, 2, 60, 0, None)
    assert rc == -2 and "N % 8" in lib.mq_last_error().decode()
    rc = lib.mq_moe_combine(FAKE, 8, None, FAKE, FAKE, 4, 2, 64, 2, None)
    assert rc == -2
    rc = lib.mq_moe_combine(FAKE + 2, 8, None, FAKE, FAKE, 4, 2, 64, 0, None)
    assert rc == -1 and "aligned" in lib.mq_last_error().decode()
    rc = lib.mq_moe_combine(None, 8, None, FAKE, FAKE, 4, 2, 64, 0, None)
    assert rc == -1
    # without inv, y must hold every (token, k) row
    rc = lib.mq_moe_combine(FAKE, 7, None, FAKE, FAKE, 4, 2, 64, 0, None)
    assert rc == -1 and "y_rows" in lib.mq_last_error().decode()
    rc = lib.mq_moe_combine(FAKE, -1, FAKE, FAKE, FAKE, 4, 2, 64, 0, None)
    assert rc == -1
    assert lib.mq_moe_combine(FAKE, 8, None, FAKE, FAKE, 0, 2, 64, 0, None) == 0


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 256, dtype=torch.bfloat16)
    w = torch.zeros(16, 32, dtype=torch.int32)
    s = torch.zeros(16, 4, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU fallback"):
        mlxturbo_amd.quantized_matmul(x, w, s, s)


# ---------------------------------------------------------------- fake backend

class _FakeLib:
    """Records ABI calls; reads index arrays back from host pointers."""

    def __init__(self):
        self.calls = []

    def mq_quantized_matmul(self, x, w, s, b, out, M, N, K, gs, bits, dtype, transpose, stream):
        self.calls.append(("qmm", dict(M=M, N=N, K=K, gs=gs, bits=bits, dtype=dtype,
                                       transpose=transpose)))
        return 0

    def mq_quantized_matmul_workspace_size(self, M, N, K, gs, bits):
        return 0

    def mq_quantized_matmul_ws(self, x, w, s, b, out, M, N, K, gs, bits, dtype, transpose, ws,
                               wsb, stream):
        return self.mq_quantized_matmul(x, w, s, b, out, M, N, K, gs, bits, dtype, transpose,
                                        stream)

    def mq_gather_qmm_workspace_size(self, P, M):
        return 0

    def mq_gather_qmm(self, x, w, s, b, lhs, rhs, out, P, B, M, N, K, E, gs, bits, dtype,
                      sorted_, ws, wsb, stream):
        read = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int32)),
                                               shape=(P,)).copy()
        # a NULL lhs means pair p reads x batch p / (P / B) (B divides P)
        assert lhs or (B > 0 and P % B == 0)
        self.calls.append(("gather", dict(P=P, B=B, M=M, N=N, K=K, E=E,
                                          lhs=read(lhs) if lhs else np.arange(P) // (P // B),
                                          lhs_null=not lhs, rhs=read(rhs), sorted=sorted_)))
        return 0

    def mq_gather_glu(self, x, wg, sg, bg, wu, su, bu, lhs, rhs, out, P, B, M, N, K, E, gs,
                      bits, dtype, ws, wsb, stream):
        read = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int32)),
                                               shape=(P,)).copy()
        self.calls.append(("glu", dict(P=P, B=B, M=M, N=N, K=K, E=E, gate=(wg, sg, bg),
                                       up=(wu, su, bu), rhs=read(rhs),
                                       lhs=read(lhs) if lhs else np.arange(P) // (P // B))))
        return 0

    def mq_moe_route(self, lg, idx, wts, rows, E, k, x, g, sg, H, dtype, stream):
        self.calls.append(("route", dict(rows=rows, E=E, k=k, H=H, dtype=dtype, x=bool(x),
                                         g=bool(g), sg=bool(sg))))
        return 0

    def mq_moe_combine_shared(self, y, y_rows, inv, w, sg, sh, out, rows, top_k, N, dtype,
                              stream):
        self.calls.append(("combine_shared", dict(rows=rows, top_k=top_k, N=N, y_rows=y_rows,
                                                  sg=bool(sg), sh=bool(sh), inv=bool(inv))))
        return 0

    def mq_dequantize(self, w, s, b, out, N, K, gs, bits, dtype, stream):
        self.calls.append(("deq", dict(N=N, K=K, gs=gs, bits=bits, dtype=dtype)))
        return 0

    def mq_quantize(self, w, wq, s, b, N, K, gs, bits, dtype, stream):
        self.calls.append(("quant", dict(N=N, K=K, gs=gs, bits=bits, dtype=dtype)))
        return 0

    def mq_gather_qmm_combine(self, x, w, s, b, rhs, wts, sg, sh, out, T, top_k, N, K, E, gs,
                              bits, dtype, stream):
        n = T * top_k
        read_i = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int32)),
                                                 shape=(n,)).copy()
        read_f = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)),
                                                 shape=(n,)).copy()
        self.calls.append(("fold", dict(T=T, top_k=top_k, N=N, K=K, E=E, gs=gs, bits=bits,
                                        dtype=dtype, rhs=read_i(rhs), w=read_f(wts),
                                        sg=bool(sg), sh=bool(sh))))
        return 0

    def mq_moe_combine(self, y, y_rows, inv, w, out, rows, top_k, N, dtype, stream):
        n = rows * top_k
        read_i = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int32)),
                                                 shape=(n,)).copy()
        read_f = lambda p: np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)),
                                                 shape=(n,)).copy()
        self.calls.append(("combine", dict(rows=rows, top_k=top_k, N=N, dtype=dtype, y_rows=y_rows,
                                           inv=read_i(inv) if inv else None, w=read_f(w))))
        return 0


@pytest.fixture
def fake(monkeypatch):
    f = _FakeLib()
    monkeypatch.setattr(_lib, "lib", lambda: f)
    monkeypatch.setattr(ops, "_require_gpu", lambda *ts: torch.device("cpu"))
    monkeypatch.setattr(ops, "_stream_ptr", lambda t: 0)
    monkeypatch.setattr(ops, "_stream_of", lambda dev: 0)
    return f


def _qweights(N, K, gs=64, bits=4, E=None):
    lead = (E,) if E else ()
    w = torch.zeros(*lead, N, K * bits // 32, dtype=torch.int32)
    s = torch.zeros(*lead, N, K // gs, dtype=torch.bfloat16)
    return w, s, s.clone()


def test_leading_dims_flatten_and_restore(fake):
    w, s, b = _qweights(48, 512)
    x = torch.zeros(2, 3, 512, dtype=torch.bfloat16)
    out = mlxturbo_amd.quantized_matmul(x, w, s, b, group_size=64, bits=4)
    assert out.shape == (2, 3, 48)
    kind, c = fake.calls[-1]
    assert kind == "qmm" and c == dict(M=6, N=48, K=512, gs=64, bits=4, dtype=0, transpose=1)


def test_qmm_contract_errors(fake):
    w, s, b = _qweights(48, 512)
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="requires biases"):
        mlxturbo_amd.quantized_matmul(x, w, s, None)
    with pytest.raises(NotImplementedError):
        mlxturbo_amd.quantized_matmul(x, w, s, b, mode="mxfp4")
    with pytest.raises(ValueError, match="does not match"):
        mlxturbo_amd.quantized_matmul(x[:, :256], w, s, b)
    with pytest.raises(ValueError, match="scales shape"):
        mlxturbo_amd.quantized_matmul(x, w, s, b, group_size=32)
    with pytest.raises(ValueError, match="bits"):
        mlxturbo_amd.quantized_matmul(x, w, s, b, bits=7)
    assert fake.calls == []


def test_qmm_without_kernel_composes_dequantize_and_gemm(fake):
    """Configurations the matmul kernels do not take run as the library's
    dequantize (in MLX's promoted dtype) plus one GEMM, never raising."""
    w, s, b = _qweights(48, 512)
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    # fp16 activations over bf16 scales: promoted to float32
    out = mlxturbo_amd.quantized_matmul(x.half(), w, s, b)
    assert out.shape == (4, 48) and out.dtype == torch.float32
    assert fake.calls[-1] == ("deq", dict(N=48, K=512, gs=64, bits=4, dtype=2))
    # float32 activations
    out = mlxturbo_amd.quantized_matmul(x.float(), w, s, b)
    assert out.dtype == torch.float32
    # transpose=False: w [K, N*bits/32] quantized along N
    wt, st, bt = _qweights(512, 128)                      # K=512 rows, N=128
    out = mlxturbo_amd.quantized_matmul(x, wt, st, bt, transpose=False)
    assert out.shape == (4, 128) and out.dtype == torch.bfloat16
    assert fake.calls[-1] == ("deq", dict(N=512, K=128, gs=64, bits=4, dtype=0))
    # 3-bit codes
    w3, s3, b3 = _qweights(48, 512, bits=3)
    out = mlxturbo_amd.quantized_matmul(x, w3, s3, b3, bits=3)
    assert out.shape == (4, 48)
    assert fake.calls[-1] == ("deq", dict(N=48, K=512, gs=64, bits=3, dtype=0))
    assert all(k == "deq" for k, _ in fake.calls)


def test_quantize_shapes(fake):
    w = torch.zeros(3, 48, 512, dtype=torch.bfloat16)
    wq, s, b = mlxturbo_amd.quantize(w, group_size=64, bits=6)
    assert wq.shape == (3, 48, 512 * 6 // 32) and wq.dtype == torch.uint32
    assert s.shape == b.shape == (3, 48, 8) and s.dtype == torch.bfloat16
    assert fake.calls[-1] == ("quant", dict(N=144, K=512, gs=64, bits=6, dtype=0))
    with pytest.raises(ValueError, match="multiple of group_size"):
        mlxturbo_amd.quantize(w[..., :100])
    with pytest.raises(ValueError, match="bfloat16, float16 or float32"):
        mlxturbo_amd.quantize(w.to(torch.int32))


def test_gather_more_than_16_rows_per_pair_is_one_row_pairs(fake):
    T, top, E, N, K, M = 3, 2, 8, 32, 256, 20
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(T, M, K, dtype=torch.bfloat16)
    idx = torch.tensor([[1, 4], [0, 4], [7, 2]], dtype=torch.int32)
    out = mlxturbo_amd.gather_qmm(x[:, None], w, s, b, rhs_indices=idx)
    assert out.shape == (T, top, M, N)
    kind, c = fake.calls[-1]
    assert kind == "gather" and len(fake.calls) == 1
    assert (c["P"], c["B"], c["M"]) == (T * top * M, T * M, 1)
    pair_lhs = np.repeat(np.arange(T), top)
    np.testing.assert_array_equal(c["lhs"], (pair_lhs[:, None] * M + np.arange(M)).reshape(-1))
    np.testing.assert_array_equal(c["rhs"], np.repeat(idx.reshape(-1).numpy(), M))


def test_gather_many_experts_runs_in_slices(fake):
    P, E, N, K = 300, 4096 + 5, 32, 256
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(P, 1, K, dtype=torch.bfloat16)
    idx = torch.tensor(np.random.default_rng(0).integers(0, E, P), dtype=torch.int32)
    mlxturbo_amd.gather_qmm(x, w, s, b, rhs_indices=idx)
    assert [k for k, _ in fake.calls] == ["gather"] * 3
    want = idx.numpy()
    for (_, c), e0 in zip(fake.calls, (0, 2048, 4096)):
        e1 = min(E, e0 + 2048)
        assert c["E"] == e1 - e0
        inside = (want >= e0) & (want < e1)
        np.testing.assert_array_equal(c["rhs"], np.where(inside, want - e0, -1))


def test_gather_without_kernel_composes_per_expert(fake):
    E, N, K = 4, 32, 256
    w, s, b = _qweights(N, K, E=E, bits=5)
    x = torch.zeros(6, 1, K, dtype=torch.bfloat16)
    idx = torch.tensor([2, 0, 2, 9, 3, -1], dtype=torch.int32)   # 9 and -1: zero rows
    out = mlxturbo_amd.gather_qmm(x, w, s, b, rhs_indices=idx, bits=5)
    assert out.shape == (6, 1, N)
    kinds = [k for k, _ in fake.calls]
    assert kinds == ["deq"] * 3                           # experts 0, 2, 3 once each
    assert all(c["bits"] == 5 and (c["N"], c["K"]) == (N, K) for _, c in fake.calls)
    assert torch.all(out[3] == 0) and torch.all(out[5] == 0)


def test_gather_broadcasts_like_switchglu(fake):
    # mlx-lm SwitchGLU: x (T,1,1,K) with indices (T,top_k) -> out (T,top_k,1,N)
    T, top, E, N, K = 3, 4, 8, 32, 256
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(T, 1, 1, K, dtype=torch.bfloat16)
    idx = torch.tensor([[0, 3, 5, 1], [3, 0, 2, 4], [3, 5, 0, 7]], dtype=torch.int32)
    out = mlxturbo_amd.gather_qmm(x, w, s, b, rhs_indices=idx)
    assert out.shape == (T, top, 1, N)
    kind, c = fake.calls[-1]
    assert kind == "gather" and c["P"] == T * top and c["B"] == T and c["M"] == 1 and c["E"] == E
    np.testing.assert_array_equal(c["rhs"], idx.reshape(-1).numpy())
    np.testing.assert_array_equal(c["lhs"], np.repeat(np.arange(T), top))
    assert c["lhs_null"]                  # repeated batches need no index table


@pytest.mark.parametrize("bx,ishape,null", [((3, 1), (3, 4), True), ((1, 1), (3, 4), True),
                                            ((), (5,), True), ((2, 3, 1), (2, 3, 4), True),
                                            ((1, 4), (3, 4), False), ((2, 1, 3), (2, 4, 3), False)])
def test_gather_default_lhs_broadcasts(fake, bx, ishape, null):
    # x's batch dims broadcast against the indices: NULL lhs exactly when
    # each x batch covers consecutive pairs, else an explicit table; either
    # way the pair -> batch map is numpy's broadcast of x's batch index
    E, N, K = 8, 32, 256
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(*bx, 1, K, dtype=torch.bfloat16)
    idx = torch.arange(int(np.prod(ishape)), dtype=torch.int32).reshape(ishape) % E
    mlxturbo_amd.gather_qmm(x, w, s, b, rhs_indices=idx)
    _, c = fake.calls[-1]
    want = np.broadcast_to(np.arange(int(np.prod(bx))).reshape(bx), ishape).reshape(-1)
    np.testing.assert_array_equal(c["lhs"], want)
    assert c["lhs_null"] == null and c["B"] == int(np.prod(bx))


def test_route_shapes_and_arguments(fake):
    logits = torch.zeros(2, 3, 64, dtype=torch.float32)
    idx, w, sg = mlxturbo_amd.moe_route(logits, 8)
    assert idx.shape == (2, 3, 8) and idx.dtype == torch.int32 and w.dtype == torch.float32
    assert sg is None
    assert fake.calls[-1] == ("route", dict(rows=6, E=64, k=8, H=0, dtype=0, x=False, g=False,
                                            sg=False))
    x = torch.zeros(2, 3, 128, dtype=torch.bfloat16)
    idx, w, sg = mlxturbo_amd.moe_route(logits, 4, x, torch.zeros(128, dtype=torch.bfloat16))
    assert sg.shape == (2, 3, 1) and sg.dtype == torch.bfloat16
    assert fake.calls[-1][1]["H"] == 128 and fake.calls[-1][1]["sg"]
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_route(logits.double(), 4)
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_route(logits, 65)
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_route(logits, 4, x)


def test_combine_shared_arguments(fake):
    rows, top_k, N = 3, 2, 64
    y = torch.zeros(rows * top_k, N, dtype=torch.bfloat16)
    w = torch.ones(rows * top_k)
    sg = torch.zeros(rows, 1, dtype=torch.bfloat16)
    sh = torch.zeros(rows, N, dtype=torch.bfloat16)
    out = mlxturbo_amd.moe_combine(y, None, w, rows, top_k, sgate=sg, shared=sh)
    assert out.shape == (rows, N)
    assert fake.calls[-1] == ("combine_shared", dict(rows=rows, top_k=top_k, N=N, y_rows=6,
                                                     sg=True, sh=True, inv=False))
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_combine(y, None, w, rows, top_k, sgate=sg)
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_combine(y, None, w, rows, top_k, sgate=sg, shared=sh[:2])


def test_gather_sorted_layout(fake):
    # mlx-lm _gather_sort: x (P,1,K) sorted rows, idx (P,) -> out (P,1,N)
    P, E, N, K = 6, 8, 32, 256
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(P, 1, K, dtype=torch.bfloat16)
    idx = torch.tensor([0, 0, 2, 5, 5, 7], dtype=torch.int64)
    out = mlxturbo_amd.gather_qmm(x, w, s, b, rhs_indices=idx, sorted_indices=True)
    assert out.shape == (P, 1, N)
    _, c = fake.calls[-1]
    np.testing.assert_array_equal(c["lhs"], np.arange(P))
    assert c["lhs_null"]                  # identity lhs travels as NULL
    assert c["sorted"] == 1


def test_gather_default_indices(fake):
    # no indices: lhs over x's batch, rhs over w's batch, broadcast together
    E, N, K = 4, 32, 256
    w, s, b = _qweights(N, K, E=E)
    x = torch.zeros(E, 2, K, dtype=torch.bfloat16)
    out = mlxturbo_amd.gather_qmm(x, w, s, b)
    assert out.shape == (E, 2, N)
    _, c = fake.calls[-1]
    np.testing.assert_array_equal(c["lhs"], np.arange(E))
    np.testing.assert_array_equal(c["rhs"], np.arange(E))


def test_dequantize_shapes(fake):
    w, s, b = _qweights(48, 512, bits=8)
    out = mlxturbo_amd.dequantize(w, s, b, group_size=64, bits=8)
    assert out.shape == (48, 512) and out.dtype == torch.bfloat16
    assert fake.calls[-1] == ("deq", dict(N=48, K=512, gs=64, bits=8, dtype=0))


def test_combine_passes_indices_and_weights(fake):
    rows, top_k, N = 3, 2, 64
    y = torch.zeros(rows * top_k, N, dtype=torch.bfloat16)
    inv = torch.tensor([5, 0, 3, 1, 4, 2], dtype=torch.int64)
    w = torch.tensor([0.5, 0.25, 1.0, 2.0, 0.125, 4.0], dtype=torch.float64)
    out = mlxturbo_amd.moe_combine(y, inv, w, rows, top_k)
    assert out.shape == (rows, N)
    _, c = fake.calls[-1]
    np.testing.assert_array_equal(c["inv"], inv.numpy())
    np.testing.assert_array_equal(c["w"], w.numpy().astype(np.float32))
    assert c["y_rows"] == rows * top_k
    mlxturbo_amd.moe_combine(y, None, w, rows, top_k)
    assert fake.calls[-1][1]["inv"] is None
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_combine(y[:5], None, w, rows, top_k)
    with pytest.raises(ValueError):
        mlxturbo_amd.moe_combine(y, inv[:4], w, rows, top_k)


def test_gather_combine_folds_or_composes(fake):
    E, N, K, top = 8, 64, 256, 4
    bank = _qweights(N, K, E=E)
    for T in (3, 16):
        x = torch.zeros(T, top, 1, K, dtype=torch.bfloat16)
        idx = torch.randint(0, E, (T, top), dtype=torch.int32)
        w = torch.rand(T, top, dtype=torch.float64)
        fake.calls.clear()
        out = mlxturbo_amd.gather_qmm_combine(x, *bank, idx, w)
        assert out.shape == (T, N) and out.dtype == torch.bfloat16
        if T * top <= 16:                   # one folded kernel
            [(kind, c)] = fake.calls
            assert kind == "fold" and (c["T"], c["top_k"], c["N"], c["K"], c["E"]) == (T, top, N, K, E)
            np.testing.assert_array_equal(c["rhs"], idx.reshape(-1).numpy())
            np.testing.assert_array_equal(c["w"], w.reshape(-1).numpy().astype(np.float32))
            assert not c["sh"]
        else:                               # beyond 64 pairs: the two passes
            assert [k for k, _ in fake.calls] == ["gather", "combine"]
            assert fake.calls[1][1]["inv"] is None
    with pytest.raises(ValueError, match="one row per"):
        mlxturbo_amd.gather_qmm_combine(torch.zeros(3, top, 2, K, dtype=torch.bfloat16), *bank,
                                        torch.zeros(3, top, dtype=torch.int32), torch.rand(3, top))
    with pytest.raises(ValueError, match="together"):
        mlxturbo_amd.gather_qmm_combine(torch.zeros(3, top, 1, K, dtype=torch.bfloat16), *bank,
                                        torch.zeros(3, top, dtype=torch.int32), torch.rand(3, top),
                                        sgate=torch.zeros(3, dtype=torch.bfloat16))


def test_glu_passes_both_banks(fake):
    T, top, E, N, K = 3, 4, 8, 32, 256
    gate, up = _qweights(N, K, E=E), _qweights(N, K, E=E)
    x = torch.zeros(T, 1, 1, K, dtype=torch.bfloat16)
    idx = torch.tensor([[0, 3, 5, 1], [3, 0, 2, 4], [3, 5, 0, 7]], dtype=torch.int32)
    out = mlxturbo_amd.gather_glu(x, *gate, *up, rhs_indices=idx)
    assert out.shape == (T, top, 1, N)
    kind, c = fake.calls[-1]
    assert kind == "glu" and (c["P"], c["B"], c["M"], c["E"]) == (T * top, T, 1, E)
    assert c["gate"] == tuple(t.data_ptr() for t in gate)
    assert c["up"] == tuple(t.data_ptr() for t in up)
    np.testing.assert_array_equal(c["rhs"], idx.reshape(-1).numpy())
    np.testing.assert_array_equal(c["lhs"], np.repeat(np.arange(T), top))
    with pytest.raises(ValueError, match="differ in shape"):
        mlxturbo_amd.gather_glu(x, *gate, *_qweights(N + 16, K, E=E), rhs_indices=idx)


def test_glu_prefill_composes_two_gathers(fake):
    # 1024+ output rows: two gather_qmm calls (the fused kernel is decode-only)
    T, top, E, N, K = 128, 8, 8, 32, 256
    gate, up = _qweights(N, K, E=E), _qweights(N, K, E=E)
    x = torch.zeros(T, 1, 1, K, dtype=torch.bfloat16)
    idx = torch.randint(0, E, (T, top), dtype=torch.int32)
    out = mlxturbo_amd.gather_glu(x, *gate, *up, rhs_indices=idx)
    assert out.shape == (T, top, 1, N) and out.dtype == torch.bfloat16
    assert [k for k, _ in fake.calls] == ["gather", "gather"]
