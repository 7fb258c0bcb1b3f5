"""mq_gather_qmm_noalloc (static device scratch, no allocation) against
mq_gather_qmm with a caller workspace, through the C ABI, bit for bit: a
prefill-sized call (prep + grouped kernels), then a smaller one on the same
scratch (prep path), then a decode-sized one (no scratch), and a call too
large for the scratch is refused before anything is launched."""

import ctypes

import numpy as np
import pytest
import torch

from mlxturbo_amd import _lib
from qmm_helpers import bits16

pytestmark = pytest.mark.gpu

SCRATCH = 4 << 20          # MQ_GATHER_NOALLOC_SCRATCH_BYTES


def _bank(E, N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randint(0, 2**31 - 1, (E, N, K // 8), generator=g, device="cuda",
                      dtype=torch.int32).view(torch.uint32)
    s = (torch.rand((E, N, K // 64), generator=g, device="cuda") * 0.01).to(torch.bfloat16)
    b = (torch.rand((E, N, K // 64), generator=g, device="cuda") * 0.02 - 0.03).to(torch.bfloat16)
    return w, s, b


def _call_both(lib, x, bank, lhs, rhs, P, B, M, N, K, E):
    w, s, b = bank
    stream = torch.cuda.current_stream().cuda_stream
    out_ws = torch.empty((P, M, N), dtype=torch.bfloat16, device="cuda")
    out_na = torch.full((P, M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    need = int(lib.mq_gather_qmm_workspace_size(P, M))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
    lp = lhs.data_ptr() if lhs is not None else None
    rc = lib.mq_gather_qmm(x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), lp,
                           rhs.data_ptr(), out_ws.data_ptr(), P, B, M, N, K, E, 64, 4, 0, 0,
                           ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, lib.mq_last_error()
    rc = lib.mq_gather_qmm_noalloc(x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), lp,
                                   rhs.data_ptr(), out_na.data_ptr(), P, B, M, N, K, E, 64, 4, 0,
                                   0, stream)
    assert rc == 0, lib.mq_last_error()
    torch.cuda.synchronize()
    return need, out_ws, out_na


def test_noalloc_gather_matches_workspace_entry():
    lib = _lib.lib()
    E, N, K = 64, 256, 512
    bank = _bank(E, N, K, 1)
    g = torch.Generator(device="cuda").manual_seed(2)
    cases = [(2048, 8, 1), (300, 4, 1), (8, 8, 1)]       # prefill, smaller prep, decode
    for T, top, M in cases:
        P = T * top
        print(f"noalloc case T={T} top={top} P={P}", flush=True)
        x = (torch.randn((T, M, K), generator=g, device="cuda")).to(torch.bfloat16)
        rhs = torch.randint(0, E, (P,), generator=g, device="cuda", dtype=torch.int32)
        lhs = torch.arange(T, device="cuda", dtype=torch.int32).repeat_interleave(top)
        need, out_ws, out_na = _call_both(lib, x, bank, lhs, rhs, P, T, M, N, K, E)
        assert need <= SCRATCH
        assert (need > 0) == (P > 256)
        np.testing.assert_array_equal(bits16(out_na), bits16(out_ws))


def test_noalloc_gather_refuses_oversize_calls():
    lib = _lib.lib()
    lo, hi = 1024, 1 << 22                       # the first P whose tables pass 4 MiB
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if lib.mq_gather_qmm_workspace_size(mid, 1) <= SCRATCH else (lo, mid)
    P = hi
    assert 200000 < P < 262144                   # ~16 bytes of tables per pair
    assert lib.mq_gather_qmm_workspace_size(P, 1) > SCRATCH
    assert lib.mq_gather_qmm_workspace_size(P - 1, 1) <= SCRATCH
    fake = 256
    rc = lib.mq_gather_qmm_noalloc(fake, fake, fake, fake, fake, fake, fake, P, P, 1, 256, 512,
                                   64, 64, 4, 0, 0, None)
    assert rc == -1 and b"static scratch" in lib.mq_last_error()
