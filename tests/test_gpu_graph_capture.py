"""Graph capture of the operators: buffers a captured kernel uses stay alive.

The Python layer caches per-stream workspaces (gather segment tables) and
index tables.  A HIP graph captured on a stream keeps pointing at the
buffers its kernels used; if a later eager call on that stream outgrows the
workspace, the old buffer must not return to the allocator, or the graph's
replays write into memory that by then belongs to other tensors.  The usual
pattern is tested: warm-up on the capture stream (the capture then only
finds the buffer cached), capture, a larger eager call, allocations of the
old buffer's size, several replays with eager work and synchronizations in
between, each replay checked against the eager result.
"""

import numpy as np
import pytest
import torch

import mlxturbo_amd as mq
from mlxturbo_amd import ops
from qmm_helpers import act, bits16, random_packed, to_dev

pytestmark = pytest.mark.gpu


def _bank(rng, E, N, K):
    w, s, b = random_packed(rng, E * N, K)
    return (to_dev(w).view(E, N, K // 8), to_dev(s, "bfloat16").view(E, N, K // 64),
            to_dev(b, "bfloat16").view(E, N, K // 64))


def test_gather_replay_after_workspace_growth():
    rng = np.random.default_rng(3)
    E, N, K = 64, 256, 512
    w, s, b = _bank(rng, E, N, K)
    P1, P2 = 2048, 16384                 # both take the prefill path (workspace tables)
    x1 = to_dev(act(rng, (P1, 1, K)), "bfloat16")
    i1 = torch.from_numpy(rng.integers(0, E, P1).astype(np.int32)).cuda()
    x2 = to_dev(act(rng, (P2, 1, K)), "bfloat16")
    i2 = torch.from_numpy(rng.integers(0, E, P2).astype(np.int32)).cuda()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        want = mq.gather_qmm(x1, w, s, b, rhs_indices=i1)          # warm-up: workspace cached
        torch.cuda.synchronize()
        key = ("cuda", torch.cuda.current_device(), stream.cuda_stream)
        old = ops._WS_CACHE[key]
        old_ptr, old_n = old.data_ptr(), old.numel()
        del old
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            got = mq.gather_qmm(x1, w, s, b, rhs_indices=i1)        # cache hit under capture
        torch.cuda.synchronize()
        big = mq.gather_qmm(x2, w, s, b, rhs_indices=i2)            # outgrows the workspace
        torch.cuda.synchronize()
        assert ops._WS_CACHE[key].numel() > old_n
        # tensors of the old buffer's size: none may land on it, and the
        # replays must leave them alone
        junk = [torch.full((old_n,), 7, dtype=torch.uint8, device="cuda") for _ in range(16)]
        assert all(j.data_ptr() != old_ptr for j in junk)
        for rep in range(4):
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits16(got), bits16(want))
            for j in junk:
                assert bool((j == 7).all()), f"replay {rep} wrote into a reused buffer"
            # the program's own eager work between replays
            again = mq.gather_qmm(x1, w, s, b, rhs_indices=i1)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits16(again), bits16(want))
    del big


@pytest.mark.parametrize("M", [16, 40])
def test_split_skinny_replays(M):
    """The split skinny launch (K slices on separate workgroups writing float
    planes into the stream's workspace, then the ordered sum kernel) under
    capture: every replay, with eager calls of other widths on the same
    stream in between, gives the eager bits."""
    rng = np.random.default_rng(30 + M)
    N, K = 5120, 17408                   # the down-proj shape: 320 tiles, 8 K slices
    assert mq._lib.lib().mq_quantized_matmul_workspace_size(M, N, K, 64, 4) == M * N * 32
    w, s, b = random_packed(rng, N, K)
    args = (to_dev(w), to_dev(s, "bfloat16"), to_dev(b, "bfloat16"))
    x = to_dev(act(rng, (64, K), scale=0.1), "bfloat16")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        want = mq.quantized_matmul(x[:M], *args)                    # warm-up
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            got = mq.quantized_matmul(x[:M], *args)
        torch.cuda.synchronize()
        for rep in range(4):
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits16(got), bits16(want), f"replay {rep}")
            other = mq.quantized_matmul(x[:64 - M], *args)          # same workspace
            torch.cuda.synchronize()
            np.testing.assert_array_equal(
                bits16(other)[:8], bits16(mq.quantized_matmul(x[:8], *args)))
