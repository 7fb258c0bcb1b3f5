"""Shared helpers for the GPU parity tests (numpy oracle data <-> torch tensors)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

TORCH_DTYPE = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def to_dev(a: np.ndarray, dtype: str | None = None, device="cuda") -> torch.Tensor:
    """uint16 storage -> bf16/f16 tensor; uint32 codes -> uint32 tensor; int32 as is."""
    a = np.ascontiguousarray(a)
    if dtype in ("bfloat16", "float16"):
        t = torch.from_numpy(a.view(np.int16)).view(TORCH_DTYPE[dtype])
    elif a.dtype == np.uint32:
        t = torch.from_numpy(a.view(np.int32)).view(torch.uint32)
    else:
        t = torch.from_numpy(a)
    return t.to(device)


def from_dev(t: torch.Tensor) -> np.ndarray:
    """bf16/f16 tensor -> float32 numpy; other dtypes as numpy."""
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.float().numpy()
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def bits16(t: torch.Tensor) -> np.ndarray:
    """Raw uint16 bit patterns of a bf16/f16 tensor."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def quantized(rng, N, K, gs=64, bits=4, dtype="bfloat16", sigma=0.02):
    w = (rng.standard_normal((N, K)) * sigma).astype(np.float32)
    return O.quantize(w, gs, bits, dtype)


def random_packed(rng, N, K, gs=64, bits=4, dtype="bfloat16"):
    """Random codes with random scales/biases (the reference's synthetic data,
    bench/test_qmm_smallm.py:42-50)."""
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = O.from_f32((rng.random((N, K // gs)) * 0.02).astype(np.float32), dtype)
    b = O.from_f32((rng.random((N, K // gs)) * 0.01 - 0.005).astype(np.float32), dtype)
    return w, s, b


def act(rng, shape, dtype="bfloat16", scale=1.0):
    return O.from_f32((rng.standard_normal(shape) * scale).astype(np.float32), dtype)


def zipf_routing(rng, T, top_k, E, s=1.1):
    """top_k distinct experts per token from Zipf(s) over E (rank -> id through
    a fixed seeded permutation)."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = np.random.default_rng(12345).permutation(E)
    out = np.empty((T, top_k), np.int32)
    for t in range(T):
        out[t] = perm[rng.choice(E, size=top_k, replace=False, p=p)]
    return out


def uniform_routing(rng, T, top_k, E):
    return np.stack([rng.choice(E, size=top_k, replace=False) for _ in range(T)]).astype(np.int32)
