"""Regenerate the golden fixtures in this directory (seeded, deterministic).

The reference ships no golden vectors (every one of its tests compares
against live ``mx.*`` ops, which cannot run here: mlx is absent and Metal-only),
so these fixtures are written by the project's own oracle after the oracle
has been pinned by the independent checks in ``tests/test_oracle.py``.  They
freeze the oracle's outputs so any later change to it is caught, and they
are the small known-answer inputs the GPU parity tests replay.

Run: ``python tests/golden/make_golden.py``
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def _x(rng, shape, dtype):
    return O.from_f32(rng.standard_normal(shape).astype(np.float32), dtype)


def _quantized(rng, N, K, gs, bits, dtype, sigma=0.02):
    w = (rng.standard_normal((N, K)) * sigma).astype(np.float32)
    return O.quantize(w, gs, bits, dtype)


def make_dequant():
    rng = np.random.default_rng(100)
    out = {}
    for bits in (4, 8):
        for gs in (32, 64, 128):
            for dtype in ("bfloat16", "float16"):
                N, K = 7, 256
                wq = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
                s = O.from_f32((rng.random((N, K // gs)) * 0.05).astype(np.float32), dtype)
                b = O.from_f32((rng.random((N, K // gs)) * 0.02 - 0.01).astype(np.float32), dtype)
                key = f"b{bits}_g{gs}_{dtype}"
                out[key + "_w"] = wq
                out[key + "_s"] = s
                out[key + "_b"] = b
                out[key + "_deq"] = O.dequantize(wq, s, b, gs, bits, dtype)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **out)


def make_qmm():
    rng = np.random.default_rng(101)
    out = {}
    cases = [("b4_g64_bf16", 3, 40, 320, 64, 4, "bfloat16"),
             ("b8_g64_bf16", 5, 24, 256, 64, 8, "bfloat16"),
             ("b4_g32_f16", 2, 33, 160, 32, 4, "float16"),
             ("b4_g128_bf16_m16", 16, 48, 512, 128, 4, "bfloat16")]
    for key, M, N, K, gs, bits, dtype in cases:
        wq, s, b = _quantized(rng, N, K, gs, bits, dtype)
        x = _x(rng, (M, K), dtype)
        out[key + "_x"] = x
        out[key + "_w"] = wq
        out[key + "_s"] = s
        out[key + "_b"] = b
        out[key + "_ref"] = O.quantized_matmul_ref(x, wq, s, b, gs, bits, dtype)
        out[key + "_meta"] = np.array([M, N, K, gs, bits, 0 if dtype == "bfloat16" else 1])
    np.savez_compressed(os.path.join(HERE, "qmm.npz"), **out)


def make_gather():
    rng = np.random.default_rng(102)
    E, N, K, gs, bits, dtype = 6, 32, 128, 64, 4, "bfloat16"
    ws, ss, bs = [], [], []
    for _ in range(E):
        wq, s, b = _quantized(rng, N, K, gs, bits, dtype)
        ws.append(wq), ss.append(s), bs.append(b)
    w, s, b = np.stack(ws), np.stack(ss), np.stack(bs)
    T, top = 3, 4
    x = _x(rng, (T, 1, K), dtype)
    rhs = np.array([[0, 3, 5, 1], [3, 0, 2, 4], [3, 5, 0, 0]], dtype=np.int32)  # duplicates
    lhs = np.repeat(np.arange(T, dtype=np.int32)[:, None], top, axis=1)
    ref = O.gather_qmm_ref(x, w, s, b, lhs, rhs, gs, bits, dtype)
    np.savez_compressed(os.path.join(HERE, "gather.npz"), x=x, w=w, s=s, b=b, lhs=lhs, rhs=rhs,
                        ref=ref, meta=np.array([E, N, K, gs, bits]))


if __name__ == "__main__":
    make_dequant()
    make_qmm()
    make_gather()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
