"""MLX-signature operators on PyTorch-ROCm tensors, backed by the HIP library.

Host side of the drop-in boundary.  Signatures and argument meaning follow
MLX 0.32's operators as the reference calls them:

* ``quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode)``
  - mx.quantized_matmul, called at mlxturbo/kernels/dispatch.py:317-327
* ``gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, transpose,
  group_size, bits, mode, sorted_indices)`` - mx.gather_qmm, called by mlx-lm's
  QuantizedSwitchLinear (mlxturbo/fused.py:2389-2394, 3105-3116)
* ``dequantize(w, scales, biases, group_size, bits, mode)`` - mx.dequantize
  (bench/test_qmm_wide_shapes.py:35-42)
* ``quantize(w, group_size, bits, mode)`` - mx.quantize (rebit.py:119,
  kernels/moe_verify_gather.py:887)
* ``gather_glu`` - fused MoE gate+up+SiLU (kernels/moe_glu.py:145-168)
* ``moe_combine`` - MoE unsort + router weight + top-k sum
  (kernels/moe_combine.py:160-195)

Errors and coverage: genuinely invalid arguments raise ``ValueError`` as MLX
does; non-affine modes raise ``NotImplementedError``.  Every affine
configuration returns a result, as the reference's wrappers do by falling
back to ``mx.quantized_matmul`` (fast_qmm.py:356-362): the kernels take 4/8
bits with bf16/fp16 activations in the scales' dtype, and the rest (other
widths, ``transpose=False``, float32 or mixed dtypes) runs as this library's
bit-exact dequantize plus one GPU GEMM.  Nothing runs on the CPU.
"""

from __future__ import annotations

import contextlib
import math
from typing import Optional, Sequence

import torch

from . import _lib

_DTYPE_CODE = {
    torch.bfloat16: _lib.MQ_BFLOAT16,
    torch.float16: _lib.MQ_FLOAT16,
    torch.float32: _lib.MQ_FLOAT32,
}

_GROUP_SIZES = (32, 64, 128)
_BITS = (2, 3, 4, 5, 6, 8)


def _stream_ptr(t: torch.Tensor) -> int:
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def _require_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(
                "mlxturbo_amd operators run on a ROCm GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Row-contiguous with a 16-byte aligned base (copies only when needed)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _check_mode(mode: str, biases) -> None:
    if mode != "affine":
        raise NotImplementedError(
            f"mode={mode!r}: only affine quantization is on this path")
    if biases is None:
        raise ValueError("affine quantization requires biases")


def _check_format(group_size: int, bits: int) -> None:
    if group_size not in _GROUP_SIZES:
        raise ValueError(f"group_size must be one of {_GROUP_SIZES}, got {group_size}")
    if bits not in _BITS:
        raise ValueError(f"bits must be one of {_BITS}, got {bits}")


def _check_quant(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int, bits: int) -> int:
    if w.dtype not in (torch.uint32, torch.int32):
        raise ValueError(f"w must be uint32 packed codes, got {w.dtype}")
    _check_format(group_size, bits)
    if (w.shape[-1] * 32) % bits:
        raise ValueError(f"w last dimension {w.shape[-1]} is not whole {bits}-bit codes")
    K = w.shape[-1] * 32 // bits
    if scales.shape != biases.shape:
        raise ValueError(f"scales {tuple(scales.shape)} and biases {tuple(biases.shape)} differ")
    if scales.dtype != biases.dtype:
        raise ValueError("scales and biases must have the same dtype")
    want = (*w.shape[:-1], K // group_size)
    if K % group_size or tuple(scales.shape) != want:
        raise ValueError(
            f"scales shape {tuple(scales.shape)} does not match w {tuple(w.shape)} "
            f"with group_size={group_size}, bits={bits} (expected {want})")
    return K


def _dtype_code(x_dtype: torch.dtype, s_dtype: torch.dtype) -> int:
    if x_dtype != s_dtype:
        raise NotImplementedError(
            f"x dtype {x_dtype} differs from scales dtype {s_dtype}; MLX would promote "
            "both, this path computes in the shared 16-bit dtype only")
    if x_dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"activation dtype {x_dtype}: bfloat16 and float16 only")
    return _DTYPE_CODE[x_dtype]


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4, mode: str = "affine"):
    """``mx.quantize(w, group_size, bits, mode="affine")``: returns
    ``(w_q, scales, biases)`` with ``w_q`` uint32 ``[..., K*bits/32]`` and
    scales/biases ``[..., K/group_size]`` in ``w``'s dtype, as the reference
    calls it when it requantizes a layer (mlxturbo/rebit.py:119) or builds
    test weights (kernels/moe_verify_gather.py:887).  One HIP kernel; the
    per-group arithmetic is the C ABI's ``mq_quantize``."""
    if mode != "affine":
        raise NotImplementedError(f"mode={mode!r}: only affine quantization is on this path")
    dev = _require_gpu(w)
    _check_format(group_size, bits)
    if w.dtype not in _DTYPE_CODE:
        raise ValueError(f"w must be bfloat16, float16 or float32, got {w.dtype}")
    if w.ndim < 1:
        raise ValueError("w must have at least one dimension")
    K = w.shape[-1]
    if K == 0 or K % group_size:
        raise ValueError(f"the last dimension {K} must be a positive multiple of "
                         f"group_size={group_size}")
    lead = tuple(w.shape[:-1])
    N = math.prod(lead)
    wq = torch.empty((*lead, K * bits // 32), dtype=torch.uint32, device=dev)
    scales = torch.empty((*lead, K // group_size), dtype=w.dtype, device=dev)
    biases = torch.empty_like(scales)
    if N == 0:
        return wq, scales, biases
    w_ = _aligned(w.reshape(N, K))
    rc = _lib.lib().mq_quantize(w_.data_ptr(), wq.data_ptr(), scales.data_ptr(),
                                biases.data_ptr(), N, K, group_size, bits,
                                _DTYPE_CODE[w.dtype], _stream_ptr(wq))
    _lib.check(rc, "quantize")
    return wq, scales, biases


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: Optional[torch.Tensor] = None,
               group_size: int = 64, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """``mx.dequantize``: ``T(float(s)*q + float(b))`` bit-exact, dtype of
    ``scales``, for every MLX width (2, 3, 4, 5, 6, 8 bits)."""
    _check_mode(mode, biases)
    dev = _require_gpu(w, scales, biases)
    K = _check_quant(w, scales, biases, group_size, bits)
    if scales.dtype not in _DTYPE_CODE:
        raise ValueError(f"scales dtype {scales.dtype} is not a float type")
    N = w.numel() // max(1, w.shape[-1]) if w.ndim else 0
    out = torch.empty((*w.shape[:-1], K), dtype=scales.dtype, device=dev)
    if out.numel() == 0:
        return out
    w_, s_, b_ = _aligned(w), _aligned(scales), _aligned(biases)
    rc = _lib.lib().mq_dequantize(w_.data_ptr(), s_.data_ptr(), b_.data_ptr(), out.data_ptr(),
                                  N, K, group_size, bits, _DTYPE_CODE[scales.dtype],
                                  _stream_ptr(out))
    _lib.check(rc, "dequantize")
    return out


def _kernel_dtype(x_dtype: torch.dtype, s_dtype: torch.dtype) -> bool:
    """Whether the matmul kernels compute in this (activation, scale) dtype pair."""
    return x_dtype == s_dtype and x_dtype in (torch.bfloat16, torch.float16)


def _result_dtype(x_dtype: torch.dtype, s_dtype: torch.dtype) -> torch.dtype:
    """MLX's promotion of (x, scales, biases) for the quantized operators."""
    dt = torch.promote_types(x_dtype, s_dtype)
    if not dt.is_floating_point:
        raise ValueError(f"quantized operators need floating activations, got {x_dtype}")
    return dt


def _composed_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                  transpose: bool, group_size: int, bits: int) -> torch.Tensor:
    """Configurations the matmul kernels do not take (2/3/5/6-bit codes,
    ``transpose=False``, float32 or mixed-dtype activations): this library's
    bit-exact :func:`dequantize` in the promoted dtype, then one GPU GEMM.
    It stands where the reference falls back to ``mx.quantized_matmul``
    (fast_qmm.py:356-362; qmv_small_m.py:309-323; dispatch.py:317-327)."""
    dt = _result_dtype(x.dtype, scales.dtype)
    deq = dequantize(w, scales.to(dt), biases.to(dt), group_size, bits)
    xx = x.to(dt)
    if transpose:
        return torch.nn.functional.linear(xx, deq)           # x @ deq^T, deq [N, K]
    return torch.matmul(xx, deq)                              # deq [K, N]


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor] = None, transpose: bool = True,
                     group_size: int = 64, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """``mx.quantized_matmul``: ``x @ dequantize(w).T`` for ``x[..., K]``
    (``transpose=False``: ``x @ dequantize(w)`` with ``w`` quantized along N).

    Leading dimensions of ``x`` are flattened to M and restored on the output
    (as mlxturbo/kernels/dispatch.py:332-382 does around its kernels).
    4- and 8-bit codes with bf16/fp16 activations in the scales' dtype run on
    the matmul kernels; every other MLX configuration runs as the library's
    dequantize plus one GPU GEMM (:func:`_composed_qmm`).
    """
    _check_mode(mode, biases)
    dev = _require_gpu(x, w, scales, biases)
    if w.ndim != 2:
        raise NotImplementedError("batched w: only 2-D weights are on this path")
    Kq = _check_quant(w, scales, biases, group_size, bits)
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")
    K, N = (Kq, w.shape[0]) if transpose else (w.shape[0], Kq)
    if x.shape[-1] != K:
        raise ValueError(
            f"x last dimension {x.shape[-1]} does not match the quantized weight K={K}")
    if not (transpose and bits in (4, 8) and _kernel_dtype(x.dtype, scales.dtype)):
        return _composed_qmm(x, w, scales, biases, transpose, group_size, bits)
    code = _DTYPE_CODE[x.dtype]
    lead = tuple(x.shape[:-1])
    M = math.prod(lead)
    out = torch.empty((*lead, N), dtype=x.dtype, device=dev)
    if M == 0 or N == 0:
        return out
    x_ = _aligned(x.reshape(M, K))
    w_, s_, b_ = _aligned(w), _aligned(scales), _aligned(biases)
    lib = _lib.lib()
    # wide problems on narrow matrices split K over workgroups into this
    # stream's workspace
    nbytes = int(lib.mq_quantized_matmul_workspace_size(M, N, K, group_size, bits))
    ws = _workspace(dev, nbytes) if nbytes else None
    rc = lib.mq_quantized_matmul_ws(x_.data_ptr(), w_.data_ptr(), s_.data_ptr(), b_.data_ptr(),
                                    out.data_ptr(), M, N, K, group_size, bits, code, 1,
                                    ws.data_ptr() if ws is not None else None,
                                    ws.numel() if ws is not None else 0, _stream_ptr(out))
    _lib.check(rc, "quantized_matmul")
    return out


class PreparedWeights:
    """Weight-side arguments of :func:`quantized_matmul`, validated once
    (the per-call cost of a layer that reuses its weights is then the x
    checks and the launch).  ``matches`` tells whether the tensors are still
    the ones validated: the same storage and no in-place write since (the
    key holds each tensor's version counter, so a ``copy_`` into the layer's
    weights, e.g. ``load_state_dict``, invalidates a cached aligned copy)."""

    __slots__ = ("w", "s", "b", "N", "K", "group_size", "bits", "dtype", "dev", "key")

    def __init__(self, w, scales, biases, group_size: int = 64, bits: int = 4,
                 mode: str = "affine"):
        _check_mode(mode, biases)
        self.dev = _require_gpu(w, scales, biases)
        if w.ndim != 2:
            raise NotImplementedError("batched w: only 2-D weights are on this path")
        self.K = _check_quant(w, scales, biases, group_size, bits)
        self.N = w.shape[0]
        self.w, self.s, self.b = _aligned(w), _aligned(scales), _aligned(biases)
        self.group_size, self.bits, self.dtype = group_size, bits, scales.dtype
        self.key = self._key(w, scales, biases, group_size, bits)

    @staticmethod
    def _key(w, scales, biases, group_size, bits):
        return (w.data_ptr(), scales.data_ptr(), biases.data_ptr(), w._version, scales._version,
                biases._version, group_size, bits)

    def matches(self, w, scales, biases, group_size: int, bits: int) -> bool:
        return self.key == self._key(w, scales, biases, group_size, bits)


_QMM_WS_BYTES: dict = {}


def quantized_matmul_prepared(x: torch.Tensor, p: PreparedWeights) -> torch.Tensor:
    """:func:`quantized_matmul` with weights validated by :class:`PreparedWeights`."""
    if (x.device != p.dev or x.dtype != p.dtype or x.ndim < 1 or x.shape[-1] != p.K
            or p.bits not in (4, 8) or not _kernel_dtype(x.dtype, p.dtype)):
        return quantized_matmul(x, p.w, p.s, p.b, group_size=p.group_size, bits=p.bits)
    N, K = p.N, p.K
    M = x.numel() // K
    out = torch.empty((*x.shape[:-1], N), dtype=x.dtype, device=p.dev)
    if M == 0 or N == 0:
        return out
    x_ = x if x.is_contiguous() and x.data_ptr() % 16 == 0 else _aligned(x)
    lib = _lib.lib()
    ws = None
    if M > 16:
        key = (M, N, K, p.group_size, p.bits)
        nbytes = _QMM_WS_BYTES.get(key)
        if nbytes is None:
            nbytes = int(lib.mq_quantized_matmul_workspace_size(M, N, K, p.group_size, p.bits))
            if len(_QMM_WS_BYTES) > 256:
                _QMM_WS_BYTES.clear()
            _QMM_WS_BYTES[key] = nbytes
        ws = _workspace(p.dev, nbytes) if nbytes else None
    rc = lib.mq_quantized_matmul_ws(x_.data_ptr(), p.w.data_ptr(), p.s.data_ptr(),
                                    p.b.data_ptr(), out.data_ptr(), M, N, K, p.group_size,
                                    p.bits, _DTYPE_CODE[x.dtype], 1,
                                    ws.data_ptr() if ws is not None else None,
                                    ws.numel() if ws is not None else 0, _stream_ptr(out))
    _lib.check(rc, "quantized_matmul")
    return out


def _stream_of(dev: torch.device) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


_WS_CACHE: dict = {}
# Buffers dropped from the caches after this process has captured a HIP
# graph: a captured kernel may still point at them (its graph can replay any
# time later), so they are kept alive instead of returned to the allocator.
_RETIRED: list = []
_SEEN_CAPTURE = False


def _capturing() -> bool:
    global _SEEN_CAPTURE
    c = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    _SEEN_CAPTURE = _SEEN_CAPTURE or c
    return c


def _retire(bufs) -> None:
    if _SEEN_CAPTURE:
        _RETIRED.extend(bufs)


def _dev_index(dev: torch.device) -> int:
    if dev.index is not None:
        return dev.index
    return torch.cuda.current_device() if dev.type == "cuda" else 0


def _workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The gather workspace of the current stream (kernels on one stream run
    in order, so consecutive calls can share it; calls on other streams get
    their own, as concurrent calls must not share one).  A buffer outgrown
    after a graph capture is kept alive (captured kernels may use it).  The
    capture check runs on every call, cache hits included: a capture that
    only ever found the buffer cached (warm-up on the capture stream, then
    capture) still pins it."""
    _capturing()
    key = (dev.type, _dev_index(dev), _stream_of(dev))
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _retire([buf])
        buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=dev)
        _WS_CACHE[key] = buf
    return buf


_LHS_CACHE: dict = {}


def _repeat_broadcast(bx: tuple, shape: tuple) -> bool:
    """True when x's batch dims ``bx`` broadcast to ``shape`` by repeating
    each batch over consecutive pairs (leading dims equal, trailing dims 1),
    e.g. tokens (T, 1) against expert indices (T, top_k): the C ABI's NULL
    lhs, pair p reading batch p / (P / B), needs no index table then."""
    bx = (1,) * (len(shape) - len(bx)) + tuple(bx)
    j = 0
    while j < len(shape) and bx[j] == shape[j]:
        j += 1
    return all(d == 1 for d in bx[j:])


def _default_lhs(dev: torch.device, bx: tuple, shape: tuple) -> Optional[torch.Tensor]:
    """x's own batch index per pair (lhs_indices=None), flattened over the
    broadcast shape; None when the C ABI's NULL lhs expresses it (identity
    or repeated batches).  Other broadcasts build a table, cached per shape
    and stream (it is written by kernels on the stream that built it)."""
    if _repeat_broadcast(bx, shape):
        return None
    capturing = _capturing()          # every call: a cached table used by a capture is pinned
    key = (dev.type, dev.index, _stream_of(dev), tuple(bx), tuple(shape))
    t = _LHS_CACHE.get(key)
    if t is None:
        B = math.prod(bx)
        t = (torch.arange(B, device=dev, dtype=torch.int32).reshape(bx).expand(shape)
             .reshape(-1).contiguous())
        # a table built under graph capture holds data only once the graph
        # replays, so it is not offered to later eager calls
        if not capturing:
            if len(_LHS_CACHE) > 64:
                _retire(_LHS_CACHE.values())
                _LHS_CACHE.clear()
            _LHS_CACHE[key] = t
    return t


def _as_index(t, dev) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        t = torch.as_tensor(t)
    if t.dtype.is_floating_point or t.dtype == torch.bool:
        raise ValueError(f"indices must be integers, got {t.dtype}")
    return t.to(device=dev)


def _gather_prep(x, banks, lhs_indices, rhs_indices, transpose, group_size, bits, mode,
                 alloc=True):
    """Validation and flattening shared by gather_qmm and gather_glu; ``banks``
    is a list of (w, scales, biases) of one shape.  Returns ``(out, args)``:
    ``args`` is None when there is nothing to compute, else the flattened
    call (``route``: "kernel", "rows" (more than 16 rows per pair), "slices"
    (more experts than the prep kernel's tables hold) or "composed" (no
    kernel for the format or dtype)).  With ``alloc=False`` (a caller that
    writes its own output) ``out`` is None."""
    for _, _, b in banks:
        _check_mode(mode, b)
    dev = _require_gpu(x, *[t for bank in banks for t in bank])
    w0 = banks[0][0]
    if x.ndim < 2 or w0.ndim < 3:
        raise ValueError("gather_qmm needs x (..., M, K) and w (..., N, K*bits/32) with a batch dim")
    for w, s, b in banks:
        if w.shape != w0.shape:
            raise ValueError(f"expert banks differ in shape: {tuple(w.shape)} and {tuple(w0.shape)}")
        Kq = _check_quant(w, s, b, group_size, bits)
        if s.dtype != banks[0][1].dtype:
            raise ValueError("expert banks differ in scale dtype")
    K, N = (Kq, w0.shape[-2]) if transpose else (w0.shape[-2], Kq)
    if x.shape[-1] != K:
        raise ValueError(
            f"x last dimension {x.shape[-1]} does not match the quantized weight K={K}")
    kernel_dtype = _kernel_dtype(x.dtype, banks[0][1].dtype)
    out_dtype = x.dtype if kernel_dtype else _result_dtype(x.dtype, banks[0][1].dtype)
    M = x.shape[-2]
    bx = tuple(x.shape[:-2])
    bw = tuple(w0.shape[:-2])
    B = math.prod(bx)
    E = math.prod(bw)
    lhs = None if lhs_indices is None else _as_index(lhs_indices, dev)
    rhs = (torch.arange(E, device=dev, dtype=torch.int32).reshape(bw) if rhs_indices is None
           else _as_index(rhs_indices, dev))
    lshape = bx if lhs is None else tuple(lhs.shape)
    try:
        shape = torch.broadcast_shapes(lshape, rhs.shape)
    except RuntimeError as exc:
        raise ValueError(f"lhs_indices {lshape} and rhs_indices "
                         f"{tuple(rhs.shape)} do not broadcast") from exc
    P = math.prod(shape)
    out = torch.empty((*shape, M, N), dtype=out_dtype, device=dev) if alloc else None
    if P == 0 or M == 0 or N == 0:
        return out, None
    lhs_f = (_default_lhs(dev, bx, tuple(shape)) if lhs is None
             else lhs.expand(shape).reshape(-1).to(torch.int32).contiguous())
    rhs_f = rhs.expand(shape).reshape(-1).to(torch.int32).contiguous()
    flat = []
    for w, s, b in banks:
        flat += [_aligned(w.reshape(E, *w.shape[-2:])),
                 _aligned(s.reshape(E, *s.shape[-2:])),
                 _aligned(b.reshape(E, *b.shape[-2:]))]
    if not (transpose and bits in (4, 8) and kernel_dtype):
        route = "composed"
    elif M > 16:
        route = "rows"
    elif P > _GATHER_FUSED_MAX_P and E > _GATHER_PREP_MAX_E:
        route = "slices"
    else:
        route = "kernel"
    args = dict(x=x.reshape(B, M, K), flat=flat, lhs=lhs_f, rhs=rhs_f, P=P, B=B, M=M, N=N, K=K,
                E=E, dev=dev, route=route, transpose=transpose, shape=tuple(shape),
                dtype=out_dtype)
    return out, args


# gather_qmm's kernels: up to this many pairs are grouped inside the matmul
# kernel, more go through the prep kernel, whose tables hold this many experts
_GATHER_FUSED_MAX_P = 256
_GATHER_PREP_MAX_E = 2048


def _ptr(t: Optional[torch.Tensor]):
    return t.data_ptr() if t is not None else None


def _gather_launch(x3, flat, lhs, rhs, out, P, B, M, N, K, E, group_size, bits,
                   sorted_indices) -> None:
    """One mq_gather_qmm call on flattened, validated arguments."""
    x_ = _aligned(x3)
    lib = _lib.lib()
    nbytes = int(lib.mq_gather_qmm_workspace_size(P, M))
    ws = _workspace(out.device, nbytes) if nbytes else None
    rc = lib.mq_gather_qmm(x_.data_ptr(), *[t.data_ptr() for t in flat], _ptr(lhs),
                           rhs.data_ptr(), out.data_ptr(), P, B, M, N, K, E, group_size, bits,
                           _DTYPE_CODE[x3.dtype], int(bool(sorted_indices)), _ptr(ws),
                           ws.numel() if ws is not None else 0, _stream_ptr(out))
    _lib.check(rc, "gather_qmm")


class GatherTables:
    """Segment tables of prefill gathers over one routing (mq_gather_tables):
    built once per MoE layer and passed to each of its gathers, as the
    reference builds ``_moe_gemm_tables`` once per layer for its up, gate and
    down grouped GEMMs (fused.py:3290-3316).  Holds its own device buffer,
    so gathers in between do not disturb it."""

    def __init__(self, buf: torch.Tensor, P: int, M: int, E: int):
        self.buf, self.P, self.M, self.E = buf, P, M, E


def gather_tables(rhs_indices: torch.Tensor, num_experts: int,
                  rows: int = 1) -> Optional[GatherTables]:
    """Tables for gathers whose pairs are the elements of ``rhs_indices``
    (each pair ``rows`` rows, x reached without an index table: mlx-lm's
    ``(T, 1)`` tokens against ``(T, top_k)`` experts, or one row per pair),
    or None below prefill widths (1024 output rows), where the gathers build
    none."""
    dev = _require_gpu(rhs_indices)
    rhs = _as_index(rhs_indices, dev).reshape(-1).to(torch.int32).contiguous()
    P = rhs.numel()
    if P * rows < _GLU_FUSED_MAX_ROWS or num_experts > _GATHER_PREP_MAX_E or rows > 16:
        return None
    lib = _lib.lib()
    nbytes = int(lib.mq_gather_qmm_workspace_size(P, rows))
    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    rc = lib.mq_gather_tables(None, rhs.data_ptr(), P, P, rows, num_experts, buf.data_ptr(),
                              nbytes, _stream_ptr(buf))
    if rc == _EUNSUPPORTED:
        return None
    _lib.check(rc, "gather_tables")
    return GatherTables(buf, P, rows, num_experts)


def _tables_launch(a, out, tables: GatherTables, group_size, bits) -> bool:
    """mq_gather_qmm_tables for a validated call; False when the call is not
    on the tables' kernel (the caller then runs the plain gather)."""
    if (tables.P, tables.M, tables.E) != (a["P"], a["M"], a["E"]) or a["lhs"] is not None:
        return False
    x_ = _aligned(a["x"])
    rc = _lib.lib().mq_gather_qmm_tables(
        x_.data_ptr(), *[t.data_ptr() for t in a["flat"]], None, a["rhs"].data_ptr(),
        out.data_ptr(), a["P"], a["B"], a["M"], a["N"], a["K"], a["E"], group_size, bits,
        _DTYPE_CODE[a["x"].dtype], tables.buf.data_ptr(), tables.buf.numel(), _stream_ptr(out))
    if rc == _EUNSUPPORTED:
        return False
    _lib.check(rc, "gather_qmm(tables)")
    return True


def gather_swiglu(x: torch.Tensor, gate, up, rhs_indices: torch.Tensor,
                  tables: GatherTables, transpose: bool = True, group_size: int = 64,
                  bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """A prefill MoE layer's gate and up projections and its activation:
    ``swiglu(gather_qmm(x, *gate, rhs_indices=rhs_indices, tables=tables),
    gather_qmm(x, *up, ...))``, bit for bit, in one launch over the layer's
    tables where the tables' kernel takes the call
    (mq_gather_swiglu_tables: each gathered x tile is read once for both
    banks), else as those three calls.  ``gate`` and ``up`` are
    ``(w, scales, biases)`` banks of one shape; x reaches pair p through
    batch ``p / top_k`` (no lhs table), as the tables were built.  The
    reference runs the gate and up grouped GEMMs over its shared tables and
    then the activation (fused.py:3294-3302)."""
    out, a = _gather_prep(x, [tuple(gate), tuple(up)], None, rhs_indices, transpose, group_size,
                          bits, mode)
    if a is None:
        return out
    if (a["route"] == "kernel" and a["lhs"] is None
            and (tables.P, tables.M, tables.E) == (a["P"], a["M"], a["E"])):
        x_ = _aligned(a["x"])
        rc = _lib.lib().mq_gather_swiglu_tables(
            x_.data_ptr(), *[t.data_ptr() for t in a["flat"]], None, a["rhs"].data_ptr(),
            out.data_ptr(), a["P"], a["B"], a["M"], a["N"], a["K"], a["E"], group_size, bits,
            _DTYPE_CODE[a["x"].dtype], tables.buf.data_ptr(), tables.buf.numel(),
            _stream_ptr(out))
        if rc != _EUNSUPPORTED:
            _lib.check(rc, "gather_swiglu")
            return out
    kw = dict(rhs_indices=rhs_indices, transpose=transpose, group_size=group_size, bits=bits,
              mode=mode, tables=tables)
    return swiglu(gather_qmm(x, *gate, **kw), gather_qmm(x, *up, **kw))


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``T(T(silu(gate)) * up)`` elementwise, ``silu(g) = g / (1 + exp(-g))``
    in float: mlx-lm SwitchGLU's activation between a MoE layer's gate / up
    and down projections (``switch_mlp.activation`` in the reference's
    prefill path, fused.py:3302), in one kernel pass (mq_swiglu)."""
    dev = _require_gpu(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError(f"gate {tuple(gate.shape)} {gate.dtype} and up {tuple(up.shape)} "
                         f"{up.dtype} differ")
    if gate.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"swiglu takes bfloat16 or float16, got {gate.dtype}")
    g, u = gate.contiguous(), up.contiguous()
    out = torch.empty_like(g)
    rc = _lib.lib().mq_swiglu(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                              _DTYPE_CODE[g.dtype], _stream_ptr(out))
    _lib.check(rc, "swiglu")
    return out


def _lhs_table(P: int, B: int, dev) -> torch.Tensor:
    """The table the C ABI's NULL lhs stands for: pair p reads batch p / (P / B)."""
    return torch.arange(P, device=dev, dtype=torch.int32) // (P // B)


def _gather_rows(a, out, group_size, bits, sorted_indices) -> torch.Tensor:
    """More than 16 rows per pair: row m of pair p is the one-row pair
    (lhs[p] * M + m, rhs[p]) of x viewed as B*M one-row batches, so the call
    is one gather of P*M one-row pairs (prefill-sized, the grouped kernel)."""
    P, B, M, N, K = a["P"], a["B"], a["M"], a["N"], a["K"]
    dev = a["dev"]
    rows = torch.arange(M, device=dev, dtype=torch.int32)
    lhs = a["lhs"] if a["lhs"] is not None else _lhs_table(P, B, dev)
    lhs1 = (lhs[:, None] * M + rows[None, :]).reshape(-1).contiguous()
    rhs1 = a["rhs"][:, None].expand(P, M).reshape(-1).contiguous()
    o = out.reshape(P * M, 1, N)
    _gather_launch(a["x"].reshape(B * M, 1, K), a["flat"], lhs1, rhs1, o, P * M, B * M, 1, N, K,
                   a["E"], group_size, bits, sorted_indices)
    return out


def _gather_slices(a, out, group_size, bits, sorted_indices) -> torch.Tensor:
    """More experts than the prep kernel's tables hold: the bank is run in
    slices of that many experts (contiguous views), pairs of other slices
    marked invalid (zero rows), and each pair's row kept from its slice."""
    P, E = a["P"], a["E"]
    rhs = a["rhs"]
    res = None
    for e0 in range(0, E, _GATHER_PREP_MAX_E):
        e1 = min(E, e0 + _GATHER_PREP_MAX_E)
        inside = (rhs >= e0) & (rhs < e1)
        r = torch.where(inside, rhs - e0, torch.full_like(rhs, -1))
        part = torch.empty_like(out) if res is not None else out
        flat = [t[e0:e1] for t in a["flat"]]
        _gather_launch(a["x"], flat, a["lhs"], r, part.reshape(P, a["M"], a["N"]), P, a["B"],
                       a["M"], a["N"], a["K"], e1 - e0, group_size, bits, sorted_indices)
        if res is None:
            res = part
        else:
            res.copy_(torch.where(inside.reshape(*a["shape"], 1, 1), part, res))
    return res


def _gather_composed(a, out, bank, group_size, bits) -> torch.Tensor:
    """Formats and dtypes without a gather kernel: each distinct expert's
    weights dequantized by this library (bit-exact) in the promoted dtype
    and applied to its pairs with one GPU GEMM; pairs with an out-of-range
    index get zero rows, as in the kernels.  (The expert list is read on the
    host, so this path synchronises the stream.)"""
    w, s, b = bank
    P, B, M, N, K, E = a["P"], a["B"], a["M"], a["N"], a["K"], a["E"]
    dt = a["dtype"]
    res = out.reshape(P, M, N)
    res.zero_()
    rhs = a["rhs"].long()
    lhs = (a["lhs"] if a["lhs"] is not None else _lhs_table(P, B, a["dev"])).long()
    valid = (rhs >= 0) & (rhs < E) & (lhs >= 0) & (lhs < B)
    rhs_h = torch.where(valid, rhs, torch.full_like(rhs, -1)).cpu()
    xs = a["x"].to(dt)
    for e in torch.unique(rhs_h).tolist():
        if e < 0:
            continue
        sel = (rhs_h == e).nonzero().reshape(-1).to(a["dev"])
        deq = dequantize(w[e], s[e].to(dt), b[e].to(dt), group_size, bits)
        xe = xs[lhs[sel]]                                     # (n_e, M, K)
        ye = (torch.nn.functional.linear(xe, deq) if a["transpose"]
              else torch.matmul(xe, deq))
        res[sel] = ye
    return out


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
               biases: Optional[torch.Tensor] = None, lhs_indices=None, rhs_indices=None,
               transpose: bool = True, group_size: int = 64, bits: int = 4,
               mode: str = "affine", sorted_indices: bool = False,
               tables: Optional["GatherTables"] = None) -> torch.Tensor:
    """``mx.gather_qmm``: per index pair, ``x[lhs] @ dequantize(w[rhs]).T``.

    ``x`` is ``(..., M, K)`` and ``w`` ``(..., N, K*bits/32)``; ``lhs_indices``
    index x's batch dims (default: all of them), ``rhs_indices`` index w's
    batch dims (default: all of them); the two broadcast together and the
    output is ``broadcast_shape + (M, N)``.  4/8-bit codes with bf16/fp16
    activations in the scales' dtype run on the gather kernels (more than 16
    rows per pair as one-row pairs, banks beyond the prep tables in expert
    slices); other formats and dtypes run as :func:`_gather_composed`.

    ``tables`` (:func:`gather_tables` of the same routing) skips building the
    segment tables where the call runs the thin grouped kernel (a MoE
    layer's gathers over one routing share one build); the result is the
    same bit for bit.
    """
    out, a = _gather_prep(x, [(w, scales, biases)], lhs_indices, rhs_indices, transpose,
                          group_size, bits, mode)
    if a is None:
        return out
    if tables is not None and a["route"] == "kernel" and _tables_launch(a, out, tables,
                                                                        group_size, bits):
        return out
    if a["route"] == "composed":
        return _gather_composed(a, out, a["flat"][:3], group_size, bits)
    if a["route"] == "rows":
        return _gather_rows(a, out, group_size, bits, sorted_indices)
    if a["route"] == "slices":
        return _gather_slices(a, out, group_size, bits, sorted_indices)
    _gather_launch(a["x"], a["flat"], a["lhs"], a["rhs"], out, a["P"], a["B"], a["M"], a["N"],
                   a["K"], a["E"], group_size, bits, sorted_indices)
    return out


def gather_glu(x: torch.Tensor, gate_w: torch.Tensor, gate_scales: torch.Tensor,
               gate_biases: Optional[torch.Tensor], up_w: torch.Tensor,
               up_scales: torch.Tensor, up_biases: Optional[torch.Tensor],
               lhs_indices=None, rhs_indices=None, transpose: bool = True,
               group_size: int = 64, bits: int = 4, mode: str = "affine",
               sorted_indices: bool = False) -> torch.Tensor:
    """Fused MoE gate+up+SiLU: ``silu(g) * u`` with ``g``, ``u`` the
    :func:`gather_qmm` products of the gate and up banks (same indices and
    broadcasting), summed in float and rounded once -- the reference's
    ``moe_glu.fused_glu`` (kernels/moe_glu.py:145-168) and
    ``moe_decode_fused.gate_up`` (kernels/moe_decode_fused.py:331-350).

    Fused in one kernel below 1024 output rows (decode / verify).  Above it
    (prefill), and for configurations the fused kernel does not take, the
    result is composed from two :func:`gather_qmm` calls and a float
    SiLU-multiply of their rounded outputs, as the reference keeps its stock
    path outside decode widths (fused.py:2476-2479)."""
    out, a = _gather_prep(x, [(gate_w, gate_scales, gate_biases), (up_w, up_scales, up_biases)],
                          lhs_indices, rhs_indices, transpose, group_size, bits, mode)
    if a is None:
        return out
    if a["route"] != "kernel" or a["P"] * a["M"] >= _GLU_FUSED_MAX_ROWS:
        kw = dict(lhs_indices=lhs_indices, rhs_indices=rhs_indices, transpose=transpose,
                  group_size=group_size, bits=bits, mode=mode, sorted_indices=sorted_indices)
        g = gather_qmm(x, gate_w, gate_scales, gate_biases, **kw)
        u = gather_qmm(x, up_w, up_scales, up_biases, **kw)
        return (torch.nn.functional.silu(g.float()) * u.float()).to(g.dtype)
    x_ = _aligned(a["x"])
    lib = _lib.lib()
    nbytes = int(lib.mq_gather_qmm_workspace_size(a["P"], a["M"]))
    ws = _workspace(a["dev"], nbytes) if nbytes else None
    rc = lib.mq_gather_glu(x_.data_ptr(), *[t.data_ptr() for t in a["flat"]],
                           _ptr(a["lhs"]), a["rhs"].data_ptr(), out.data_ptr(), a["P"],
                           a["B"], a["M"], a["N"], a["K"], a["E"], group_size, bits,
                           _DTYPE_CODE[x.dtype], _ptr(ws), ws.numel() if ws is not None else 0,
                           _stream_ptr(out))
    _lib.check(rc, "gather_glu")
    return out


# mq_gather_glu fuses below this many output rows (P * M)
_GLU_FUSED_MAX_ROWS = 1024

# mq_gather_qmm_combine folds up to this many (token, expert) pairs
_FOLD_MAX_P = 16
_EUNSUPPORTED = -2


def gather_qmm_combine(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                       biases: Optional[torch.Tensor], rhs_indices: torch.Tensor,
                       weights: torch.Tensor, transpose: bool = True, group_size: int = 64,
                       bits: int = 4, mode: str = "affine", sgate: Optional[torch.Tensor] = None,
                       shared: Optional[torch.Tensor] = None) -> torch.Tensor:
    """MoE down projection and combine: ``x`` holds one row per (token,
    expert) pair (``(T, top_k, 1, K)`` or anything of ``T * top_k * K``
    elements), ``rhs_indices`` ``(T, top_k)`` the experts, ``weights`` the
    router weights of the same shape; returns ``(T, N)`` =
    ``moe_combine(gather_qmm(x, w, ..., rhs_indices), None, weights, T,
    top_k, sgate, shared)``, bit for bit.

    For one or two decode tokens (up to 16 pairs) it is one kernel
    (mq_gather_qmm_combine: each workgroup computes 16 output columns of
    every pair and sums them per token), where the reference runs its decode
    down kernel and then the combine (kernels/moe_decode_fused.py:378-397,
    kernels/moe_combine.py:160-195); otherwise, and for configurations that
    kernel does not take, the two calls run (faster there)."""
    dev = _require_gpu(x, w, scales, biases, rhs_indices, weights, sgate, shared)
    if rhs_indices.ndim < 1 or rhs_indices.shape[-1] < 1:
        raise ValueError("rhs_indices must be (..., top_k)")
    top_k = int(rhs_indices.shape[-1])
    T = rhs_indices.numel() // top_k
    if weights.numel() != T * top_k:
        raise ValueError(f"weights has {weights.numel()} entries, expected {T * top_k}")
    if x.numel() != T * top_k * x.shape[-1]:
        raise ValueError("x must hold one row per (token, expert) pair")
    xs = x.reshape(T, top_k, 1, x.shape[-1])
    idx = rhs_indices.reshape(T, top_k)
    if (sgate is None) != (shared is None):
        raise ValueError("sgate and shared are given together")

    def composed():
        y = gather_qmm(xs, w, scales, biases, rhs_indices=idx, transpose=transpose,
                       group_size=group_size, bits=bits, mode=mode)
        return moe_combine(y.reshape(T * top_k, y.shape[-1]), None, weights, T, top_k, sgate,
                           shared)

    if T == 0 or T * top_k > _FOLD_MAX_P:
        return composed()
    _, a = _gather_prep(xs, [(w, scales, biases)], None, idx, transpose, group_size, bits, mode,
                        alloc=False)
    if a is None or a["route"] != "kernel" or a["M"] != 1 or a["dtype"] != x.dtype:
        return composed()
    N = a["N"]
    if shared is not None:
        if sgate.numel() != T or tuple(shared.shape) != (T, N):
            raise ValueError(f"sgate must hold {T} gates and shared be ({T}, {N})")
        if sgate.dtype != x.dtype or shared.dtype != x.dtype:
            raise ValueError("sgate and shared must have x's dtype")
    out = torch.empty((T, N), dtype=x.dtype, device=dev)
    w_ = weights.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    sg_ = sgate.reshape(-1).contiguous() if sgate is not None else None
    sh_ = shared.contiguous() if shared is not None else None
    x_ = _aligned(a["x"])
    lib = _lib.lib()
    rc = lib.mq_gather_qmm_combine(x_.data_ptr(), *[t.data_ptr() for t in a["flat"]],
                                   a["rhs"].data_ptr(), w_.data_ptr(), _ptr(sg_), _ptr(sh_),
                                   out.data_ptr(), T, top_k, N, a["K"], a["E"], group_size, bits,
                                   _DTYPE_CODE[x.dtype], _stream_ptr(out))
    if rc == _EUNSUPPORTED:
        return composed()
    _lib.check(rc, "gather_qmm_combine")
    return out


def moe_combine(y: torch.Tensor, inv: Optional[torch.Tensor], w: torch.Tensor, rows: int,
                top_k: int, sgate: Optional[torch.Tensor] = None,
                shared: Optional[torch.Tensor] = None) -> torch.Tensor:
    """MoE combine epilogue (kernels/moe_combine.py:160-195): from the down
    projection's expert-ordered output ``y`` ``(M, N)`` build ``(rows, N)``
    with ``out[t] = sum_k w[t*top_k + k] * y[inv[t*top_k + k]]``, float
    accumulation in k order, one rounding.  ``inv`` (int, ``(rows*top_k,)``)
    is the sorted row of each (token, k) -- ``argsort(order)``; ``None``
    when ``y`` is already in (token, k) order.  ``w`` is the router weight
    per (token, k), cast to float32 as the reference does.

    With the shared expert's sigmoided gate ``sgate`` (``(rows,)`` or
    ``(rows, 1)``, as :func:`moe_route` returns it) and its output
    ``shared`` ``(rows, N)``, both in y's dtype, the shared expert is merged
    in as the reference's decode combine rounds it
    (kernels/moe_route_decode.py:353-398): ``T(float(T(sum)) +
    float(T(sgate * shared)))``."""
    dev = _require_gpu(y, w, inv, sgate, shared)
    if y.ndim != 2:
        raise ValueError("y must be (M, N)")
    if y.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"moe_combine supports bf16/fp16 y, got {y.dtype}")
    M, N = y.shape
    rows, top_k = int(rows), int(top_k)
    if w.numel() != rows * top_k:
        raise ValueError(f"w has {w.numel()} weights, expected rows*top_k={rows * top_k}")
    if inv is None:
        if M != rows * top_k:
            raise ValueError(f"y has {M} rows, expected rows*top_k={rows * top_k} without inv")
        inv_ = None
    else:
        if inv.numel() != rows * top_k:
            raise ValueError(f"inv has {inv.numel()} entries, expected {rows * top_k}")
        inv_ = inv.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
    if (sgate is None) != (shared is None):
        raise ValueError("sgate and shared are given together")
    if shared is not None:
        if sgate.numel() != rows or tuple(shared.shape) != (rows, N):
            raise ValueError(f"sgate must hold {rows} gates and shared be ({rows}, {N})")
        if sgate.dtype != y.dtype or shared.dtype != y.dtype:
            raise ValueError("sgate and shared must have y's dtype")
    w_ = w.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    y_ = _aligned(y)
    out = torch.empty((rows, N), dtype=y.dtype, device=dev)
    if rows == 0:
        return out
    lib = _lib.lib()
    code = _dtype_code(y.dtype, y.dtype)
    if shared is None:
        rc = lib.mq_moe_combine(y_.data_ptr(), M, inv_.data_ptr() if inv_ is not None else None,
                                w_.data_ptr(), out.data_ptr(), rows, top_k, N, code,
                                _stream_ptr(out))
        _lib.check(rc, "moe_combine")
    else:
        sg_ = sgate.reshape(-1).contiguous()
        sh_ = _aligned(shared)
        rc = lib.mq_moe_combine_shared(y_.data_ptr(), M,
                                       inv_.data_ptr() if inv_ is not None else None,
                                       w_.data_ptr(), sg_.data_ptr(), sh_.data_ptr(),
                                       out.data_ptr(), rows, top_k, N, code, _stream_ptr(out))
        _lib.check(rc, "moe_combine_shared")
    return out


def moe_route(logits: torch.Tensor, top_k: int, x: Optional[torch.Tensor] = None,
              sgw: Optional[torch.Tensor] = None):
    """MoE routing (kernels/moe_route_decode.py:269-327 ``route``): for
    float32 router ``logits`` ``(..., E)`` the ``top_k`` experts in
    descending order (equal values: the smaller index first, as torch.topk),
    as int32 ``(..., top_k)``, and their softmax weights (float32, the
    largest logit subtracted, summed in float in that order).  With ``x``
    ``(..., H)`` and the shared expert's gate weight ``sgw`` ``(H,)`` (bf16 or
    fp16) also ``sigmoid(T(x . sgw))`` ``(..., 1)`` evaluated as MLX does in
    T; else None.  Returns ``(idx, weights, sgate)``."""
    dev = _require_gpu(logits, x, sgw)
    if logits.dtype != torch.float32:
        raise ValueError(f"moe_route takes float32 logits, got {logits.dtype}")
    if logits.ndim < 1:
        raise ValueError("logits must have an expert dimension")
    E = logits.shape[-1]
    lead = tuple(logits.shape[:-1])
    rows = math.prod(lead)
    top_k = int(top_k)
    if not 1 <= top_k <= E:
        raise ValueError(f"top_k={top_k} must be in 1..E={E}")
    if (x is None) != (sgw is None):
        raise ValueError("x and sgw are given together")
    idx = torch.empty((*lead, top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((*lead, top_k), dtype=torch.float32, device=dev)
    sg = None
    H, code = 0, 0
    if x is not None:
        if x.dtype not in (torch.bfloat16, torch.float16) or sgw.dtype != x.dtype:
            raise ValueError("x and sgw must share a bf16 / fp16 dtype")
        H = x.shape[-1]
        if tuple(x.shape[:-1]) != lead or sgw.numel() != H:
            raise ValueError(f"x must be {lead} + (H,) and sgw (H,), got {tuple(x.shape)}, "
                             f"{tuple(sgw.shape)}")
        sg = torch.empty((*lead, 1), dtype=x.dtype, device=dev)
        code = _DTYPE_CODE[x.dtype]
    if rows == 0:
        return idx, wts, sg
    l_ = logits.reshape(rows, E).contiguous()
    x_ = x.reshape(rows, H).contiguous() if x is not None else None
    g_ = sgw.reshape(-1).contiguous() if sgw is not None else None
    rc = _lib.lib().mq_moe_route(l_.data_ptr(), idx.data_ptr(), wts.data_ptr(), rows, E, top_k,
                                 _ptr(x_), _ptr(g_), _ptr(sg), H, code, _stream_ptr(idx))
    _lib.check(rc, "moe_route")
    return idx, wts, sg


def moe_block(x: torch.Tensor, logits: torch.Tensor, top_k: int, gate, up, down,
              sgw: Optional[torch.Tensor] = None, shared: Optional[torch.Tensor] = None,
              group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """A decode MoE block after its router matmul, as the reference's decode
    path runs it (kernels/moe_route_decode.py:151-327 and 353-398 around
    moe_decode_fused.py:331-397): ``moe_route`` (top-k, softmax weights and,
    with ``sgw``, the shared expert's gate ``sigmoid(T(x . sgw))``), the
    fused gate+up+SiLU gather over the selected experts, and the down
    projection with the router-weighted combine folded in, the shared
    expert's output ``shared`` ``(T, H)`` merged with its gate.  ``x`` is
    ``(T, H)``, ``logits`` float32 ``(T, E)``; ``gate``, ``up``, ``down``
    are ``(w, scales, biases)`` banks.  Returns ``(T, H_out)``: the same
    bits as calling the three steps one by one.  Up to 64 (token, expert)
    pairs over up to 512 experts the routing runs inside the gate+up
    launch (mq_moe_glu_route), one launch less on the dependent chain; up to
    8 tokens run the whole block as one launch (mq_moe_block) where its tile
    configuration applies."""
    if (sgw is None) != (shared is None):
        raise ValueError("sgw and shared are given together")
    T, H = x.shape
    if 1 <= T <= _BLOCK_MAX_T:
        out = _block_fused(x, logits, top_k, gate, up, down, sgw, shared, group_size, bits)
        if out is not None:
            return out
    routed = _glu_routed(x, logits, top_k, gate, up, sgw, group_size, bits)
    if routed is not None:
        h, idx, wts, sg = routed
    else:
        idx, wts, sg = moe_route(logits, top_k, x, sgw) if sgw is not None else \
            moe_route(logits, top_k)
        h = gather_glu(x.reshape(T, 1, 1, H), *gate, *up, rhs_indices=idx,
                       group_size=group_size, bits=bits)           # (T, k, 1, I)
    return gather_qmm_combine(h, *down, idx, wts, group_size=group_size, bits=bits,
                              sgate=sg, shared=shared)


# mq_moe_block / mq_moe_layer take up to this many tokens
_BLOCK_MAX_T = 8


def _block_fused(x, logits, top_k, gate, up, down, sgw, shared, group_size, bits):
    """The block of T <= 8 tokens in one launch (mq_moe_block: the same bits
    as the routed gate+up launch followed by the down projection and the
    combine, the down tiles starting behind a grid-wide arrival inside the
    launch), or None where that launch does not apply."""
    T = x.shape[0]
    (wd, sd, bd) = down
    E = logits.shape[-1]
    if (wd.ndim != 3 or wd.shape[0] != E or bd is None or sd.dtype != x.dtype
            or wd.dtype not in (torch.uint32, torch.int32)):
        return None
    routed_ok = _glu_routed_args(x, logits, top_k, gate, up, sgw, group_size, bits)
    if routed_ok is None:
        return None
    N1, K1 = routed_ok
    N2 = wd.shape[1]
    if _check_quant(wd, sd, bd, group_size, bits) != N1:
        raise ValueError(f"down bank K={wd.shape[-1] * 32 // bits} does not match the gate/up "
                         f"rows N={N1}")
    if shared is not None and (tuple(shared.shape) != (T, N2) or shared.dtype != x.dtype):
        raise ValueError(f"shared must be ({T}, {N2}) of x's dtype")
    _require_gpu(wd, sd, bd, shared)
    dev = x.device
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    sgate = torch.empty((T, 1), dtype=x.dtype, device=dev) if sgw is not None else None
    h = torch.empty((T, top_k, 1, N1), dtype=x.dtype, device=dev)
    out = torch.empty((T, N2), dtype=x.dtype, device=dev)
    x_ = _aligned(x.contiguous())
    lg = logits.contiguous()
    g_ = sgw.reshape(-1).contiguous() if sgw is not None else None
    sh_ = shared.contiguous() if shared is not None else None
    (wg, sg_, bg), (wu, su, bu) = gate, up
    banks = [_aligned(t) for t in (wg, sg_, bg, wu, su, bu, wd, sd, bd)]
    rc = _lib.lib().mq_moe_block(x_.data_ptr(), lg.data_ptr(), *[t.data_ptr() for t in banks],
                                 _ptr(g_), _ptr(sh_), idx.data_ptr(), wts.data_ptr(),
                                 _ptr(sgate), h.data_ptr(), out.data_ptr(), T, top_k, N1, K1,
                                 N2, E, group_size, bits, _DTYPE_CODE[x.dtype], _stream_ptr(out))
    if rc == _EUNSUPPORTED:
        return None
    _lib.check(rc, "moe_block")
    return out


def moe_layer(x: torch.Tensor, rhs_indices: torch.Tensor, weights: torch.Tensor, gate, up,
              down, group_size: int = 64, bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """A decode MoE layer after its routing (the reference's fused decode
    route, kernels/moe_decode_fused.py:331-397 with the combine of
    kernels/moe_combine.py:160-195): ``gather_glu(x, gate, up, rhs_indices)``
    then ``gather_qmm_combine(h, down, rhs_indices, weights)``.  ``x`` is
    ``(T, K)``, ``rhs_indices`` and the router ``weights`` ``(T, top_k)``;
    ``gate``, ``up``, ``down`` are ``(w, scales, biases)`` banks.  Returns
    ``(T, N)``, the bits of the two calls; up to 8 tokens run both in one
    launch (mq_moe_layer) where its tile configurations apply."""
    T, K = x.shape
    idx = rhs_indices.reshape(T, -1)
    if 1 <= T <= _BLOCK_MAX_T and mode == "affine":
        out = _layer_fused(x, idx, weights, gate, up, down, group_size, bits)
        if out is not None:
            return out
    h = gather_glu(x.reshape(T, 1, 1, K), *gate, *up, rhs_indices=idx, group_size=group_size,
                   bits=bits, mode=mode)
    return gather_qmm_combine(h, *down, idx, weights.reshape(idx.shape), group_size=group_size,
                              bits=bits, mode=mode)


def _layer_fused(x, idx, weights, gate, up, down, group_size, bits):
    """The layer of T <= 8 tokens in one launch (mq_moe_layer), or None where
    that launch does not apply."""
    (wg, sg_, bg), (wu, su, bu), (wd, sd, bd) = gate, up, down
    T, top_k = x.shape[0], idx.shape[-1]
    if (x.dtype not in (torch.bfloat16, torch.float16) or bits not in (4, 8)
            or bg is None or bu is None or bd is None or wg.ndim != 3 or wg.shape != wu.shape
            or wd.ndim != 3 or wd.shape[0] != wg.shape[0] or top_k > 8 or T > _BLOCK_MAX_T
            or T * top_k > 64 or idx.numel() != T * top_k or weights.numel() != T * top_k
            or sg_.dtype != x.dtype or su.dtype != x.dtype or sd.dtype != x.dtype
            or any(w.dtype not in (torch.uint32, torch.int32) for w in (wg, wu, wd))):
        return None
    dev = _require_gpu(x, idx, weights, wg, sg_, bg, wu, su, bu, wd, sd, bd)
    E, N1 = wg.shape[0], wg.shape[1]
    K1 = _check_quant(wg, sg_, bg, group_size, bits)
    _check_quant(wu, su, bu, group_size, bits)
    if K1 != x.shape[-1]:
        raise ValueError(f"x last dimension {x.shape[-1]} does not match the quantized weight "
                         f"K={K1}")
    if _check_quant(wd, sd, bd, group_size, bits) != N1:
        return None
    N2 = wd.shape[1]
    h = torch.empty((T, top_k, 1, N1), dtype=x.dtype, device=dev)
    out = torch.empty((T, N2), dtype=x.dtype, device=dev)
    x_ = _aligned(x.contiguous())
    idx_ = idx.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
    w_ = weights.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    banks = [_aligned(t) for t in (wg, sg_, bg, wu, su, bu, wd, sd, bd)]
    rc = _lib.lib().mq_moe_layer(x_.data_ptr(), idx_.data_ptr(), w_.data_ptr(),
                                 *[t.data_ptr() for t in banks], h.data_ptr(), out.data_ptr(), T,
                                 top_k, N1, K1, N2, E, group_size, bits, _DTYPE_CODE[x.dtype],
                                 _stream_ptr(out))
    if rc == _EUNSUPPORTED:
        return None
    _lib.check(rc, "moe_layer")
    return out


def _glu_routed_args(x, logits, top_k, gate, up, sgw, group_size, bits):
    """(N, K) of the routed gate+up launch's banks, or None where that launch
    does not apply (more than 64 pairs or 512 experts, other formats)."""
    T, H = x.shape
    (wg, sg_, bg), (wu, su, bu) = gate, up
    E = logits.shape[-1]
    if (x.dtype not in (torch.bfloat16, torch.float16) or logits.dtype != torch.float32
            or tuple(logits.shape) != (T, E) or T * top_k > 64 or E > 512 or top_k > E
            or bits not in (4, 8) or bg is None or bu is None
            or wg.ndim != 3 or wg.shape != wu.shape or wg.shape[0] != E
            or sg_.dtype != x.dtype or su.dtype != x.dtype
            or (sgw is not None and sgw.dtype != x.dtype)):
        return None
    _require_gpu(x, logits, wg, sg_, bg, wu, su, bu, sgw)
    K = _check_quant(wg, sg_, bg, group_size, bits)
    _check_quant(wu, su, bu, group_size, bits)
    if K != H:
        raise ValueError(f"x last dimension {H} does not match the quantized weight K={K}")
    return wg.shape[1], K


def _glu_routed(x, logits, top_k, gate, up, sgw, group_size, bits):
    """Routing and the fused gate+up+SiLU in one launch (mq_moe_glu_route:
    the same bits as moe_route then gather_glu), or None where that launch
    does not apply (more than 64 pairs or 512 experts, other formats)."""
    T, H = x.shape
    (wg, sg_, bg), (wu, su, bu) = gate, up
    E = logits.shape[-1]
    nk = _glu_routed_args(x, logits, top_k, gate, up, sgw, group_size, bits)
    if nk is None:
        return None
    N, K = nk
    dev = x.device
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    sgate = torch.empty((T, 1), dtype=x.dtype, device=dev) if sgw is not None else None
    h = torch.empty((T, top_k, 1, N), dtype=x.dtype, device=dev)
    x_ = _aligned(x.contiguous())
    lg = logits.contiguous()
    g_ = sgw.reshape(-1).contiguous() if sgw is not None else None
    banks = [_aligned(t) for t in (wg, sg_, bg, wu, su, bu)]
    rc = _lib.lib().mq_moe_glu_route(x_.data_ptr(), lg.data_ptr(),
                                     *[t.data_ptr() for t in banks], _ptr(g_), idx.data_ptr(),
                                     wts.data_ptr(), _ptr(sgate), h.data_ptr(), T, top_k, N, K,
                                     E, group_size, bits, _DTYPE_CODE[x.dtype], _stream_ptr(h))
    if rc == _EUNSUPPORTED:
        return None
    _lib.check(rc, "moe_glu_route")
    return h, idx, wts, sgate


def launch_count() -> int:
    """Kernel launches made through the library so far (proof the HIP path ran)."""
    return _lib.launch_count()


def set_row_identity(on: bool) -> bool:
    """Run one-row ``quantized_matmul`` calls on the 2..32-row kernel family,
    so every output row is bit-identical whatever the number of rows in the
    call (a decode step and a speculative verify of the same token agree bit
    for bit).  Off by default: one-row calls then take their own faster
    kernel, within the output tolerance of the wide rows but rounded in
    another order.  The reference's counterpart is its opt-in small-M route,
    whose rows of 2..8-row calls are bit-identical to the one-row call
    (kernels/qmv_small_m.py:289-307, dispatch.py:337-347).  Process-wide;
    returns the previous setting."""
    return bool(_lib.lib().mq_set_row_identity(1 if on else 0))


@contextlib.contextmanager
def row_identity(on: bool = True):
    """``set_row_identity(on)`` for the ``with`` block, restored after."""
    prev = set_row_identity(on)
    try:
        yield
    finally:
        set_row_identity(prev)


__all__: Sequence[str] = ("quantize", "dequantize", "quantized_matmul", "quantized_matmul_prepared",
                          "PreparedWeights", "gather_qmm", "gather_glu", "moe_combine",
                          "gather_tables", "GatherTables", "swiglu", "moe_block",
                          "launch_count", "set_row_identity", "row_identity")
