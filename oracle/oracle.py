"""CPU oracle for MLX-format affine quantized matmul.  TEST INFRASTRUCTURE ONLY.

Nothing in the ``mlxturbo_amd`` package imports this module.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker of the HIP path, never as the thing measured or
shipped.

The algorithm restated here lives in MLX 0.32.2 (``mlx==0.32.2`` pinned in the
reference's ``uv.lock:284-300``; not vendored, not importable here).  The
reference's in-tree statements of it are cited per function.  Every function
below is pinned by independent checks in ``tests/test_oracle.py`` and
``tests/test_quantize_oracle.py``:

=====================  ========================================================
function               pinned by
=====================  ========================================================
pack / unpack          hand-written words (0x76543210 -> codes 0..7; 3/5/6-bit
                       byte patterns), round trip, and the reference's own
                       per-width decode formulas (_steel_flat.py:1184-1254)
                       applied to random bytes
bf16_bits / f16_bits   torch's own float->bf16/fp16 casts (RNE), exhaustive
                       special values (ties, carries into the exponent, inf,
                       subnormals)
dequantize             closed form cases: q=0 -> b, s=0 -> b, exactness of
                       s*q in fp32, and a float64 route rounded once
quantized_matmul_ref   brute-force pure-Python loop on tiny shapes, linearity
                       in x, row independence, column independence
gather_qmm_ref         dense matmul on w[idx] per pair, sort invariance
gather_glu_ref         closed-form SiLU values (silu(0) = 0, silu(1) =
                       1/(1+e^-1), silu(x) -> x / 0 at +-20), a zero gate
                       bank zeroes the output whatever the up bank, swapping
                       gate and up changes it, linearity in the up bank
moe_combine_ref        pure-Python loop on tiny shapes, one-hot weights copy
                       rows, identity inv equals the unsorted layout, linearity
                       in w; the shared-expert merge: gate 0 / shared 0 leave
                       the sum's rounding alone, gate 1 adds shared exactly
                       where the sum is exact
moe_route_ref          brute force over all expert subsets on tiny E (the
                       chosen set maximises the sum of logits), torch.topk's
                       indices and softmax on distinct logits, ties broken
                       by the smaller index, weights summing to one
sigmoid_t              closed-form points (sigmoid(0) = 1/2, large |s|
                       saturating to 0 / 1), symmetry s(-x) = 1 - s(x) up to
                       T's rounding, and a float64 sigmoid within two T ulps
quantize               exact affine grids round-trip bit for bit for every
                       width, group size, dtype and both scale signs; known
                       codes for points off the grid (half-to-even); a
                       hand-derived edge-exact scale (min -1, max 0.55 ->
                       0.1); constant and below-floor constant groups; a
                       far-end error bound from each group's range; seven
                       planted mistakes each fail these checks.  MLX's own
                       quantizer source is absent, so its conventions where
                       these checks are blind (a tie between |min| and |max|)
                       remain unpinned
=====================  ========================================================
"""

from __future__ import annotations

import numpy as np

DTYPES = ("bfloat16", "float16", "float32")


# --------------------------------------------------------------------- packing

BITS = (2, 3, 4, 5, 6, 8)


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes ``[..., K]`` into uint32 words: a little-endian
    bitstream, code ``i`` at bits ``[bits*i, bits*i + bits)`` of the row.

    For 2/4/8 bits this is "code ``j`` of word ``i`` is element
    ``i*(32/bits) + j`` at bit ``bits*j``" (mlxturbo/fast_qmm.py:96-106 reads
    nibble ``t`` of word ``p0`` as element ``t``; _steel_flat.py:1251-1254
    reads byte ``i`` as element ``i``).  For 3/5/6 bits, eight (3, 5 bits) or
    four (6 bits) codes fill 3/5/3 bytes, lowest code in the lowest bits
    (_steel_flat.py:1158-1167 pack factor and bytes per pack; the decode of
    each code at 1195-1206, 1218-1233, 1237-1247).
    """
    if bits not in BITS:
        raise ValueError(f"bits={bits} is not an MLX affine width {BITS}")
    codes = np.asarray(codes, dtype=np.uint64)
    K = codes.shape[-1]
    if (K * bits) % 32:
        raise ValueError("K*bits must be a multiple of 32")
    if codes.size and int(codes.max()) >= (1 << bits):
        raise ValueError("code out of range")
    if 32 % bits == 0:                                   # whole codes per word
        per = 32 // bits
        c = codes.reshape(*codes.shape[:-1], K // per, per)
        return (c << (np.arange(per, dtype=np.uint64) * bits)).sum(axis=-1).astype(np.uint32)
    shifts = np.arange(bits, dtype=np.uint64)
    stream = ((codes[..., None] >> shifts) & 1).astype(np.uint8)       # [..., K, bits]
    stream = stream.reshape(*codes.shape[:-1], K * bits // 8, 8)
    byte = (stream << np.arange(8, dtype=np.uint8)).sum(axis=-1, dtype=np.uint32)
    byte = byte.astype(np.uint8).reshape(*codes.shape[:-1], K * bits // 32, 4)
    word = (byte.astype(np.uint32) << (np.arange(4, dtype=np.uint32) * 8)).sum(
        axis=-1, dtype=np.uint64)
    return word.astype(np.uint32)


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of :func:`pack`: uint32 ``[..., Kw]`` -> codes ``[..., Kw*32/bits]``."""
    if bits not in BITS:
        raise ValueError(f"bits={bits} is not an MLX affine width {BITS}")
    w = np.asarray(w, dtype=np.uint32)
    Kw = w.shape[-1]
    if 32 % bits == 0:                                   # whole codes per word
        per = 32 // bits
        c = (w[..., None] >> (np.arange(per, dtype=np.uint32) * bits)) & np.uint32((1 << bits) - 1)
        return c.reshape(*w.shape[:-1], Kw * per)
    stream = ((w[..., None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint32)
    stream = stream.reshape(*w.shape[:-1], Kw * 32 // bits, bits)
    return (stream << np.arange(bits, dtype=np.uint32)).sum(axis=-1, dtype=np.uint32)


# ------------------------------------------------------------ float formats

def bf16_bits(f32: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even), returned as uint16 bits.

    Integer formulation: add 0x7FFF plus the lowest kept bit, truncate.
    NaN maps to a quiet NaN with the sign kept.
    """
    u = np.asarray(f32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
    nan = np.isnan(np.asarray(f32, dtype=np.float32))
    r = np.where(nan, ((u >> 16) & 0x8000) | 0x7FC0, r)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits(f32: np.ndarray) -> np.ndarray:
    """Round float32 to IEEE half (RNE), as uint16 bits (numpy's cast is RNE)."""
    with np.errstate(over="ignore"):
        return np.asarray(f32, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(bits_or_vals: np.ndarray, dtype: str) -> np.ndarray:
    """Decode storage (uint16 bits for 16-bit types, float32 otherwise) to float32."""
    if dtype == "bfloat16":
        return bf16_to_f32(bits_or_vals)
    if dtype == "float16":
        return f16_to_f32(bits_or_vals)
    return np.asarray(bits_or_vals, dtype=np.float32)


def from_f32(f32: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to ``dtype`` storage (uint16 bits, or float32)."""
    if dtype == "bfloat16":
        return bf16_bits(f32)
    if dtype == "float16":
        return f16_bits(f32)
    return np.asarray(f32, dtype=np.float32)


# ------------------------------------------------------------------ dequant

def dequantize_f32(w: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                   group_size: int, bits: int, dtype: str) -> np.ndarray:
    """``fp32(s*q + b)`` before the final rounding to ``dtype``.

    MLX computes ``float s = float(scale); float b = float(bias);``
    ``w = static_cast<T>(s*q + b)`` (_steel_flat.py:1179-1180, 1210-1215 for
    4-bit, 1251-1254 for 8-bit).  ``s*q`` is exact in float32 for 16-bit
    scale types (<= 11+8 significant bits), so the value is ``s*q+b`` rounded
    once to float32, whether or not the hardware fuses the multiply-add.
    """
    codes = unpack(w, bits).astype(np.float32)
    s = to_f32(scales, dtype)
    b = to_f32(biases, dtype)
    K = codes.shape[-1]
    if K % group_size:
        raise ValueError("K must be a multiple of group_size")
    s = np.repeat(s, group_size, axis=-1)
    b = np.repeat(b, group_size, axis=-1)
    if s.shape != codes.shape:
        raise ValueError(f"scales shape {scales.shape} does not match w {w.shape}")
    with np.errstate(over="ignore", invalid="ignore"):
        return (s * codes + b).astype(np.float32)


def dequantize(w, scales, biases, group_size: int = 64, bits: int = 4,
               dtype: str = "bfloat16") -> np.ndarray:
    """Bit-exact dequantized weights in ``dtype`` storage (uint16 bits or float32).

    Reference: mx.dequantize / QuantizedBlockLoader (_steel_flat.py:1169-1256,
    1324-1335: the prefill tile loader dequantizes to T=bfloat16 in
    threadgroup memory).
    """
    return from_f32(dequantize_f32(w, scales, biases, group_size, bits, dtype), dtype)


# ------------------------------------------------------------------- matmul

def quantized_matmul_ref(x, w, scales, biases, group_size: int = 64, bits: int = 4,
                         dtype: str = "bfloat16", transpose: bool = True) -> np.ndarray:
    """fp32 reference ``x . deq(W)^T`` over ``dtype``-rounded dequantized weights.

    ``x`` is ``dtype`` storage ``[M, K]``.  Accumulation is float64, rounded
    once to float32 at the end.  This is the reference the reference's own
    fp32 checks use: test_qmm_wide_shapes.py:35-42 (``mx.dequantize`` then
    ``.astype(float32)`` then matmul), moe_verify_gather.py:923-939.
    With ``transpose=False`` ``w`` is ``[K, N*bits/32]`` and the result is
    ``x . deq(W)`` (MLX's non-transposed layout).
    """
    xf = to_f32(x, dtype).astype(np.float64)
    deq = to_f32(dequantize(w, scales, biases, group_size, bits, dtype), dtype)
    deq = deq.astype(np.float64)
    if transpose:
        out = xf @ deq.T
    else:
        out = xf @ deq
    return out.astype(np.float32)


def gather_qmm_ref(x, w, scales, biases, lhs_indices, rhs_indices,
                   group_size: int = 64, bits: int = 4, dtype: str = "bfloat16",
                   transpose: bool = True) -> np.ndarray:
    """Per-pair loop: ``out[p] = x_b[lhs[p]] . deq(w_e[rhs[p]])^T``.

    ``x`` is ``[B, M, K]`` (batch flattened), ``w`` ``[E, N, Kw]``; indices are
    flat ``[P]``.  Semantics of ``mx.gather_qmm`` as used by mlx-lm's
    ``QuantizedSwitchLinear`` (moe_verify_gather.py:11-27, fused.py:2389-2394).
    Returns float32 ``[P, M, N]``.
    """
    lhs = np.asarray(lhs_indices).reshape(-1)
    rhs = np.asarray(rhs_indices).reshape(-1)
    out = []
    cache = {}
    for p in range(lhs.shape[0]):
        e = int(rhs[p])
        if e not in cache:
            deq = to_f32(dequantize(w[e], scales[e], biases[e], group_size, bits, dtype), dtype)
            cache[e] = deq.astype(np.float64)
        xf = to_f32(x[int(lhs[p])], dtype).astype(np.float64)
        out.append(xf @ cache[e].T if transpose else xf @ cache[e])
    return np.stack(out).astype(np.float32)


def gather_glu_ref(x, gate, up, lhs_indices, rhs_indices, group_size: int = 64,
                   bits: int = 4, dtype: str = "bfloat16") -> np.ndarray:
    """Fused MoE gate+up+SiLU: ``silu(g) * u`` with ``g`` / ``u`` the
    :func:`gather_qmm_ref` products of the gate and up banks (``gate`` and
    ``up`` are ``(w, scales, biases)``), ``silu(g) = g / (1 + exp(-g))``,
    evaluated in float64 and returned un-rounded float32 ``[P, M, N]``.
    Restates the epilogue of kernels/moe_glu.py:94-101 (float sums, float
    sigmoid, product rounded once to T) and kernels/moe_decode_fused.py:
    135-223 (same epilogue with per-token x rows)."""
    g = gather_qmm_ref(x, *gate, lhs_indices, rhs_indices, group_size, bits, dtype)
    u = gather_qmm_ref(x, *up, lhs_indices, rhs_indices, group_size, bits, dtype)
    g = g.astype(np.float64)
    with np.errstate(over="ignore"):
        act = g / (1.0 + np.exp(-g))
    return (act * u.astype(np.float64)).astype(np.float32)


# ------------------------------------------------------------- moe combine

def moe_combine_ref(y, inv, w, rows: int, top_k: int, dtype: str = "bfloat16",
                    sgate=None, shared=None) -> np.ndarray:
    """``out[t] = sum_k w[t*top_k + k] * y[inv[t*top_k + k]]`` accumulated in
    float32 in k order (each step rounded once, as an fma), returned
    un-rounded float32 ``[rows, N]``.  ``inv`` ``None`` means rows of ``y``
    are in (token, k) order.  Restates kernels/moe_combine.py:63-97 (the
    per-thread loop ``acc += wk * (float)p[v]``) and its caller contract
    (moe_combine.py:160-195: inv = argsort(order), w cast to float32).

    With ``sgate`` ([rows], the sigmoided shared-expert gate) and ``shared``
    ([rows, N]) in ``dtype``: the shared expert merged in as the reference's
    decode combine rounds it (kernels/moe_route_decode.py:392-398): the sum
    rounded to T, ``T(sgate * shared)``, their float32 sum returned (the
    caller's final rounding to T is the kernel's last one).
    """
    yf = to_f32(y, dtype).astype(np.float64)
    w = np.asarray(w, dtype=np.float32).reshape(-1).astype(np.float64)
    idx = (np.arange(rows * top_k) if inv is None else np.asarray(inv).reshape(-1))
    out = np.zeros((rows, yf.shape[1]), dtype=np.float32)
    for k in range(top_k):
        sel = idx[np.arange(rows) * top_k + k]
        # w*y is exact in float64 (24 + 8 significant bits); the sum with the
        # float32 accumulator rounds once to float32
        out = (w[np.arange(rows) * top_k + k][:, None] * yf[sel] + out.astype(np.float64)
               ).astype(np.float32)
    if shared is not None:
        s1 = to_f32(from_f32(out, dtype), dtype)
        sg = to_f32(np.asarray(sgate).reshape(-1), dtype).astype(np.float64)[:, None]
        sh = to_f32(np.asarray(shared).reshape(rows, -1), dtype).astype(np.float64)
        # a 16-bit by 16-bit product is exact in float32: one rounding to T
        m1 = to_f32(from_f32((sg * sh).astype(np.float32), dtype), dtype)
        out = (s1 + m1).astype(np.float32)
    return out


# ----------------------------------------------------------------- routing

def sigmoid_t(s, dtype: str = "bfloat16") -> np.ndarray:
    """MLX's Sigmoid evaluated in T one operation at a time, as the reference
    writes it (kernels/moe_route_decode.py:141-146: ``y = 1 / (1 + exp(|x|));
    x < 0 ? y : 1 - y`` on T values): every intermediate rounded to T.  ``s``
    holds T values; returns the T results as float32."""
    r = lambda a: to_f32(from_f32(np.asarray(a, np.float32), dtype), dtype)
    x = np.asarray(s, np.float32)
    e = r(np.exp(np.abs(x).astype(np.float64)))
    d = r(1.0 + e.astype(np.float64))
    y = r(1.0 / d.astype(np.float64))
    return np.where(x < 0, y, r(1.0 - y.astype(np.float64)))


def moe_route_ref(logits, top_k: int, x=None, sgw=None, dtype: str = "bfloat16"):
    """Top-k routing with softmax weights, restating the reference's decode
    route (kernels/moe_route_decode.py:205-244 and 269-327): per row, the
    top_k experts in descending order of logit (equal values: the smaller
    expert index first; -0 equals +0), ``ex_j = exp(v_j - v_0)`` in float32,
    ``w_j = ex_j / sum`` with the sum accumulated in float32 in selection
    order.  Returns ``(idx int32 [rows, k], w float32 [rows, k], sgate)``;
    with ``x`` ([rows, H], T values) and ``sgw`` ([H]) ``sgate`` is
    ``sigmoid_t(T(x . sgw))`` as float32 (the dot exact in float64, then
    rounded to float32 and to T: a kernel summing in float32 in another
    order may differ from it by one T ulp), else None."""
    L = np.asarray(logits, np.float32)
    rows, E = L.shape
    idx = np.zeros((rows, top_k), np.int32)
    w = np.zeros((rows, top_k), np.float32)
    for r in range(rows):
        order = sorted(range(E), key=lambda e: (-float(L[r, e]), e))[:top_k]
        v = L[r, order]
        # the difference rounded in float32 (as the reference's float code),
        # its exp correctly rounded
        ex = np.exp((v - v[0]).astype(np.float64)).astype(np.float32)
        tot = np.float32(0.0)
        for e in ex:
            tot = np.float32(tot + e)
        idx[r] = order
        w[r] = ex / tot
    sg = None
    if x is not None:
        xs = to_f32(np.asarray(x), dtype).astype(np.float64).reshape(rows, -1)
        gw = to_f32(np.asarray(sgw), dtype).astype(np.float64).reshape(-1)
        dot = (xs @ gw).astype(np.float32)
        sg = sigmoid_t(to_f32(from_f32(dot, dtype), dtype), dtype)
    return idx, w, sg


# ----------------------------------------------------------------- quantize

def quantize(w_fp: np.ndarray, group_size: int = 64, bits: int = 4,
             dtype: str = "bfloat16"):
    """Affine quantizer in the form MLX documents (``mx.quantize``, mode
    "affine"; called by the reference at rebit.py:119 and
    kernels/moe_verify_gather.py:887).

    Per group: ``scale = max((max-min)/(2^bits-1), 1e-7)``, signed towards the
    edge of larger magnitude; the edge maps to a code exactly
    (``q0 = round(edge/scale)``, ``scale = edge/q0`` when ``q0 != 0``) and
    ``bias = edge`` (0 when ``q0 == 0``); codes
    ``q = clip(round((w-bias)/scale), 0, 2^bits-1)`` use the float32 scale and
    bias, which are then rounded to ``dtype`` for storage.  Rounding is
    half-to-even (``mx.round``).  NaN propagates through the group minimum and
    maximum (numpy's reductions) and a NaN code becomes 0.  MLX's source is
    not in the container; the tests pin this restatement by exact grids,
    known answers and error bounds, not by MLX's own outputs.
    """
    w = np.asarray(w_fp, dtype=np.float32)
    K = w.shape[-1]
    if K % group_size:
        raise ValueError("K must be a multiple of group_size")
    g = w.reshape(*w.shape[:-1], K // group_size, group_size)
    wmax = g.max(axis=-1)
    wmin = g.min(axis=-1)
    n_bins = np.float32((1 << bits) - 1)
    mask = np.abs(wmin) > np.abs(wmax)
    scale = np.maximum((wmax - wmin) / n_bins, np.float32(1e-7)).astype(np.float32)
    scale = np.where(mask, scale, -scale).astype(np.float32)
    edge = np.where(mask, wmin, wmax).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    scale = np.where(q0 != 0, edge / np.where(q0 != 0, q0, np.float32(1)), scale).astype(np.float32)
    bias = np.where(q0 == 0, np.float32(0), edge).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint((g - bias[..., None]) / scale[..., None])
    q = np.nan_to_num(q, nan=0.0)
    q = np.clip(q, 0, n_bins).astype(np.uint32).reshape(w.shape)
    return pack(q, bits), from_f32(scale, dtype), from_f32(bias, dtype)


# ---------------------------------------------------------------- tolerance

def ulp_bf16(a: np.ndarray) -> np.ndarray:
    """Spacing of bfloat16 numbers at |a| (normal range)."""
    a = np.maximum(np.abs(np.asarray(a, dtype=np.float64)), 2.0 ** -126)
    e = np.floor(np.log2(a))
    return 2.0 ** (e - 7)


def ulp_f16(a: np.ndarray) -> np.ndarray:
    a = np.maximum(np.abs(np.asarray(a, dtype=np.float64)), 2.0 ** -14)
    e = np.floor(np.log2(a))
    return 2.0 ** (e - 10)


def check_output(out_f32: np.ndarray, ref_f32: np.ndarray, dtype: str = "bfloat16",
                 rel_l2: float = None, max_ulp: float = 2.0) -> dict:
    """The correctness contract for matmul outputs (the tolerance lives here).

    * ``relL2(out, round_dtype(ref)) <= 1e-3`` and
    * ``|out - ref| <= 2 ulp(max(|ref|, 2^-8 * rms(ref row)))`` elementwise,

    where ``ref`` is the fp32-accumulated product over dtype-rounded
    dequantized weights.  The rms floor keeps cancellation-near-zero outputs
    from demanding sub-ulp accuracy (the reference moved to atol+rtol and RMS
    normalisation for the same reason: moe_verify_gather.py:942-956,
    bench/test_moe_combine_fold.py:35-40).  For float32 outputs (the
    composed routes) relL2 must be <= 1e-5 and the elementwise bound is 2 x
    2^-12 of max(|ref|, 2^-4 * rms(ref row)): float32 GEMMs summing in another
    order stay far inside (their error is ~1e-6 of the row rms), while a
    result that went through bf16 (errors up to 2^-9 of |ref|) does not.
    """
    if rel_l2 is None:
        rel_l2 = 1e-5 if dtype == "float32" else 1e-3
    out = np.asarray(out_f32, dtype=np.float64)
    ref = np.asarray(ref_f32, dtype=np.float64)
    if out.shape != ref.shape:
        raise AssertionError(f"shape {out.shape} != {ref.shape}")
    ref_r = to_f32(from_f32(ref.astype(np.float32), dtype), dtype).astype(np.float64)
    num = np.linalg.norm((out - ref_r).ravel())
    den = np.linalg.norm(ref_r.ravel())
    rl2 = float(num / den) if den > 0 else float(num)
    if ref.ndim >= 1 and ref.size:
        rows = ref.reshape(-1, ref.shape[-1])
        rms = np.sqrt(np.mean(rows ** 2, axis=-1, keepdims=True))
        fl = 2.0 ** -4 if dtype == "float32" else 2.0 ** -8
        floor = np.broadcast_to(rms * fl, rows.shape).reshape(ref.shape)
    else:
        floor = np.zeros_like(ref)
    mag = np.maximum(np.abs(ref), floor)
    ulp = ulp_bf16(mag) if dtype == "bfloat16" else (ulp_f16(mag) if dtype == "float16"
                                                      else np.abs(mag) * 2.0 ** -12 + 1e-30)
    err_ulp = np.abs(out - ref) / ulp
    worst = float(err_ulp.max()) if err_ulp.size else 0.0
    ok = (rl2 <= rel_l2) and (worst <= max_ulp) and bool(np.all(np.isfinite(out)))
    return {"ok": ok, "rel_l2": rl2, "max_ulp": worst}
