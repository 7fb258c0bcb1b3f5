"""Module-level drop-in: MLX-format quantized layers as torch modules.

Torch counterparts of the layers the reference routes through its kernels:

* :class:`QuantizedLinear` - ``mlx.nn.QuantizedLinear`` (MLX-format ``weight``
  uint32 ``[N, K*bits/32]``, ``scales``/``biases`` ``[N, K/group_size]``,
  optional ``bias``), whose forward is ``quantized_matmul(x, w, s, b,
  transpose=True)`` plus ``bias``.
* :class:`QuantizedSwitchLinear` / :class:`SwitchGLU` - mlx-lm's expert banks
  ``[E, N, K*bits/32]`` applied per (token, expert) pair with ``gather_qmm``
  (reference call sites: mlxturbo/fused.py:2389-2394, 3105-3116;
  qwen4_exp.py:1795-1802), including the ``_gather_sort`` path that sorts
  pairs by expert and passes ``sorted_indices=True`` (fused.py:2402-2418).

Every forward runs the HIP kernels; there is no CPU path.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops


def _check_quantized(weight: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor], group_size: int, bits: int) -> int:
    if weight.dtype != torch.uint32 and weight.dtype != torch.int32:
        raise ValueError(f"weight must hold packed uint32 words, got {weight.dtype}")
    k = weight.shape[-1] * 32 // bits
    if scales.shape[-1] * group_size != k:
        raise ValueError(
            f"scales last dim {scales.shape[-1]} x group_size {group_size} != K={k}")
    if biases is not None and biases.shape != scales.shape:
        raise ValueError("biases must have the shape of scales")
    return k


class QuantizedLinear(torch.nn.Module):
    """``mlx.nn.QuantizedLinear`` on MLX-format tensors (affine mode).

    Parameters are registered as buffers under MLX's names (``weight``,
    ``scales``, ``biases``, ``bias``) so weights loaded from an MLX checkpoint
    keep their keys.
    """

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor,
                 biases: Optional[torch.Tensor], bias: Optional[torch.Tensor] = None,
                 group_size: int = 64, bits: int = 4, mode: str = "affine"):
        super().__init__()
        self.input_dims = _check_quantized(weight, scales, biases, group_size, bits)
        self.output_dims = weight.shape[0]
        self.group_size = group_size
        self.bits = bits
        self.mode = mode
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)

    def prepared_weights(self) -> Optional["ops.PreparedWeights"]:
        """The layer's weights validated once (:class:`ops.PreparedWeights`),
        rebuilt when a tensor is replaced or written in place; ``None`` for
        configurations the full operator handles (non-affine modes, weights
        off the GPU, missing biases)."""
        if self.mode != "affine" or self.weight.device.type != "cuda" or self.biases is None:
            return None
        p = self.__dict__.get("_mq_prepared")
        if p is None or not p.matches(self.weight, self.scales, self.biases, self.group_size,
                                      self.bits):
            p = ops.PreparedWeights(self.weight, self.scales, self.biases, self.group_size,
                                    self.bits, self.mode)
            self.__dict__["_mq_prepared"] = p
        return p

    def quantized_forward(self, x: torch.Tensor) -> torch.Tensor:
        p = self.prepared_weights()
        if p is None:
            # the full operator raises the reference's errors
            out = ops.quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                                       group_size=self.group_size, bits=self.bits,
                                       mode=self.mode)
        else:
            out = ops.quantized_matmul_prepared(x, p)
        if self.bias is not None:
            out = out + self.bias
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.quantized_forward(x)

    @classmethod
    def from_linear(cls, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                    group_size: int = 64, bits: int = 4) -> "QuantizedLinear":
        """Quantize a float weight ``[N, K]`` (``mlx.nn.QuantizedLinear.
        from_linear``): ``mx.quantize`` on the GPU; scales and biases keep
        the weight's dtype."""
        wq, s, b = ops.quantize(weight, group_size=group_size, bits=bits)
        return cls(wq, s, b, bias=bias, group_size=group_size, bits=bits)

    def dequantized_weight(self) -> torch.Tensor:
        """The layer's weight as ``mx.dequantize`` gives it, ``[N, K]``."""
        return ops.dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits,
                              self.mode)

    def extra_repr(self) -> str:
        return (f"input_dims={self.input_dims}, output_dims={self.output_dims}, "
                f"group_size={self.group_size}, bits={self.bits}, mode={self.mode!r}")


class QuantizedSwitchLinear(torch.nn.Module):
    """mlx-lm's ``QuantizedSwitchLinear``: an expert bank applied per index.

    ``forward(x, indices, sorted_indices=False)`` with ``x`` ``(..., M, K)``
    (mlx-lm expands tokens to ``(T, 1, 1, K)``) and ``indices`` ``(T, top_k)``
    returns ``(T, top_k, M, N)``.
    """

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor,
                 biases: Optional[torch.Tensor], bias: Optional[torch.Tensor] = None,
                 group_size: int = 64, bits: int = 4, mode: str = "affine"):
        super().__init__()
        if weight.ndim != 3:
            raise ValueError("an expert bank weight is [E, N, K*bits/32]")
        self.input_dims = _check_quantized(weight, scales, biases, group_size, bits)
        self.num_experts, self.output_dims = weight.shape[0], weight.shape[1]
        self.group_size = group_size
        self.bits = bits
        self.mode = mode
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        self.register_buffer("bias", bias)

    def forward(self, x: torch.Tensor, indices: torch.Tensor,
                sorted_indices: bool = False,
                tables: Optional[ops.GatherTables] = None) -> torch.Tensor:
        out = ops.gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices,
                             transpose=True, group_size=self.group_size, bits=self.bits,
                             mode=self.mode, sorted_indices=sorted_indices, tables=tables)
        if self.bias is not None:
            # bias [E, N] per expert, broadcast over the M rows of each pair
            out = out + self.bias[indices.long()].unsqueeze(-2)
        return out


class SwitchGLU(torch.nn.Module):
    """mlx-lm's ``SwitchGLU``: ``down(silu(gate(x)) * up(x))`` over the top-k
    experts of each token, with the ``_gather_sort`` reordering for long
    inputs (pairs sorted by expert once, then unsorted at the end, as
    mlx-lm does at 64+ indices: fused.py:2402-2418).

    At prefill widths (1024+ pairs) the layer runs as the reference's prefill
    path does (fused.py:3283-3316): the segment tables are built once for
    the routing and shared by the gate, up and down gathers; the gate and up
    gathers read x through the token of each pair (no gathered copy of x)
    and run with the SwiGLU as one launch (:func:`ops.gather_swiglu`); the
    router-weighted sum is one combine.  The
    pairs stay in (token, expert) order throughout (the grouped kernels
    group them by expert themselves), so no sort or unsort runs.  Each step
    computes what the sort path computes, bit for bit."""

    SORT_THRESHOLD = 64
    TABLES_THRESHOLD = 1024

    def __init__(self, gate_proj: QuantizedSwitchLinear, up_proj: QuantizedSwitchLinear,
                 down_proj: QuantizedSwitchLinear, fuse_gate_up: bool = False,
                 prefill_tables: bool = True):
        """``fuse_gate_up``: at decode widths (fewer than 1024 pairs) compute
        ``silu(gate) * up`` in one fused kernel (:func:`ops.gather_glu`, float
        sums, one rounding) with no expert sort -- the reference's opt-in
        ``moe_dec_fused`` route (fused.py:2456-2492).  Off by default, as in
        the reference, because it rounds differently from mlx-lm's SwiGLU."""
        super().__init__()
        self.gate_proj = gate_proj
        self.up_proj = up_proj
        self.down_proj = down_proj
        self.fuse_gate_up = fuse_gate_up
        self.prefill_tables = prefill_tables

    def _prefill(self, xe: torch.Tensor, idx: torch.Tensor,
                 scores: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        """The prefill layer over shared tables, or None where it does not
        apply (biases on the projections, other formats, no tables)."""
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        if not self.prefill_tables or idx.numel() < self.TABLES_THRESHOLD:
            return None
        if g.bias is not None or u.bias is not None or d.bias is not None:
            return None
        if xe.dtype not in (torch.bfloat16, torch.float16) or g.scales.dtype != xe.dtype:
            return None
        E = g.num_experts
        if u.num_experts != E or d.num_experts != E:
            return None
        # the gathers run the thin grouped kernel, which takes the tables,
        # below 96 rows per active expert and at K <= 2048 (the library's
        # gather_thin_path); elsewhere each gather builds its own
        P = idx.numel()
        if P >= 96 * min(P, E) or max(g.input_dims, u.input_dims, d.input_dims) > 2048:
            return None
        tables = ops.gather_tables(idx, E)
        if tables is None:
            return None
        if (g.weight.shape == u.weight.shape and g.scales.dtype == u.scales.dtype
                and (g.group_size, g.bits, g.mode) == (u.group_size, u.bits, u.mode)):
            # gate, up and the SwiGLU in one launch where the tables' kernel
            # takes it (each x tile read once for both banks)
            h = ops.gather_swiglu(xe, (g.weight, g.scales, g.biases),
                                  (u.weight, u.scales, u.biases), idx, tables,
                                  group_size=g.group_size, bits=g.bits, mode=g.mode)
        else:
            h = ops.swiglu(g(xe, idx, tables=tables), u(xe, idx, tables=tables))
        y = d(h, idx, tables=tables)                            # (T, k, 1, N)
        T, top_k = idx.shape
        if scores is not None:
            return ops.moe_combine(y.reshape(-1, y.shape[-1]), None, scores.reshape(-1), T, top_k)
        return y.reshape(T, top_k, y.shape[-1])

    def _fused(self, pairs: int) -> bool:
        g, u = self.gate_proj, self.up_proj
        return (self.fuse_gate_up and pairs < ops._GLU_FUSED_MAX_ROWS and g.bias is None
                and u.bias is None and g.weight.shape == u.weight.shape
                and (g.group_size, g.bits, g.mode) == (u.group_size, u.bits, u.mode))

    def _down_combine(self, h: torch.Tensor, idx: torch.Tensor,
                      scores: torch.Tensor) -> torch.Tensor:
        """Down projection of h (one row per pair, pairs in (token, k)
        order) and the router-weighted top-k sum: one kernel at decode widths
        (:func:`ops.gather_qmm_combine`), identical to the two passes."""
        d = self.down_proj
        return ops.gather_qmm_combine(h, d.weight, d.scales, d.biases, idx,
                                      scores.reshape(idx.shape), group_size=d.group_size,
                                      bits=d.bits, mode=d.mode)

    def forward(self, x: torch.Tensor, indices: torch.Tensor,
                scores: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x: (..., K), indices: (..., top_k) -> (..., top_k, K_out); with
        router ``scores`` (..., top_k) -> (..., K_out): the router-weighted
        sum over the top-k experts, folded into one combine pass over the
        down projection's (possibly expert-sorted) output (the reference's
        combine mode, kernels/moe_combine.py; fused.py:3283-3316)."""
        lead = x.shape[:-1]
        top_k = indices.shape[-1]
        xe = x.reshape(-1, 1, 1, x.shape[-1])                      # (T, 1, 1, K)
        idx = indices.reshape(-1, top_k)
        if self._fused(idx.numel()):
            g, u = self.gate_proj, self.up_proj
            d = self.down_proj
            if (idx.shape[0] <= ops._BLOCK_MAX_T and scores is not None and d.bias is None
                    and g.mode == "affine"
                    and (d.group_size, d.bits, d.mode) == (g.group_size, g.bits, g.mode)):
                # up to 8 tokens: the whole layer in one launch where it applies
                out = ops._layer_fused(x.reshape(idx.shape[0], -1), idx, scores,
                                     (g.weight, g.scales, g.biases),
                                     (u.weight, u.scales, u.biases),
                                     (d.weight, d.scales, d.biases), g.group_size, g.bits)
                if out is not None:
                    return out.reshape(*lead, out.shape[-1])
            h = ops.gather_glu(xe, g.weight, g.scales, g.biases, u.weight, u.scales, u.biases,
                               rhs_indices=idx, group_size=g.group_size, bits=g.bits,
                               mode=g.mode)                        # (T, k, 1, I)
            if scores is not None and self.down_proj.bias is None:
                out = self._down_combine(h, idx, scores)
                return out.reshape(*lead, out.shape[-1])
            y = self.down_proj(h, idx)                             # (T, k, 1, N)
            if scores is not None:
                out = ops.moe_combine(y.reshape(-1, y.shape[-1]), None, scores.reshape(-1),
                                      idx.shape[0], top_k)
                return out.reshape(*lead, y.shape[-1])
            return y.reshape(*lead, top_k, y.shape[-1])
        pre = self._prefill(xe, idx, scores)
        if pre is not None:
            return pre.reshape(*lead, *pre.shape[1:]) if scores is None else \
                pre.reshape(*lead, pre.shape[-1])
        do_sort = idx.numel() >= self.SORT_THRESHOLD
        if do_sort:
            flat = idx.reshape(-1)
            order = torch.argsort(flat, stable=True)
            inv = torch.argsort(order)
            xe = xe.reshape(-1, 1, x.shape[-1])[order // top_k].unsqueeze(-2)  # (P, 1, 1, K)
            idx_use = flat[order].reshape(-1, 1)
        else:
            idx_use = idx
        g = self.gate_proj(xe, idx_use, sorted_indices=do_sort)
        u = self.up_proj(xe, idx_use, sorted_indices=do_sort)
        # SwiGLU in T as MLX evaluates it: each op in float, rounded to T
        # (one kernel pass for bf16 / fp16)
        if g.dtype in (torch.bfloat16, torch.float16) and g.dtype == u.dtype:
            h = ops.swiglu(g, u)
        else:
            act = torch.nn.functional.silu(g.float()).to(g.dtype)
            h = (act.float() * u.float()).to(g.dtype)
        if scores is not None and not do_sort and self.down_proj.bias is None:
            out = self._down_combine(h, idx, scores)
            return out.reshape(*lead, out.shape[-1])
        y = self.down_proj(h, idx_use, sorted_indices=do_sort)  # (T or P, k, 1, N)
        if scores is not None:
            rows = idx.shape[0]
            out = ops.moe_combine(y.reshape(-1, y.shape[-1]), inv if do_sort else None,
                                  scores.reshape(-1), rows, top_k)
            return out.reshape(*lead, y.shape[-1])
        if do_sort:
            y = y.reshape(-1, y.shape[-1])[inv].reshape(*lead, top_k, y.shape[-1])
        else:
            y = y.reshape(*lead, top_k, y.shape[-1])
        return y


__all__ = ["QuantizedLinear", "QuantizedSwitchLinear", "SwitchGLU"]
