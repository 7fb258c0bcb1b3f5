"""Shape-by-M routing of quantized linear layers (the reference's dispatch).

Mirrors mlxturbo/kernels/dispatch.py on torch modules:

* :data:`DEFAULT_ROUTE_TABLE`, :func:`select_route` (dispatch.py:59-68,
  102-117): per ``(K, N)`` geometry, an M-indexed row of routes for the
  flattened width M = prod(x.shape[:-1]); unknown shapes and widths outside
  the row take ``stock``.
* :func:`quantized_matmul` (dispatch.py:302-382): flatten, route, restore the
  shape; non-affine modes, missing biases or non-2-D weights take ``stock``.
* :class:`DispatchedQuantizedLinear`, :func:`enable`, :func:`dispatch_scope`
  (dispatch.py:385-466): per-instance class swap (module identity, buffer
  names and loaded tensors are kept); ``enable(active=False)`` installs
  routing that is live only inside ``dispatch_scope()``.
* :func:`enable_class` / :func:`disable_class`: the class-level patch of
  ``fast_qmm.enable/disable`` (fast_qmm.py:395-472), reversible.

On MI355X every route is a HIP kernel of this library: ``stock`` is
:func:`mlxturbo_amd.quantized_matmul` with the library's own width choice
(the one-row quad kernel, the skinny streaming kernel for 2..32 rows, and
above that 32- or 16-row skinny launches or the MFMA tile kernel, whichever
the library's per-geometry cost model prices lower); ``skinny`` and
``wide`` name the two families.  At K=5120, N=17408 one skinny launch of
16 rows costs ~21 us and of 32 rows ~23 us, while the MFMA tile kernel does
96 rows in ~53 us and 512 rows in ~112 us.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from math import prod
from typing import Any, Optional

import torch

from . import ops
from .nn import QuantizedLinear

STOCK = "stock"
SKINNY = "skinny"
WIDE = "wide"
_ROUTES = frozenset((STOCK, SKINNY, WIDE))
SKINNY_MAX_M = 16


def _row() -> tuple[str, ...]:
    """M-indexed row for M = 0..16: the skinny kernel at every verify width."""
    return tuple([STOCK] + [SKINNY] * SKINNY_MAX_M)


# The reference's measured production geometries (dispatch.py:59-68).  Its
# rows choose among Metal kernels per M; here the per-geometry choice is the
# library's own cost model (csrc/launch.h wide_route / wide_plan: skinny
# launch time 3 us + weight bytes at 3.6 TB/s times a factor per row count,
# wide tile time per round of workgroups, each constant measured on MI355X),
# which every call consults, so the default rows only name the streaming
# kernels at M = 1..16 (what the model picks there on every geometry) and a
# row is where a caller forces 16-row launches above 16 rows ("skinny").
DEFAULT_ROUTE_TABLE: dict[tuple[int, int], tuple[str, ...]] = {
    (5120, 17408): _row(),     # MLP up/gate
    (17408, 5120): _row(),     # MLP down
    (5120, 12288): _row(),     # attention q
    (5120, 248320): _row(),    # lm_head
    (21504, 5376): _row(),
}

_DISPATCH_ACTIVE = ContextVar("mlxturbo_amd_dispatch_active", default=False)


def select_route(k: int, n: int, m: int,
                 table: Optional[dict[tuple[int, int], tuple[str, ...]]] = None) -> str:
    """Return ``stock``, ``skinny`` or ``wide`` for one flattened matmul."""
    route_table = DEFAULT_ROUTE_TABLE if table is None else table
    row = route_table.get((k, n))
    if row is None or m < 0:
        return STOCK
    if m >= len(row):
        return WIDE if m > SKINNY_MAX_M else STOCK
    route = row[m]
    if route not in _ROUTES:
        raise ValueError(f"invalid quantized-matmul route {route!r}")
    return route


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: Optional[torch.Tensor], *, group_size: int, bits: int,
                     mode: str = "affine",
                     table: Optional[dict[tuple[int, int], tuple[str, ...]]] = None,
                     prepared: Optional[ops.PreparedWeights] = None) -> torch.Tensor:
    """Dispatch a QuantizedLinear matmul by ``(K, N, M)``.

    ``skinny`` runs the streaming kernel in launches of up to 16 rows even for
    wider inputs (a route-table override); ``wide`` and ``stock`` defer to
    the library's width choice.  ``prepared`` (the layer's validated weights)
    skips re-validating them on every call.
    """
    def stock():
        if prepared is not None:
            return ops.quantized_matmul_prepared(x, prepared)
        return ops.quantized_matmul(x, w, scales, biases, transpose=True,
                                    group_size=group_size, bits=bits, mode=mode)

    if mode != "affine" or biases is None or x.ndim < 2 or w.ndim != 2:
        return stock()
    k = x.shape[-1]
    n = w.shape[0]
    m = prod(x.shape[:-1])
    route = select_route(k, n, m, table)
    if route != SKINNY or m <= SKINNY_MAX_M:
        return stock()
    flat = x.reshape(m, k)
    parts = [ops.quantized_matmul(flat[i:i + SKINNY_MAX_M], w, scales, biases, transpose=True,
                                  group_size=group_size, bits=bits, mode=mode)
             for i in range(0, m, SKINNY_MAX_M)]
    return torch.cat(parts, 0).reshape(*x.shape[:-1], n)


class DispatchedQuantizedLinear(QuantizedLinear):
    """QuantizedLinear with shape-by-M routing, live when enabled as always
    active or inside :func:`dispatch_scope`; otherwise the base forward."""

    _mq_dispatch_always = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        active = self._mq_dispatch_always or _DISPATCH_ACTIVE.get()
        if not active:
            return super().forward(x)
        out = quantized_matmul(x, self.weight, self.scales, self.biases,
                               group_size=self.group_size, bits=self.bits, mode=self.mode,
                               prepared=self.prepared_weights())
        if self.bias is not None:
            out = out + self.bias
        return out


@contextmanager
def dispatch_scope():
    """Temporarily activate layers enabled with ``active=False``."""
    token = _DISPATCH_ACTIVE.set(True)
    try:
        yield
    finally:
        _DISPATCH_ACTIVE.reset(token)


def enable(model: Any, *, active: bool = True):
    """Swap every :class:`QuantizedLinear` below ``model`` to the dispatched
    class in place (``__class__`` only; identity and buffers are kept).
    Idempotent; ``active=False`` routes only inside :func:`dispatch_scope`."""
    for _, module in model.named_modules():
        if isinstance(module, QuantizedLinear) and not isinstance(module,
                                                                  DispatchedQuantizedLinear):
            module.__class__ = DispatchedQuantizedLinear
        if isinstance(module, DispatchedQuantizedLinear):
            module._mq_dispatch_always = active
    return model


def disable(model: Any):
    """Undo :func:`enable` below ``model``."""
    for _, module in model.named_modules():
        if isinstance(module, DispatchedQuantizedLinear):
            module.__class__ = QuantizedLinear
            module.__dict__.pop("_mq_dispatch_always", None)
    return model


_ORIGINAL_FORWARD = None


def enable_class() -> None:
    """Route every :class:`QuantizedLinear` (existing and future instances)
    through :func:`quantized_matmul`'s table, by patching the class."""
    global _ORIGINAL_FORWARD
    if _ORIGINAL_FORWARD is not None:
        return
    _ORIGINAL_FORWARD = QuantizedLinear.forward

    def forward(self, x):
        out = quantized_matmul(x, self.weight, self.scales, self.biases,
                               group_size=self.group_size, bits=self.bits, mode=self.mode,
                               prepared=self.prepared_weights())
        if self.bias is not None:
            out = out + self.bias
        return out

    QuantizedLinear.forward = forward


def disable_class() -> None:
    global _ORIGINAL_FORWARD
    if _ORIGINAL_FORWARD is not None:
        QuantizedLinear.forward = _ORIGINAL_FORWARD
        _ORIGINAL_FORWARD = None


__all__ = ["DEFAULT_ROUTE_TABLE", "DispatchedQuantizedLinear", "SKINNY", "STOCK", "WIDE",
           "disable", "disable_class", "dispatch_scope", "enable", "enable_class",
           "quantized_matmul", "select_route"]
