"""Re-quantize loaded layers to another bit width / group size in place.

Mirrors mlxturbo/rebit.py: ``_requantize`` (rebit.py:96-120) dequantizes a
quantized linear (or takes a float one) and quantizes it again with
``mx.quantize``; ``parse`` reads the ``"class=bits[:group]"`` spec
(rebit.py:123-137); ``apply`` walks a model and replaces the layers of each
class (rebit.py:140-166).  Here the layers are this package's torch
:class:`~mlxturbo_amd.nn.QuantizedLinear` modules and both steps are this
library's HIP kernels (bit-exact dequantize, then quantize).

The reference finds a class's layers by attribute walks over its own model
(``model.model.layers[i].linear_attn.in_proj_qkv`` ...); ``apply`` takes the
same class names and matches them against module paths with the patterns in
:data:`CLASS_PATTERNS` (mlx-lm's module names), or a caller's own table.
"""

from __future__ import annotations

import fnmatch
from typing import Dict, Iterable, Optional, Tuple

import torch

from .nn import QuantizedLinear

CLASSES = ("gdn", "hc", "attn", "head", "router", "shared")

# module-path patterns of each class (the attribute walks of rebit.py:60-93)
CLASS_PATTERNS: Dict[str, Tuple[str, ...]] = {
    "gdn": tuple(f"*.linear_attn.{a}" for a in ("in_proj_qkv", "in_proj_z", "in_proj_b",
                                                 "in_proj_a", "out_proj")),
    "hc": tuple(f"*.{h}.{a}" for h in ("attn_hyper_connection", "mlp_hyper_connection")
                for a in ("input_mix_weight_down", "input_mix_weight_up", "block_inject_weight")),
    "attn": tuple(f"*.self_attn.{a}" for a in ("q_proj", "k_proj", "v_proj", "o_proj")),
    "head": ("lm_head",),
    "router": ("*.mlp.gate",),
    "shared": tuple(f"*.mlp.shared_expert.{a}" for a in ("gate_proj", "up_proj", "down_proj"))
    + ("*.mlp.shared_expert_gate",),
}


def requantize(layer, bits: int, group_size: int = 64) -> QuantizedLinear:
    """A new :class:`QuantizedLinear` holding ``layer``'s weight at ``bits`` /
    ``group_size``: a quantized layer is dequantized first (double
    quantization, as rebit.py:96-120 does); a ``torch.nn.Linear`` or any
    module with a float ``weight`` is quantized directly.  ``bias`` is kept."""
    if isinstance(layer, QuantizedLinear):
        w = layer.dequantized_weight()
    else:
        w = layer.weight.detach()
    if w.shape[-1] % group_size:
        raise ValueError(f"in_dims={w.shape[-1]} is not a multiple of group_size={group_size}")
    bias = getattr(layer, "bias", None)
    new = QuantizedLinear.from_linear(w, bias=None if bias is None else bias.detach(),
                                      group_size=group_size, bits=bits)
    del w
    return new


def parse(spec: str) -> Dict[str, Tuple[int, int]]:
    """``"gdn=4,hc=4:32"`` -> ``{"gdn": (4, 64), "hc": (4, 32)}``."""
    out: Dict[str, Tuple[int, int]] = {}
    for part in spec.split(","):
        part = part.strip()
        if not part:
            continue
        cls, _, rhs = part.partition("=")
        bits, _, gs = rhs.partition(":")
        if cls not in CLASSES:
            raise ValueError(f"unknown class {cls!r} (known: {CLASSES})")
        out[cls] = (int(bits), int(gs) if gs else 64)
    return out


def _targets(model: torch.nn.Module, patterns: Iterable[str]):
    pats = tuple(patterns)
    for name, module in list(model.named_modules()):
        if not name:
            continue
        if not (isinstance(module, (QuantizedLinear, torch.nn.Linear))):
            continue
        if any(fnmatch.fnmatchcase(name, p) or fnmatch.fnmatchcase("." + name, p)
               for p in pats):
            parent_name, _, attr = name.rpartition(".")
            parent = model.get_submodule(parent_name) if parent_name else model
            yield parent, attr, module


def apply(model: torch.nn.Module, spec: str, patterns: Optional[Dict[str, Iterable[str]]] = None,
          verbose: bool = False) -> Dict[str, int]:
    """Re-quantize every layer of each class in ``spec`` in place; layers
    already at the requested width and group size are left alone.  Returns
    the number of layers replaced per class."""
    table = CLASS_PATTERNS if patterns is None else patterns
    counts: Dict[str, int] = {}
    for cls, (bits, gs) in parse(spec).items():
        n = 0
        for parent, attr, lin in list(_targets(model, table.get(cls, ()))):
            if isinstance(lin, QuantizedLinear) and lin.bits == bits and lin.group_size == gs:
                continue
            setattr(parent, attr, requantize(lin, bits, gs))
            n += 1
        counts[cls] = n
        if verbose:
            print(f"  rebit {cls}: {n} layers to {bits}bit/gs{gs}", flush=True)
    return counts


__all__ = ["CLASSES", "CLASS_PATTERNS", "apply", "parse", "requantize"]
