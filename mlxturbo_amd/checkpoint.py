"""Read MLX-format quantized checkpoints into the torch layers of this package.

An MLX checkpoint directory (as written by mlx-lm / the reference's
``convert.save_with_mtp``, convert.py:178-240) holds ``config.json`` and
safetensors shards (``model.safetensors``, or ``model-0000i-of-0000n.
safetensors`` with ``model.safetensors.index.json``'s ``weight_map``).  A
quantized linear ``<prefix>`` is the tensors ``<prefix>.weight`` (uint32
``[N, K*bits/32]``, or ``[E, N, K*bits/32]`` for an expert bank),
``<prefix>.scales`` / ``<prefix>.biases`` (``[N, K/group_size]``) and an
optional ``<prefix>.bias``.

``config["quantization"]`` gives the default ``group_size`` / ``bits`` /
``mode`` and, keyed by module path, per-module overrides (a dict, or ``false``
for a module left unquantized) -- how mixed-bit checkpoints record e.g. an
8-bit lm_head over a 4-bit body (KERNEL-INTEL.md:46-51 of the reference;
rebit.py re-quantizes such classes in place).  A module with no entry whose
tensor shapes disagree with the default bit width has its width inferred
from the shapes (``weight_cols * 32 / (scales_cols * group_size)``).

Tensors are memory-mapped from the shards and copied to the device once;
nothing is converted or repacked.
"""

from __future__ import annotations

import json
import os
from typing import Dict, Iterable, Optional, Tuple, Union

import torch
from safetensors import safe_open

from .nn import QuantizedLinear, QuantizedSwitchLinear

_BITS = (2, 3, 4, 5, 6, 8)


def read_config(path: str) -> dict:
    with open(os.path.join(path, "config.json")) as f:
        return json.load(f)


def weight_map(path: str) -> Dict[str, str]:
    """Tensor name -> shard file name."""
    index = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            return dict(json.load(f)["weight_map"])
    single = os.path.join(path, "model.safetensors")
    if not os.path.exists(single):
        raise FileNotFoundError(f"no model.safetensors or index in {path}")
    with safe_open(single, framework="pt") as f:
        return {k: "model.safetensors" for k in f.keys()}


def load_tensors(path: str, names: Optional[Iterable[str]] = None,
                 device: Union[str, torch.device] = "cuda") -> Dict[str, torch.Tensor]:
    """Load ``names`` (default: every tensor) from the shards onto ``device``."""
    wmap = weight_map(path)
    wanted = list(wmap) if names is None else list(names)
    missing = [n for n in wanted if n not in wmap]
    if missing:
        raise KeyError(f"tensors not in the checkpoint: {missing[:5]}")
    by_shard: Dict[str, list] = {}
    for n in wanted:
        by_shard.setdefault(wmap[n], []).append(n)
    out = {}
    for shard, keys in by_shard.items():
        with safe_open(os.path.join(path, shard), framework="pt") as f:
            for k in keys:
                out[k] = f.get_tensor(k).to(device)
    return out


def quant_params(config: dict, prefix: str, weight_cols: int,
                 scales_cols: int) -> Optional[Tuple[int, int, str]]:
    """(group_size, bits, mode) of module ``prefix``, or None if the
    checkpoint leaves it unquantized."""
    q = config.get("quantization") or config.get("quantization_config")
    if not q:
        return None
    override = q.get(prefix)
    if override is False:
        return None
    gs = int(q.get("group_size", 64))
    bits = int(q.get("bits", 4))
    mode = q.get("mode", "affine")
    if isinstance(override, dict):
        gs = int(override.get("group_size", gs))
        bits = int(override.get("bits", bits))
        mode = override.get("mode", mode)
    elif weight_cols * 32 != scales_cols * gs * bits:
        # no entry: infer the width from the shapes (mixed-bit checkpoints)
        num = weight_cols * 32
        den = scales_cols * gs
        if den == 0 or num % den or num // den not in _BITS:
            raise ValueError(f"{prefix}: weight cols {weight_cols} and scales cols "
                             f"{scales_cols} fit no bit width at group_size {gs}")
        bits = num // den
    return gs, bits, mode


def quantized_layers(path: str, device: Union[str, torch.device] = "cuda",
                     prefixes: Optional[Iterable[str]] = None
                     ) -> Dict[str, Union[QuantizedLinear, QuantizedSwitchLinear]]:
    """Every quantized linear of the checkpoint (or those in ``prefixes``) as
    a :class:`QuantizedLinear` (2-D weight) or :class:`QuantizedSwitchLinear`
    (3-D expert bank), keyed by module path."""
    config = read_config(path)
    wmap = weight_map(path)
    if prefixes is None:
        prefixes = sorted(k[: -len(".scales")] for k in wmap if k.endswith(".scales")
                          and k[: -len(".scales")] + ".weight" in wmap)
    layers = {}
    for prefix in prefixes:
        names = [prefix + ".weight", prefix + ".scales"]
        for opt in (".biases", ".bias"):
            if prefix + opt in wmap:
                names.append(prefix + opt)
        t = load_tensors(path, names, device)
        w, s = t[prefix + ".weight"], t[prefix + ".scales"]
        qp = quant_params(config, prefix, w.shape[-1], s.shape[-1])
        if qp is None:
            continue
        gs, bits, mode = qp
        if w.dtype != torch.uint32:
            w = w.view(torch.uint32) if w.dtype == torch.int32 else w
        cls = QuantizedSwitchLinear if w.ndim == 3 else QuantizedLinear
        layers[prefix] = cls(w, s, t.get(prefix + ".biases"), t.get(prefix + ".bias"),
                             group_size=gs, bits=bits, mode=mode)
    return layers


__all__ = ["load_tensors", "quant_params", "quantized_layers", "read_config", "weight_map"]
