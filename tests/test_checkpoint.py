"""MLX checkpoint reading (mlxturbo_amd.checkpoint): config quantization with
per-module overrides, sharded safetensors, mixed bit widths, expert banks.
The checkpoint is synthetic, written with safetensors in MLX's layout."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from mlxturbo_amd import checkpoint
from mlxturbo_amd.nn import QuantizedLinear, QuantizedSwitchLinear
from oracle import oracle as O
from qmm_helpers import act, from_dev, quantized, to_dev


def _qt(rng, N, K, gs=64, bits=4, E=None):
    if E:
        parts = [quantized(rng, N, K, gs=gs, bits=bits) for _ in range(E)]
        w, s, b = (np.stack([p[i] for p in parts]) for i in range(3))
    else:
        w, s, b = quantized(rng, N, K, gs=gs, bits=bits)
    return (torch.from_numpy(w.view(np.int32)).view(torch.uint32),
            torch.from_numpy(s.view(np.int16)).view(torch.bfloat16),
            torch.from_numpy(b.view(np.int16)).view(torch.bfloat16), (w, s, b))


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    rng = np.random.default_rng(9)
    d = str(tmp_path_factory.mktemp("mlx_ckpt"))
    layers = {
        "model.layers.0.mlp.gate_proj": (64, 256, 64, 4, None),
        "model.layers.0.mlp.switch_mlp.up_proj": (32, 128, 64, 4, 4),
        "lm_head": (48, 256, 64, 8, None),                       # override in config
        "model.layers.1.self_attn.q_proj": (40, 128, 64, 8, None),  # width inferred
        "model.layers.1.self_attn.k_proj": (40, 128, 32, 4, None),  # override gs 32
        "model.layers.1.mlp.gate": (16, 128, 64, 4, None),          # override false
    }
    tensors, raw = {}, {}
    for name, (N, K, gs, bits, E) in layers.items():
        w, s, b, r = _qt(rng, N, K, gs, bits, E)
        tensors[name + ".weight"], tensors[name + ".scales"], tensors[name + ".biases"] = w, s, b
        raw[name] = r
    tensors["lm_head.bias"] = torch.arange(48, dtype=torch.float32).to(torch.bfloat16)
    tensors["model.embed_tokens.weight"] = torch.zeros(10, 8, dtype=torch.bfloat16)
    names = sorted(tensors)
    shards = [names[: len(names) // 2], names[len(names) // 2:]]
    wmap = {}
    for i, keys in enumerate(shards):
        fname = f"model-{i + 1:05d}-of-00002.safetensors"
        save_file({k: tensors[k].contiguous() for k in keys}, os.path.join(d, fname),
                  metadata={"format": "mlx"})
        wmap.update({k: fname for k in keys})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    config = {"model_type": "synthetic", "quantization": {
        "group_size": 64, "bits": 4, "mode": "affine",
        "lm_head": {"group_size": 64, "bits": 8},
        "model.layers.1.self_attn.k_proj": {"group_size": 32, "bits": 4},
        "model.layers.1.mlp.gate": False}}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(config, f)
    return d, tensors, raw


def test_weight_map_and_tensors(ckpt):
    d, tensors, _ = ckpt
    wmap = checkpoint.weight_map(d)
    assert set(wmap) == set(tensors)
    got = checkpoint.load_tensors(d, ["lm_head.weight", "lm_head.bias"], device="cpu")
    assert torch.equal(got["lm_head.weight"], tensors["lm_head.weight"])
    assert got["lm_head.weight"].dtype == torch.uint32
    with pytest.raises(KeyError):
        checkpoint.load_tensors(d, ["nope.weight"], device="cpu")


def test_quantized_layers_formats(ckpt):
    d, tensors, _ = ckpt
    layers = checkpoint.quantized_layers(d, device="cpu")
    assert set(layers) == {"model.layers.0.mlp.gate_proj", "model.layers.0.mlp.switch_mlp.up_proj",
                           "lm_head", "model.layers.1.self_attn.q_proj",
                           "model.layers.1.self_attn.k_proj"}
    g = layers["model.layers.0.mlp.gate_proj"]
    assert type(g) is QuantizedLinear and (g.bits, g.group_size) == (4, 64)
    assert (g.input_dims, g.output_dims) == (256, 64)
    sw = layers["model.layers.0.mlp.switch_mlp.up_proj"]
    assert type(sw) is QuantizedSwitchLinear and sw.num_experts == 4
    head = layers["lm_head"]
    assert (head.bits, head.group_size) == (8, 64) and head.bias is not None
    assert torch.equal(head.weight, tensors["lm_head.weight"])
    assert layers["model.layers.1.self_attn.q_proj"].bits == 8       # inferred from shapes
    assert layers["model.layers.1.self_attn.k_proj"].group_size == 32


def test_quant_params_rules():
    cfg = {"quantization": {"group_size": 64, "bits": 4, "x": False, "y": {"bits": 8}}}
    assert checkpoint.quant_params(cfg, "x", 32, 4) is None
    assert checkpoint.quant_params(cfg, "y", 64, 4) == (64, 8, "affine")
    assert checkpoint.quant_params(cfg, "z", 32, 4) == (64, 4, "affine")
    assert checkpoint.quant_params(cfg, "z", 48, 4) == (64, 6, "affine")   # inferred
    assert checkpoint.quant_params(cfg, "z", 64, 4) == (64, 8, "affine")
    with pytest.raises(ValueError):
        checkpoint.quant_params(cfg, "z", 33, 4)
    assert checkpoint.quant_params({}, "z", 32, 4) is None


@pytest.mark.gpu
def test_loaded_layers_run(ckpt):
    d, _, raw = ckpt
    layers = checkpoint.quantized_layers(d)
    rng = np.random.default_rng(10)
    x = act(rng, (3, 256))
    head = layers["lm_head"]
    out = head(to_dev(x, "bfloat16"))
    w, s, b = raw["lm_head"]
    ref = O.quantized_matmul_ref(x, w, s, b, 64, 8) + np.arange(48, dtype=np.float32)
    res = O.check_output(from_dev(out), ref)
    assert res["ok"], res
