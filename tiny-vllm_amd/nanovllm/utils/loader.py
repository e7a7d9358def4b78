"""safetensors -> model parameters, with the quantized-artifact checks
(reference: nanovllm/utils/loader.py).

Every tensor is routed to its parameter's `weight_loader` hook (which does the
TP sharding); names of unpacked checkpoints (q_proj, k_proj, gate_proj, ...)
are mapped onto the packed parameters through the model's
`packed_modules_mapping`. After loading an "int8" or "w8a8" model, every
`*.qweight` and `*.scales` / `*.w_scales` parameter must have been loaded,
otherwise RuntimeError lists the missing ones (reference loader.py:27-41).
"""
from __future__ import annotations

import os
from glob import glob

import torch
from safetensors import safe_open
from torch import nn


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor):
    param.data.copy_(loaded_weight)


def _has_parameter(model: nn.Module, name: str) -> bool:
    try:
        model.get_parameter(name)
    except AttributeError:
        return False
    return True


def _load(model: nn.Module, name: str, tensor: torch.Tensor, loaded: set[str], *args) -> None:
    param = model.get_parameter(name)
    getattr(param, "weight_loader", default_weight_loader)(param, tensor, *args)
    loaded.add(name)


def _validate_quantized_loaded(model: nn.Module, loaded: set[str], scale_suffix: str, label: str) -> None:
    expected = {n for n, _ in model.named_parameters() if n.endswith(".qweight") or n.endswith(scale_suffix)}
    missing = sorted(expected - loaded)
    if missing:
        preview = ", ".join(missing[:8])
        if len(missing) > 8:
            preview += f", ... ({len(missing)} missing total)"
        raise RuntimeError(f"Missing {label} quantized tensors. Expected qweight/{scale_suffix[1:]} for quantized "
                           f"linear layers, but did not load: {preview}")


def load_model(model: nn.Module, path: str, quantization: str | None = None) -> None:
    mapping = getattr(model, "packed_modules_mapping", {})
    loaded: set[str] = set()
    files = glob(os.path.join(path, "*.safetensors"))
    if not files:
        raise FileNotFoundError(f"No safetensors files found in {path}")
    for file in files:
        with safe_open(file, "pt", "cpu") as f:
            for name in f.keys():
                tensor = f.get_tensor(name)
                if _has_parameter(model, name):
                    _load(model, name, tensor, loaded)
                    continue
                for key, (packed, shard_id) in mapping.items():
                    if key in name:
                        _load(model, name.replace(key, packed), tensor, loaded, shard_id)
                        break
                else:
                    _load(model, name, tensor, loaded)
    if quantization == "int8":
        _validate_quantized_loaded(model, loaded, ".scales", "INT8")
    elif quantization == "w8a8":
        _validate_quantized_loaded(model, loaded, ".w_scales", "W8A8")
    # derived weight copies (the MLP's regrouped gate_up for the fused
    # SiLU-and-mul GEMM) are rebuilt from the new weights on next use
    for mod in model.modules():
        if hasattr(mod, "_glu_weights"):
            del mod._glu_weights
