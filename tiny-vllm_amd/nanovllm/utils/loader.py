"""Checkpoint and quantized-artifact loading into the model's parameters.

What it must do (the artifact contract of nanovllm/utils/loader.py:27-68 and
scripts/quantize.py): every tensor of every `*.safetensors` file in the
directory goes to the `weight_loader` hook of its parameter, which does the
tensor-parallel sharding. Unpacked checkpoint names (q_proj, k_proj, v_proj,
gate_proj, up_proj) land in the packed parameter named by the model's
`packed_modules_mapping`, with the shard id as the loader's extra argument.
After an "int8" / "w8a8" load every `*.qweight` and `*.scales` /
`*.w_scales` parameter must have been written, otherwise a RuntimeError
names the missing ones (same message as the reference, since tooling may
match on it).

How: the name -> (parameter, loader args) resolution is computed once per
model into a table (`_ParamIndex`), tensors are streamed file by file, and
the bookkeeping of what was written is a set of parameter names checked at
the end against the quantization mode's required suffixes.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from glob import glob

import torch
from safetensors import safe_open
from torch import nn

# quantization mode -> (label used in the error, required scale suffix)
_REQUIRED = {"int8": ("INT8", "scales"), "w8a8": ("W8A8", "w_scales")}


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor):
    """Loader of parameters without a hook: plain copy."""
    param.data.copy_(loaded_weight)


@dataclass(frozen=True)
class _Target:
    name: str
    param: nn.Parameter
    args: tuple


class _ParamIndex:
    """Resolves checkpoint tensor names to model parameters."""

    def __init__(self, model: nn.Module):
        self.params = dict(model.named_parameters())
        # longest source keys first, so e.g. "up_proj" never shadows a longer
        # key that contains it
        mapping = getattr(model, "packed_modules_mapping", {})
        self.packed = sorted(mapping.items(), key=lambda kv: -len(kv[0]))

    def resolve(self, tensor_name: str) -> _Target:
        if tensor_name in self.params:
            return _Target(tensor_name, self.params[tensor_name], ())
        for src, (dst, shard_id) in self.packed:
            if src in tensor_name:
                name = tensor_name.replace(src, dst)
                return _Target(name, self._param(name, tensor_name), (shard_id,))
        return _Target(tensor_name, self._param(tensor_name, tensor_name), ())

    def _param(self, name: str, tensor_name: str) -> nn.Parameter:
        try:
            return self.params[name]
        except KeyError:
            raise AttributeError(f"checkpoint tensor {tensor_name!r} has no parameter {name!r} in the model") from None

    def required(self, scale_suffix: str) -> set[str]:
        return {n for n in self.params if n.endswith(".qweight") or n.endswith("." + scale_suffix)}


def _missing_error(label: str, scale_suffix: str, missing: list[str]) -> RuntimeError:
    shown = ", ".join(missing[:8])
    if len(missing) > 8:
        shown += f", ... ({len(missing)} missing total)"
    return RuntimeError(f"Missing {label} quantized tensors. Expected qweight/{scale_suffix} for quantized "
                        f"linear layers, but did not load: {shown}")


def load_model(model: nn.Module, path: str, quantization: str | None = None) -> None:
    files = sorted(glob(os.path.join(path, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"No safetensors files found in {path}")
    index = _ParamIndex(model)
    written: set[str] = set()
    for file in files:
        with safe_open(file, "pt", "cpu") as f:
            for tensor_name in f.keys():
                target = index.resolve(tensor_name)
                loader = getattr(target.param, "weight_loader", default_weight_loader)
                loader(target.param, f.get_tensor(tensor_name), *target.args)
                written.add(target.name)
    if quantization in _REQUIRED:
        label, suffix = _REQUIRED[quantization]
        missing = sorted(index.required(suffix) - written)
        if missing:
            raise _missing_error(label, suffix, missing)
