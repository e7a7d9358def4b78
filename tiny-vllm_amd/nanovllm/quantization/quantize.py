"""Offline quantizer: Hugging Face Qwen3 safetensors -> tiny-vLLM INT8 / W8A8
artifact (reference: scripts/quantize.py).

    python -m nanovllm.quantization.quantize --model SRC --output DST \\
        [--quantization int8|w8a8] [--overwrite]

Artifact layout (unchanged from the reference, so either loader reads it):
  * q/k/v weights of a layer are concatenated along dim 0 (q, k, v order) and
    quantized per output channel -> `<layer>.self_attn.qkv_proj.qweight` int8
    [N, K] and `.scales` (int8) or `.w_scales` (w8a8) fp32 [N];
  * gate/up likewise -> `<layer>.mlp.gate_up_proj.*` (gate, up order);
  * o_proj / down_proj are quantized in place;
  * q/k/v and gate/up biases, if present, are concatenated the same way;
  * every other tensor is copied unchanged, into one `model.safetensors`;
  * every non-safetensors file of SRC (config, tokenizer, ...) is copied.
A layer with only some of its q/k/v or gate/up shards is an error.
"""
from __future__ import annotations

import argparse
import shutil
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from nanovllm.quantization.utils import quantize_int8_per_channel

QKV = ("q", "k", "v")
GATE_UP = ("gate", "up")
# suffix -> (group, shard id, is_bias)
_GROUPED = {
    **{f"{s}_proj.weight": ("qkv", s, False) for s in QKV},
    **{f"{s}_proj.bias": ("qkv", s, True) for s in QKV},
    **{f"{s}_proj.weight": ("gate_up", s, False) for s in GATE_UP},
    **{f"{s}_proj.bias": ("gate_up", s, True) for s in GATE_UP},
}
_DIRECT = ("o_proj.weight", "down_proj.weight")
_ORDER = {"qkv": QKV, "gate_up": GATE_UP}


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description="Quantize Qwen3 linear weights to INT8 (W8A16) or W8A8 formats.")
    ap.add_argument("--model", required=True, type=Path, help="Source Hugging Face model directory")
    ap.add_argument("--output", required=True, type=Path, help="Output quantized model directory")
    ap.add_argument("--quantization", default="int8", choices=["int8", "w8a8"], help="Format to generate")
    ap.add_argument("--overwrite", action="store_true", help="Remove an existing output directory first")
    return ap.parse_args(argv)


def copy_model_files(model_dir: Path, output_dir: Path) -> None:
    for src in model_dir.iterdir():
        dst = output_dir / src.name
        if src.is_file():
            if src.suffix == ".safetensors" or src.name.endswith(".safetensors.index.json"):
                continue
            shutil.copy2(src, dst)
        elif src.is_dir():
            shutil.copytree(src, dst, ignore=shutil.ignore_patterns("*.safetensors"), dirs_exist_ok=True)


def load_tensors(model_dir: Path) -> dict[str, torch.Tensor]:
    tensors: dict[str, torch.Tensor] = {}
    files = sorted(model_dir.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"No safetensors files found in {model_dir}")
    for file in files:
        with safe_open(file, "pt", "cpu") as f:
            for name in f.keys():
                if name in tensors:
                    raise ValueError(f"Duplicate tensor name across safetensors files: {name}")
                tensors[name] = f.get_tensor(name)
    return tensors


def _put_quantized(out: dict[str, torch.Tensor], prefix: str, weight: torch.Tensor, quantization: str) -> None:
    q, s = quantize_int8_per_channel(weight)
    out[f"{prefix}.qweight"] = q.contiguous()
    out[f"{prefix}.{'w_scales' if quantization == 'w8a8' else 'scales'}"] = s.contiguous()


def build_quantized_tensors(tensors: dict[str, torch.Tensor], quantization: str) -> dict[str, torch.Tensor]:
    out: dict[str, torch.Tensor] = {}
    # (group, is_bias) -> {layer prefix -> {shard id -> tensor}}
    groups: dict[tuple[str, bool], dict[str, dict[str, torch.Tensor]]] = {}
    for name, tensor in tensors.items():
        for suffix, (group, shard, is_bias) in _GROUPED.items():
            if name.endswith(suffix):
                groups.setdefault((group, is_bias), {}).setdefault(name[: -len(suffix)], {})[shard] = tensor
                break
        else:
            if name.endswith(_DIRECT):
                _put_quantized(out, name[: -len(".weight")], tensor, quantization)
            else:
                out[name] = tensor.contiguous()
    for (group, is_bias), layers in groups.items():
        order = _ORDER[group]
        for prefix, shards in layers.items():
            missing = [s for s in order if s not in shards]
            if missing:
                kind = f"{'qkv' if group == 'qkv' else 'gate/up'} {'bias' if is_bias else 'weight'}"
                raise ValueError(f"Missing {kind} shards for {prefix}: {missing}")
            packed = torch.cat([shards[s] for s in order], dim=0)
            name = f"{prefix}{group}_proj"
            if is_bias:
                out[f"{name}.bias"] = packed.contiguous()
            else:
                _put_quantized(out, name, packed, quantization)
    return out


def main(argv=None) -> None:
    args = parse_args(argv)
    if not args.model.is_dir():
        raise NotADirectoryError(args.model)
    if args.output.exists() and args.overwrite:
        shutil.rmtree(args.output)
    args.output.mkdir(parents=True, exist_ok=True)
    copy_model_files(args.model, args.output)
    quantized = build_quantized_tensors(load_tensors(args.model), args.quantization)
    save_file(quantized, args.output / "model.safetensors")
    print(f"Wrote {args.quantization.upper()} quantized model to {args.output}")


if __name__ == "__main__":
    main()
