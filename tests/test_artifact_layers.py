"""CPU tests of the host side around the kernels: the offline quantizer
(artifact layout of scripts/quantize.py), the loader and its validation
(utils/loader.py), and the tensor-parallel quantized Linear layers
(layers/linear.py), including a 2-rank gloo run of the TP sharding.
"""
from __future__ import annotations

import json
import os
import socket

import numpy as np
import pytest
import torch
import torch.multiprocessing as mp
from safetensors.torch import load_file, save_file
from torch import nn

import oracle

HID, HEADS, KV_HEADS, HEAD_DIM, INTER, LAYERS = 64, 4, 2, 16, 96, 2
Q, KV = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM


def _hf_checkpoint(seed: int = 0, qkv_bias: bool = False) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (torch.randn(*shape, generator=g) * 0.05).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": w(100, HID), "model.norm.weight": torch.ones(HID, dtype=torch.bfloat16)}
    for i in range(LAYERS):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = w(Q, HID)
        t[p + "self_attn.k_proj.weight"] = w(KV, HID)
        t[p + "self_attn.v_proj.weight"] = w(KV, HID)
        t[p + "self_attn.o_proj.weight"] = w(HID, Q)
        t[p + "mlp.gate_proj.weight"] = w(INTER, HID)
        t[p + "mlp.up_proj.weight"] = w(INTER, HID)
        t[p + "mlp.down_proj.weight"] = w(HID, INTER)
        t[p + "input_layernorm.weight"] = torch.ones(HID, dtype=torch.bfloat16)
        if qkv_bias:
            for s, n in (("q", Q), ("k", KV), ("v", KV)):
                t[p + f"self_attn.{s}_proj.bias"] = w(n)
    return t


def _write_model(dirpath, tensors):
    dirpath.mkdir(parents=True, exist_ok=True)
    save_file(tensors, dirpath / "model.safetensors")
    (dirpath / "config.json").write_text(json.dumps({"hidden_size": HID}))
    (dirpath / "tokenizer.json").write_text("{}")


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_quantize_cli_artifact_layout(tmp_path, mode):
    from nanovllm.quantization.quantize import main
    src = _hf_checkpoint(qkv_bias=True)
    _write_model(tmp_path / "src", src)
    main(["--model", str(tmp_path / "src"), "--output", str(tmp_path / "dst"), "--quantization", mode])
    out = load_file(tmp_path / "dst" / "model.safetensors")
    assert (tmp_path / "dst" / "config.json").is_file() and (tmp_path / "dst" / "tokenizer.json").is_file()
    scale = "w_scales" if mode == "w8a8" else "scales"
    for i in range(LAYERS):
        p = f"model.layers.{i}."
        for name, parts in (("self_attn.qkv_proj", ["q", "k", "v"]), ("mlp.gate_up_proj", ["gate", "up"])):
            kind = "self_attn" if name.startswith("self_attn") else "mlp"
            packed = torch.cat([src[p + f"{kind}.{s}_proj.weight"] for s in parts], 0)
            q_ref, s_ref = oracle.quantize_rows(packed.float().numpy())
            assert out[p + name + ".qweight"].dtype == torch.int8
            assert out[p + name + f".{scale}"].dtype == torch.float32
            np.testing.assert_array_equal(out[p + name + ".qweight"].numpy(), q_ref)
            np.testing.assert_array_equal(out[p + name + f".{scale}"].numpy(), s_ref)
        for name in ("self_attn.o_proj", "mlp.down_proj"):
            q_ref, s_ref = oracle.quantize_rows(src[p + name + ".weight"].float().numpy())
            np.testing.assert_array_equal(out[p + name + ".qweight"].numpy(), q_ref)
            assert p + name + ".weight" not in out
        bias = torch.cat([src[p + f"self_attn.{s}_proj.bias"] for s in "qkv"], 0)
        assert torch.equal(out[p + "self_attn.qkv_proj.bias"], bias)
        assert p + "self_attn.q_proj.weight" not in out
        assert torch.equal(out[p + "input_layernorm.weight"], src[p + "input_layernorm.weight"])
    assert torch.equal(out["model.embed_tokens.weight"], src["model.embed_tokens.weight"])


def test_quantize_rejects_partial_groups():
    from nanovllm.quantization.quantize import build_quantized_tensors
    t = _hf_checkpoint()
    del t["model.layers.1.self_attn.v_proj.weight"]
    with pytest.raises(ValueError, match=r"Missing qkv weight shards for model.layers.1.self_attn.: \['v'\]"):
        build_quantized_tensors(t, "int8")
    t = _hf_checkpoint()
    del t["model.layers.0.mlp.up_proj.weight"]
    with pytest.raises(ValueError, match="gate/up weight"):
        build_quantized_tensors(t, "w8a8")


class TinyQwen3Linears(nn.Module):
    """The four quantized projections of each layer, named as in Qwen3."""
    packed_modules_mapping = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v"),
                              "gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}

    def __init__(self, quantization):
        from nanovllm.layers.linear import MergedColumnParallelLinear, QKVParallelLinear, RowParallelLinear
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList()
        for _ in range(LAYERS):
            layer = nn.Module()
            layer.self_attn = nn.Module()
            layer.self_attn.qkv_proj = QKVParallelLinear(HID, HEAD_DIM, HEADS, KV_HEADS, quantization=quantization)
            layer.self_attn.o_proj = RowParallelLinear(Q, HID, quantization=quantization)
            layer.mlp = nn.Module()
            layer.mlp.gate_up_proj = MergedColumnParallelLinear(HID, [INTER, INTER], quantization=quantization)
            layer.mlp.down_proj = RowParallelLinear(INTER, HID, quantization=quantization)
            layer.input_layernorm = nn.Module()
            layer.input_layernorm.weight = nn.Parameter(torch.empty(HID, dtype=torch.bfloat16))
            self.model.layers.append(layer)
        self.model.embed_tokens = nn.Module()
        self.model.embed_tokens.weight = nn.Parameter(torch.empty(100, HID, dtype=torch.bfloat16))
        self.model.norm = nn.Module()
        self.model.norm.weight = nn.Parameter(torch.empty(HID, dtype=torch.bfloat16))


def _quantized_dir(tmp_path, mode):
    from nanovllm.quantization.quantize import main
    src = _hf_checkpoint(seed=3)
    _write_model(tmp_path / "src", src)
    main(["--model", str(tmp_path / "src"), "--output", str(tmp_path / mode), "--quantization", mode])
    return src, tmp_path / mode


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_loader_fills_quantized_layers_and_forward_matches_torch_path(tmp_path, mode):
    from nanovllm.utils.loader import load_model
    src, qdir = _quantized_dir(tmp_path, mode)
    model = TinyQwen3Linears(mode)
    load_model(model, str(qdir), mode)
    art = load_file(qdir / "model.safetensors")
    scale = "w_scales" if mode == "w8a8" else "scales"
    lay = model.model.layers[1].mlp.gate_up_proj
    assert torch.equal(lay.qweight.data, art["model.layers.1.mlp.gate_up_proj.qweight"])
    assert torch.equal(getattr(lay, scale).data, art[f"model.layers.1.mlp.gate_up_proj.{scale}"])
    x = (torch.randn(3, HID, generator=torch.Generator().manual_seed(1))).to(torch.bfloat16)
    y = lay(x)
    if mode == "int8":
        ref = oracle.w8a16_torch_path(x, lay.qweight.data, lay.scales.data)
    else:
        xq, a_s = oracle.quantize_rows_torch(x)
        ref = oracle.w8a8_torch_path(xq, a_s, lay.qweight.data, lay.w_scales.data, None, torch.bfloat16)
    assert torch.equal(y, ref)


def test_loader_reports_missing_quantized_tensors(tmp_path):
    from nanovllm.utils.loader import load_model
    src, qdir = _quantized_dir(tmp_path, "int8")
    art = load_file(qdir / "model.safetensors")
    del art["model.layers.0.self_attn.o_proj.scales"]
    save_file(art, qdir / "model.safetensors")
    with pytest.raises(RuntimeError, match=r"Missing INT8 quantized tensors.*model.layers.0.self_attn.o_proj.scales"):
        load_model(TinyQwen3Linears("int8"), str(qdir), "int8")


def test_loader_unquantized_packed_mapping(tmp_path):
    from nanovllm.utils.loader import load_model
    src = _hf_checkpoint(seed=5)
    _write_model(tmp_path / "bf16", src)
    model = TinyQwen3Linears(None).to(torch.bfloat16)
    load_model(model, str(tmp_path / "bf16"))
    qkv = model.model.layers[0].self_attn.qkv_proj.weight.data
    p = "model.layers.0.self_attn."
    assert torch.equal(qkv, torch.cat([src[p + "q_proj.weight"], src[p + "k_proj.weight"], src[p + "v_proj.weight"]]))
    gu = model.model.layers[1].mlp.gate_up_proj.weight.data
    p = "model.layers.1.mlp."
    assert torch.equal(gu, torch.cat([src[p + "gate_proj.weight"], src[p + "up_proj.weight"]]))


# --------------------------------------------------------------- TP = 2 (gloo)

def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _tp_worker(rank, world, port, qdir, mode, outdir):
    import sys
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    torch.distributed.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from nanovllm.utils.loader import load_model
        model = TinyQwen3Linears(mode)
        load_model(model, qdir, mode)
        layer = model.model.layers[0]
        x = torch.randn(5, HID, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
        res = {
            "qkv_q": layer.self_attn.qkv_proj.qweight.data.clone(),
            "gu_q": layer.mlp.gate_up_proj.qweight.data.clone(),
            "down_q": layer.mlp.down_proj.qweight.data.clone(),
            "qkv_y": layer.self_attn.qkv_proj(x),
            "down_y": layer.mlp.down_proj(torch.randn(5, INTER, generator=torch.Generator().manual_seed(10))
                                          .to(torch.bfloat16)[:, rank * INTER // world:(rank + 1) * INTER // world]
                                          .contiguous()),
        }
        torch.save(res, os.path.join(outdir, f"rank{rank}.pt"))
    finally:
        torch.distributed.destroy_process_group()
    sys.stdout.flush()


@pytest.mark.parametrize("mode", ["int8", "w8a8"])
def test_tensor_parallel_sharding_two_ranks(tmp_path, mode):
    src, qdir = _quantized_dir(tmp_path, mode)
    art = load_file(qdir / "model.safetensors")
    mp.spawn(_tp_worker, args=(2, _free_port(), str(qdir), mode, str(tmp_path)), nprocs=2, join=True)
    r = [torch.load(tmp_path / f"rank{i}.pt", weights_only=True) for i in range(2)]
    p = "model.layers.0."
    qkv = art[p + "self_attn.qkv_proj.qweight"]
    q_all, k_all, v_all = qkv[:Q], qkv[Q:Q + KV], qkv[Q + KV:]
    for i in range(2):
        exp = torch.cat([q_all.chunk(2)[i], k_all.chunk(2)[i], v_all.chunk(2)[i]])
        assert torch.equal(r[i]["qkv_q"], exp)
        gu = art[p + "mlp.gate_up_proj.qweight"]
        exp = torch.cat([gu[:INTER].chunk(2)[i], gu[INTER:].chunk(2)[i]])
        assert torch.equal(r[i]["gu_q"], exp)
        assert torch.equal(r[i]["down_q"], art[p + "mlp.down_proj.qweight"].chunk(2, 1)[i])
    # Row-parallel: both ranks hold the all-reduced sum of their partial products.
    assert torch.equal(r[0]["down_y"], r[1]["down_y"])
