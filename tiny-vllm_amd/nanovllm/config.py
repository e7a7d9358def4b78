"""Engine configuration (reference: nanovllm/config.py).

Same fields, defaults and checks as the reference, with two differences
forced by this build's setting:
  * `model` is either a directory holding a Hugging Face `config.json` (and,
    optionally, safetensors weights and a tokenizer) or a `Qwen3Config`
    instance, which builds a randomly initialised model of that architecture
    (no checkpoints are available offline);
  * `tensor_parallel_size` must be 1: the engine drives one GPU. The layers
    themselves shard when torch.distributed is initialised.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, fields

from nanovllm.models.qwen3 import Qwen3Config


def qwen3_config_from_dir(path: str) -> tuple[Qwen3Config, int]:
    """Read config.json of a Qwen3 model directory -> (Qwen3Config, eos id)."""
    with open(os.path.join(path, "config.json")) as f:
        raw = json.load(f)
    names = {f.name for f in fields(Qwen3Config)}
    cfg = Qwen3Config(**{k: v for k, v in raw.items() if k in names})
    if "head_dim" not in raw:
        cfg.head_dim = cfg.hidden_size // cfg.num_attention_heads
    eos = raw.get("eos_token_id", -1)
    if isinstance(eos, list):
        eos = eos[0]
    return cfg, int(eos if eos is not None else -1)


@dataclass
class Config:
    model: str | Qwen3Config
    hf_config: Qwen3Config | None = None
    eos: int = -1
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = False
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    quantization: str | None = None
    quantized_model_path: str | None = None
    quant_group_size: int = 128
    quantize_lm_head: bool = False
    seed: int = 0

    def __post_init__(self):
        if self.tensor_parallel_size != 1:
            raise ValueError("this engine drives one GPU: tensor_parallel_size must be 1")
        assert self.kvcache_block_size % 256 == 0
        if self.quantization not in (None, "int8", "w8a8", "int4_awq"):
            raise ValueError(f"Unsupported quantization mode: {self.quantization}")
        if self.quantization == "int4_awq":
            raise NotImplementedError("int4_awq quantization is not implemented yet")
        if self.quantize_lm_head:
            raise NotImplementedError("quantize_lm_head is not implemented for the first INT8 phase")
        if self.quantized_model_path is not None:
            assert os.path.isdir(self.quantized_model_path)
        if isinstance(self.model, Qwen3Config):
            self.hf_config = self.model
        else:
            assert os.path.isdir(self.model), f"model directory not found: {self.model}"
            self.hf_config, eos = qwen3_config_from_dir(self.model)
            if self.eos == -1:
                self.eos = eos
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)
        assert self.max_num_batched_tokens >= self.max_model_len
