"""Quantization maths and Qwen3 target names (reference: nanovllm/quantization/utils.py).

Both quantizers are symmetric int8 with an fp32 scale:
    s = max(amax / 127, eps)                        (fp32, IEEE round-to-nearest)
    q = clamp(round_half_even(float(w) / s), -127, 127)
`quantize_int8_per_channel` is applied row-wise to weights [N, K] (one scale
per output channel); `quantize_int8_per_row_dynamic` row-wise to activations
[M, K] (one scale per token). -128 is never produced.
"""
from pathlib import Path

import torch

QWEN3_INT8_WEIGHT_SUFFIXES = (
    ".self_attn.q_proj.weight",
    ".self_attn.k_proj.weight",
    ".self_attn.v_proj.weight",
    ".self_attn.o_proj.weight",
    ".mlp.gate_proj.weight",
    ".mlp.up_proj.weight",
    ".mlp.down_proj.weight",
)


def is_qwen3_int8_target_weight(name: str) -> bool:
    return name.endswith(QWEN3_INT8_WEIGHT_SUFFIXES)


def _quantize_rows(t: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    t32 = t.float()
    scales = torch.clamp_min(t32.abs().amax(dim=1) / 127.0, eps)
    q = torch.clamp(torch.round(t32 / scales[:, None]), -127, 127).to(torch.int8)
    return q, scales.to(torch.float32)


def quantize_int8_per_channel(weight: torch.Tensor, eps: float = 1e-8) -> tuple[torch.Tensor, torch.Tensor]:
    """Offline per-output-channel weight quantization (reference utils.py:21-25)."""
    return _quantize_rows(weight, eps)


def quantize_int8_per_row_dynamic(x: torch.Tensor, eps: float = 1e-8) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token activation quantization (reference utils.py:28-32). GPU
    tensors go to the fused HIP kernel (bit-identical) unless the W8A8
    backend is forced to `fallback`."""
    if x.is_cuda and x.dim() == 2 and x.dtype in (torch.float16, torch.bfloat16):
        from nanovllm.quantization.cuda import _get_w8a8_backend_preference
        if _get_w8a8_backend_preference() == "native":
            from nanovllm.quantization import _hip
            return _hip.act_quant(x.contiguous(), eps)
    return _quantize_rows(x, eps)


def iter_model_files(model_path: Path):
    for path in model_path.iterdir():
        if path.is_file() and path.suffix != ".safetensors":
            yield path
