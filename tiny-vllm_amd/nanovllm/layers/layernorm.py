"""RMSNorm (reference: nanovllm/layers/layernorm.py:6-49) on the fused HIP
producer kernel.

`forward(x, residual=None)` keeps the reference's contract: without a
residual it returns rmsnorm(x); with one it returns (rmsnorm(x + residual),
x + residual), the norm taken of the fp32 sum and the new residual rounded
to x's dtype. With `quant=True` the normalised rows are returned as a
QuantizedActivation (per-token int8 codes + scales, bit-identical to
quantize_int8_per_row_dynamic of the rounded output), for a W8A8 projection
to consume without a bf16 round trip.

GPU tensors always take the HIP kernel (a failure raises); CPU tensors take
the reference's torch expression.
"""
from __future__ import annotations

import torch
from torch import nn

from nanovllm.quantization import _hip
from nanovllm.quantization.activation import QuantizedActivation


def rms_forward_torch(x: torch.Tensor, weight: torch.Tensor, eps: float,
                      residual: torch.Tensor | None = None):
    """The reference's torch expression (layernorm.py:16-40)."""
    dtype = x.dtype
    h = x.float()
    if residual is not None:
        h = h + residual.float()
        residual = h.to(dtype)
    y = (h * torch.rsqrt(h.pow(2).mean(dim=-1, keepdim=True) + eps)).to(dtype) * weight
    return y if residual is None else (y, residual)


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None, quant: bool = False):
        if not x.is_cuda:
            out = rms_forward_torch(x, self.weight, self.eps, residual)
            if quant:
                from nanovllm.quantization.utils import quantize_int8_per_row_dynamic
                y = out if residual is None else out[0]
                q = QuantizedActivation(*quantize_int8_per_row_dynamic(y.reshape(-1, y.shape[-1])), y.dtype,
                                        tuple(y.shape))
                return q if residual is None else (q, out[1])
            return out
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous()
        if residual is not None:
            residual = residual.reshape(-1, shape[-1]).contiguous()
        y, q = _hip.rmsnorm(x2, self.weight, self.eps, residual, out=not quant, quant=quant)
        out = QuantizedActivation(q[0], q[1], x.dtype, tuple(shape)) if quant else y.view(shape)
        return out if residual is None else (out, residual.view(shape))
