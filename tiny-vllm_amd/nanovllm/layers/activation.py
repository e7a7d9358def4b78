"""SiluAndMul (reference: nanovllm/layers/activation.py:6-14) on the fused
HIP producer kernel: silu(x[..., :I]) * x[..., I:], computed in fp32 with one
rounding (as the reference's compiled function). With `quant=True` the result
is returned as a QuantizedActivation for the W8A8 down projection. GPU
tensors always take the HIP kernel; CPU tensors take the torch expression.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nanovllm.quantization import _hip
from nanovllm.quantization.activation import QuantizedActivation


class SiluAndMul(nn.Module):
    def forward(self, x: torch.Tensor, quant: bool = False):
        shape = (*x.shape[:-1], x.shape[-1] // 2)
        if not x.is_cuda:
            g, u = x.float().chunk(2, -1)
            y = (F.silu(g) * u).to(x.dtype)
            if quant:
                from nanovllm.quantization.utils import quantize_int8_per_row_dynamic
                return QuantizedActivation(*quantize_int8_per_row_dynamic(y.reshape(-1, shape[-1])), x.dtype, shape)
            return y
        y, q = _hip.silu_mul(x.reshape(-1, x.shape[-1]).contiguous(), out=not quant, quant=quant)
        return QuantizedActivation(q[0], q[1], x.dtype, shape) if quant else y.view(shape)
