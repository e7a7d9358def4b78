"""Carrier for activations that arrive already quantized.

A producer kernel that fuses the per-token int8 quantization
(quantize_int8_per_row_dynamic, reference utils.py:28-32) into its epilogue
hands the W8A8 projection a QuantizedActivation instead of a bf16 tensor;
W8A8QuantMethod.apply then runs the GEMM on the codes directly. No reference
counterpart: the reference always quantizes inside W8A8QuantMethod.apply
(w8a8.py:25-40), with identical codes.
"""
from __future__ import annotations

from typing import NamedTuple

import torch


class QuantizedActivation(NamedTuple):
    xq: torch.Tensor        # int8 [M, K]
    scales: torch.Tensor    # fp32 [M]
    dtype: torch.dtype      # dtype of the activation it encodes (output dtype of the projection)
    shape: tuple            # logical shape (..., K) of that activation

    @property
    def is_cuda(self) -> bool:
        return self.xq.is_cuda
