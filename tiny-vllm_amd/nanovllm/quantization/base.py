"""Quantized-linear plugin interface (reference: nanovllm/quantization/base.py:7-24)."""
from abc import ABC, abstractmethod

import torch
from torch import nn


class QuantMethod(ABC):
    """A quantization scheme for a Linear layer.

    `create_weights` registers the quantized parameters on `layer`,
    `apply` computes the layer output for activations `x`, and
    `quantize_activation` returns (x_q, scales) for schemes that quantize
    activations, else None.
    """

    @abstractmethod
    def create_weights(self, layer: nn.Module, input_size: int, output_size: int) -> None:
        raise NotImplementedError

    @abstractmethod
    def apply(self, x: torch.Tensor, layer: nn.Module, bias: torch.Tensor | None = None) -> torch.Tensor:
        raise NotImplementedError

    @abstractmethod
    def quantize_activation(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor] | None:
        raise NotImplementedError
