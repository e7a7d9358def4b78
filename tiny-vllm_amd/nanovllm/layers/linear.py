"""Tensor-parallel Linear layers with the quantized-linear plug-in
(reference: nanovllm/layers/linear.py).

These are the call sites of the hot path: every qkv / o / gate_up / down
projection of Qwen3 is one of these layers, and with `quantization` set to
"int8" (W8A16) or "w8a8" its forward goes through
`quant_method.apply(x, layer[, bias])` to the gfx950 kernels.

Kept identical to the reference because checkpoints and the offline artifact
depend on it:
  * parameter names (`weight`, or `qweight` + `scales` / `w_scales`, `bias`),
    dtypes and shapes per rank;
  * the `weight_loader` hooks and their sharding: column-parallel layers
    shard dim 0 (output channels, and the per-channel scales with them),
    row-parallel layers shard dim 1 (input channels; scales are replicated);
    merged / QKV layers place each shard (or each packed q|k|v, gate|up
    segment of a quantized artifact) at its per-rank offset;
  * bias only on TP rank 0 for row-parallel layers, then an all-reduce.

The TP rank / size come from torch.distributed when it is initialized and
default to a single rank otherwise.
"""
from __future__ import annotations

import torch
import torch.distributed as dist
import torch.nn.functional as F
from torch import nn

from nanovllm.quantization import Int8WeightOnlyQuantMethod, W8A8QuantMethod


def divide(numerator: int, denominator: int) -> int:
    assert numerator % denominator == 0, f"{numerator} is not divisible by {denominator}"
    return numerator // denominator


def _tp() -> tuple[int, int]:
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(), dist.get_world_size()
    return 0, 1


def _shard(t: torch.Tensor, dim: int, rank: int, size: int) -> torch.Tensor:
    return t.chunk(size, dim)[rank]


class LinearBase(nn.Module):
    """Holds either a float `weight` or the quantized parameters of the chosen
    QuantMethod (reference linear.py:13-68)."""

    def __init__(self, input_size: int, output_size: int, bias: bool = False, tp_dim: int | None = None,
                 quantization: str | None = None):
        super().__init__()
        if quantization not in (None, "int8", "w8a8"):
            raise NotImplementedError(f"Unsupported linear quantization: {quantization}")
        self.tp_dim = tp_dim
        self.tp_rank, self.tp_size = _tp()
        self.quantization = quantization
        if quantization == "int8":
            self.quant_method = Int8WeightOnlyQuantMethod()
        elif quantization == "w8a8":
            self.quant_method = W8A8QuantMethod()
        else:
            self.quant_method = None
        # Bumped by every weight_loader call: loaders write through
        # `param.data`, which does not advance the parameter's _version, so
        # caches derived from the weights key on this counter as well.
        self.weights_generation = 0
        if self.quant_method is None:
            self.weight = nn.Parameter(torch.empty(output_size, input_size))
            self.weight.weight_loader = self._tracked(self.weight_loader)
        else:
            self.quant_method.create_weights(self, input_size, output_size)
            self.qweight.weight_loader = self._tracked(self.qweight_loader)
            for name in ("scales", "w_scales"):
                if hasattr(self, name):
                    getattr(self, name).weight_loader = self._tracked(self.scales_loader)
        if bias:
            self.bias = nn.Parameter(torch.empty(output_size))
            self.bias.weight_loader = self._tracked(self.bias_loader)
        else:
            self.register_parameter("bias", None)

    def _tracked(self, loader):
        def load(*args, **kwargs):
            loader(*args, **kwargs)
            self.weights_generation += 1
        return load

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param.data.copy_(loaded_weight)

    def bias_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.weight_loader(param, loaded_weight)

    def qweight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.weight_loader(param, loaded_weight)

    def scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.weight_loader(param, loaded_weight)

    def apply_linear(self, x: torch.Tensor) -> torch.Tensor:
        if self.quant_method is not None:
            return self.quant_method.apply(x, self)
        return F.linear(x, self.weight, self.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class ReplicatedLinear(LinearBase):
    def __init__(self, input_size: int, output_size: int, bias: bool = False, quantization: str | None = None):
        super().__init__(input_size, output_size, bias, quantization=quantization)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.apply_linear(x)


class ColumnParallelLinear(LinearBase):
    """Output channels sharded over TP ranks (reference linear.py:89-117)."""

    def __init__(self, input_size: int, output_size: int, bias: bool = False, quantization: str | None = None):
        _, tp_size = _tp()
        super().__init__(input_size, divide(output_size, tp_size), bias, 0, quantization)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        n = param.data.size(self.tp_dim)
        param.data.copy_(loaded_weight.narrow(self.tp_dim, self.tp_rank * n, n))

    def scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        n = param.data.size(0)
        param.data.copy_(loaded_weight.narrow(0, self.tp_rank * n, n))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.apply_linear(x)


class MergedColumnParallelLinear(ColumnParallelLinear):
    """Several column-parallel outputs stacked along dim 0, e.g. gate|up
    (reference linear.py:120-175)."""

    def __init__(self, input_size: int, output_sizes: list[int], bias: bool = False,
                 quantization: str | None = None):
        self.output_sizes = output_sizes
        super().__init__(input_size, sum(output_sizes), bias, quantization)

    def _segments(self):
        """(dst_offset, dst_size, src_offset, src_size) of each merged output on this rank."""
        out = []
        for i, size in enumerate(self.output_sizes):
            before = sum(self.output_sizes[:i])
            out.append((before // self.tp_size, size // self.tp_size, before, size))
        return out

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: int):
        dst_off, dst_size, _, _ = self._segments()[loaded_shard_id]
        dst = param.data.narrow(self.tp_dim, dst_off, dst_size)
        dst.copy_(_shard(loaded_weight, self.tp_dim, self.tp_rank, self.tp_size))

    def _packed_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, dim: int):
        # A quantized artifact stores the merged outputs already concatenated.
        for dst_off, dst_size, src_off, src_size in self._segments():
            src = _shard(loaded_weight.narrow(dim, src_off, src_size), dim, self.tp_rank, self.tp_size)
            param.data.narrow(dim, dst_off, dst_size).copy_(src)

    def packed_weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self._packed_loader(param, loaded_weight, self.tp_dim)

    def packed_scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self._packed_loader(param, loaded_weight, 0)

    def bias_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: int | None = None):
        if loaded_shard_id is None:
            self.packed_scales_loader(param, loaded_weight)
        else:
            self.weight_loader(param, loaded_weight, loaded_shard_id)

    def qweight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.packed_weight_loader(param, loaded_weight)

    def scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.packed_scales_loader(param, loaded_weight)


class QKVParallelLinear(ColumnParallelLinear):
    """q|k|v projections stacked along dim 0; heads sharded over TP ranks
    (reference linear.py:178-244)."""

    def __init__(self, hidden_size: int, head_size: int, total_num_heads: int,
                 total_num_kv_heads: int | None = None, bias: bool = False, quantization: str | None = None):
        _, tp_size = _tp()
        total_num_kv_heads = total_num_kv_heads or total_num_heads
        self.head_size = head_size
        self.num_heads = divide(total_num_heads, tp_size)
        self.num_kv_heads = divide(total_num_kv_heads, tp_size)
        output_size = (total_num_heads + 2 * total_num_kv_heads) * head_size
        super().__init__(hidden_size, output_size, bias, quantization)

    def qkv_shards(self):
        """(dst_offset, dst_size, src_offset, src_size) of q, k, v on this rank."""
        q = self.num_heads * self.head_size
        kv = self.num_kv_heads * self.head_size
        t = self.tp_size
        return ((0, q, 0, q * t), (q, kv, q * t, kv * t), (q + kv, kv, (q + kv) * t, kv * t))

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str):
        assert loaded_shard_id in ("q", "k", "v")
        dst_off, dst_size, _, _ = self.qkv_shards()["qkv".index(loaded_shard_id)]
        dst = param.data.narrow(self.tp_dim, dst_off, dst_size)
        dst.copy_(_shard(loaded_weight, self.tp_dim, self.tp_rank, self.tp_size))

    def _packed_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, dim: int):
        for dst_off, dst_size, src_off, src_size in self.qkv_shards():
            src = _shard(loaded_weight.narrow(dim, src_off, src_size), dim, self.tp_rank, self.tp_size)
            param.data.narrow(dim, dst_off, dst_size).copy_(src)

    def packed_weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self._packed_loader(param, loaded_weight, self.tp_dim)

    def packed_scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self._packed_loader(param, loaded_weight, 0)

    def bias_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str | None = None):
        if loaded_shard_id is None:
            self.packed_scales_loader(param, loaded_weight)
        else:
            self.weight_loader(param, loaded_weight, loaded_shard_id)

    def qweight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.packed_weight_loader(param, loaded_weight)

    def scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        self.packed_scales_loader(param, loaded_weight)


class RowParallelLinear(LinearBase):
    """Input channels sharded over TP ranks; partial outputs all-reduced
    (reference linear.py:247-276). Per-channel scales are replicated: each
    rank dequantizes its partial product before the reduction."""

    def __init__(self, input_size: int, output_size: int, bias: bool = False, quantization: str | None = None):
        _, tp_size = _tp()
        super().__init__(divide(input_size, tp_size), output_size, bias, 1, quantization)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        k = param.data.size(self.tp_dim)
        param.data.copy_(loaded_weight.narrow(self.tp_dim, self.tp_rank * k, k))

    def scales_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bias = self.bias if self.tp_rank == 0 else None
        if self.quant_method is not None:
            y = self.quant_method.apply(x, self, bias)
        else:
            y = F.linear(x, self.weight, bias)
        if self.tp_size > 1:
            dist.all_reduce(y)
        return y
