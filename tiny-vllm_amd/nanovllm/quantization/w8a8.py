"""W8A8 method: per-channel int8 weights, per-token dynamic int8 activations
(reference: nanovllm/quantization/w8a8.py)."""
import torch
from torch import nn

from nanovllm.quantization import _hip
from nanovllm.quantization.activation import QuantizedActivation
from nanovllm.quantization.base import QuantMethod
from nanovllm.quantization.cuda import (_get_phase, _get_w8a8_backend_preference, _log_w8a8_backend_event_once,
                                       _strict_native, apply_w8a8_linear, native_w8a8_fused_linear)
from nanovllm.quantization.utils import quantize_int8_per_row_dynamic


def _native(*tensors: torch.Tensor | None) -> bool:
    return _get_w8a8_backend_preference() == "native" and all(t is None or t.is_cuda for t in tensors)


class W8A8QuantMethod(QuantMethod):
    """Parameters `qweight` int8 [out, in] and `w_scales` fp32 [out]
    (reference w8a8.py:11-19)."""

    def create_weights(self, layer: nn.Module, input_size: int, output_size: int) -> None:
        layer.qweight = nn.Parameter(torch.empty(output_size, input_size, dtype=torch.int8), requires_grad=False)
        layer.w_scales = nn.Parameter(torch.empty(output_size, dtype=torch.float32), requires_grad=False)

    def quantize_activation(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-row dynamic int8 quantization of x viewed as [-1, K]
        (reference w8a8.py:21-23). On the GPU this is one HIP kernel that is
        bit-identical to quantize_int8_per_row_dynamic."""
        x_2d = x.contiguous().view(-1, x.shape[-1])
        if _native(x_2d):
            return _hip.act_quant(x_2d)
        return quantize_int8_per_row_dynamic(x_2d)

    def apply(self, x: torch.Tensor, layer: nn.Module, bias: torch.Tensor | None = None) -> torch.Tensor:
        bias = bias if bias is not None else layer.bias
        if isinstance(x, QuantizedActivation):
            # codes + scales from a producer kernel with the quantization fused in
            return apply_w8a8_linear(x.xq, x.scales, layer.qweight, layer.w_scales, bias=bias, out_dtype=x.dtype,
                                     out_shape=(*x.shape[:-1], layer.qweight.shape[0]))
        if _native(x, layer.qweight, layer.w_scales, bias):
            # quantize + GEMM in one ABI call (reference w8a8.py:25-40 does
            # quantize_activation then apply_w8a8_linear; same numerics).
            _hip.load_library()  # a missing library is never hidden behind the torch path
            try:
                return native_w8a8_fused_linear(x, layer.qweight, layer.w_scales, bias)
            except Exception as exc:
                if _strict_native():
                    raise
                # the reference's fallback (cuda.py:487-503): log once, then torch
                _log_w8a8_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback",
                                             x_q=x, qweight=layer.qweight, out_dtype=x.dtype,
                                             reason=f"native_unavailable {type(exc).__name__}: {exc}")
                x_q, a_scales = quantize_int8_per_row_dynamic(x.contiguous().view(-1, x.shape[-1]))
                return apply_w8a8_linear(x_q, a_scales, layer.qweight, layer.w_scales, bias=bias,
                                         out_dtype=x.dtype, out_shape=(*x.shape[:-1], layer.qweight.shape[0]))
        x_q, a_scales = self.quantize_activation(x)
        return apply_w8a8_linear(x_q, a_scales, layer.qweight, layer.w_scales, bias=bias, out_dtype=x.dtype,
                                 out_shape=(*x.shape[:-1], layer.qweight.shape[0]))
