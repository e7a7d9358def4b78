"""Backend dispatch for the quantized linears (W8A16 and W8A8).

Keeps the reference's module name and public functions
(nanovllm/quantization/cuda.py): `apply_int8_weight_only_linear`,
`apply_w8a8_linear`, `native_*`, `*_fallback`, the environment switches
`NANOVLLM_INT8_BACKEND` / `NANOVLLM_W8A8_BACKEND` and the one-shot path log
enabled by `NANOVLLM_INT8_LOG_PATH` / `NANOVLLM_W8A8_LOG_PATH`, with the same
line format (cuda.py:36-109). "cuda" is torch's device namespace, which on
ROCm means the HIP device; the native backend is the gfx950 HIP library
behind the C ABI (`_hip.py`).

Failure handling follows the reference (cuda.py:344-356, 487-503): when the
native call raises (an unsupported shape or alignment, a launch error), the
failure is logged once as `path=python_fallback reason=native_unavailable ...`
and the torch path computes the result. Two deliberate differences:
* `NANOVLLM_NATIVE_STRICT=1` turns that fallback off, so the exception
  propagates. Tests, the smoke check and the benchmark set it, so no
  measurement or parity check can be served by the torch path.
* A missing or unloadable HIP library always raises (it is a broken install,
  not a per-call condition), so a GPU deployment can never run on the slower
  torch path without noticing.

W8A16 numerics: by default the native kernels apply each channel's fp32 scale
once per output, after the dot product. `NANOVLLM_INT8_DEQUANT_ROUNDING=reference`
selects the reference kernel's rounding instead: every weight is dequantized to
the activation dtype as dtype(dtype(q) * dtype(s)) before the dot product
(int8_weight_only_gemm.cu:401-411, the same expression as the torch path,
cuda.py:293-300). No reference counterpart as a switch.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from nanovllm.quantization import _hip
from nanovllm.utils.context import get_context

_LOGGED_KERNEL_EVENTS: set[str] = set()
# "cutlass" and "auto" are accepted for compatibility; there is no CUTLASS on
# ROCm, and both are served by the native HIP kernels (logged once).
_SUPPORTED_BACKENDS = {"auto", "native", "fallback", "cutlass"}
_SUPPORTED_W8A8_BACKENDS = {"native", "fallback"}
_OFF_VALUES = ("", "0", "false", "off", "no")


def _should_log_kernel_path() -> bool:
    return os.environ.get("NANOVLLM_INT8_LOG_PATH", "").lower() not in _OFF_VALUES


def _should_log_w8a8_kernel_path() -> bool:
    return os.environ.get("NANOVLLM_W8A8_LOG_PATH", "").lower() not in _OFF_VALUES


def _get_backend_preference() -> str:
    value = os.environ.get("NANOVLLM_INT8_BACKEND", "native").strip().lower()
    return value if value in _SUPPORTED_BACKENDS else "native"


def _get_w8a8_backend_preference() -> str:
    value = os.environ.get("NANOVLLM_W8A8_BACKEND", "native").strip().lower()
    return value if value in _SUPPORTED_W8A8_BACKENDS else "native"


def _strict_native() -> bool:
    """NANOVLLM_NATIVE_STRICT: re-raise native failures instead of falling back."""
    return os.environ.get("NANOVLLM_NATIVE_STRICT", "").strip().lower() not in _OFF_VALUES


def _rounded_dequant() -> bool:
    """NANOVLLM_INT8_DEQUANT_ROUNDING=reference: the reference kernel's per-weight rounding."""
    return os.environ.get("NANOVLLM_INT8_DEQUANT_ROUNDING", "fp32").strip().lower() in ("reference", "activation")


def _get_phase() -> str:
    return "prefill" if get_context().is_prefill else "decode"


def _log_kernel_event_once(event: str, message: str) -> None:
    if event in _LOGGED_KERNEL_EVENTS:
        return
    _LOGGED_KERNEL_EVENTS.add(event)
    print(message)


def _log_backend_event_once(*, backend: str, phase: str, path: str, x: torch.Tensor, qweight: torch.Tensor,
                            reason: str | None = None) -> None:
    if not _should_log_kernel_path():
        return
    event = f"int8:{backend}:{phase}:{path}:{reason or ''}:{x.dtype}"
    message = (f"[nanovllm.int8] backend={backend} phase={phase} path={path} "
               f"x_dtype={x.dtype} x_shape={tuple(x.shape)} qweight_shape={tuple(qweight.shape)}")
    if reason is not None:
        message += f" reason={reason}"
    _log_kernel_event_once(event, message)


def _log_w8a8_backend_event_once(*, backend: str, phase: str, path: str, x_q: torch.Tensor, qweight: torch.Tensor,
                                 out_dtype: torch.dtype, reason: str | None = None) -> None:
    if not _should_log_w8a8_kernel_path():
        return
    event = f"w8a8:{backend}:{phase}:{path}:{reason or ''}:{out_dtype}"
    message = (f"[nanovllm.w8a8] backend={backend} phase={phase} path={path} "
               f"out_dtype={out_dtype} x_q_shape={tuple(x_q.shape)} qweight_shape={tuple(qweight.shape)}")
    if reason is not None:
        message += f" reason={reason}"
    _log_kernel_event_once(event, message)


def _on_gpu(*tensors: torch.Tensor | None) -> bool:
    return all(t is None or t.is_cuda for t in tensors)


def _validate_int8(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None) -> None:
    """Argument checks of the reference (cuda.py:21-33, 236-241)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"INT8 weight-only linear requires float16/bfloat16 activations, got {x.dtype}")
    if qweight.dtype != torch.int8 or scales.dtype != torch.float32:
        raise RuntimeError("qweight must be int8 and scales float32")
    if x.shape[-1] != qweight.shape[-1]:
        raise RuntimeError(f"Incompatible shapes: x[-1]={x.shape[-1]} vs qweight[-1]={qweight.shape[-1]}")
    if scales.dim() != 1 or scales.numel() != qweight.shape[0]:
        raise RuntimeError("scales must be 1D with one value per output channel")
    if bias is not None and (bias.dim() != 1 or bias.numel() != qweight.shape[0]):
        raise RuntimeError("bias must be 1D with one value per output channel")


def native_int8_weight_only_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                                   bias: torch.Tensor | None = None) -> torch.Tensor:
    """W8A16 on the gfx950 HIP kernels (reference: cuda.py:261-274)."""
    _validate_int8(x, qweight, scales, bias)
    if not _on_gpu(x, qweight, scales, bias):
        raise RuntimeError("native INT8 weight-only backend requires GPU tensors")
    n = qweight.shape[0]
    x_2d = x.contiguous().view(-1, x.shape[-1])
    bias = None if bias is None else bias.contiguous()
    if _rounded_dequant():
        _log_backend_event_once(backend="native", phase=_get_phase(), path="rounded_dequant", x=x_2d,
                                qweight=qweight)
        y = _hip.w8a16_gemm_rounded(x_2d, qweight.contiguous(), scales.contiguous(), bias)
        return y.view(*x.shape[:-1], n)
    path = _hip.select_path(_hip.OP_W8A16, x_2d.shape[0], n, x_2d.shape[1], x.dtype)
    _log_backend_event_once(backend="native", phase=_get_phase(), path=path, x=x_2d, qweight=qweight)
    y = _hip.w8a16_gemm(x_2d, qweight.contiguous(), scales.contiguous(), bias)
    return y.view(*x.shape[:-1], n)


def cutlass_int8_weight_only_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                                    bias: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's CUTLASS backend (cuda.py:277-290) has no ROCm counterpart;
    its prefill role is taken by the native tiled MFMA kernel."""
    return native_int8_weight_only_linear(x, qweight, scales, bias)


def int8_weight_only_linear_fallback(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's torch path (cuda.py:293-300): dequantize in x.dtype, then F.linear."""
    weight = qweight.to(x.dtype) * scales.to(x.dtype).unsqueeze(1)
    return F.linear(x, weight, bias)


def apply_int8_weight_only_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                                  bias: torch.Tensor | None = None) -> torch.Tensor:
    """Dispatch of the W8A16 linear (reference: cuda.py:303-366)."""
    backend = _get_backend_preference()
    if backend == "fallback":
        _log_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback", x=x,
                                qweight=qweight, reason="backend_forced_fallback")
        return int8_weight_only_linear_fallback(x, qweight, scales, bias)
    if not _on_gpu(x, qweight, scales, bias):
        _log_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback", x=x,
                                qweight=qweight, reason="cpu_tensors")
        return int8_weight_only_linear_fallback(x, qweight, scales, bias)
    if backend in ("cutlass", "auto"):
        _log_backend_event_once(backend="cutlass", phase=_get_phase(), path="unavailable", x=x, qweight=qweight,
                                reason="no CUTLASS on ROCm; served by the native HIP kernels")
    _hip.load_library()  # a missing library is never hidden behind the torch path
    try:
        return native_int8_weight_only_linear(x, qweight, scales, bias)
    except Exception as exc:
        if _strict_native():
            raise
        _log_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback", x=x,
                                qweight=qweight, reason=f"native_unavailable {type(exc).__name__}: {exc}")
        return int8_weight_only_linear_fallback(x, qweight, scales, bias)

def _validate_w8a8(x_q: torch.Tensor, a_scales: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                   bias: torch.Tensor | None, out_dtype: torch.dtype) -> None:
    """Argument checks of the reference (cuda.py:369-391, 404-413)."""
    if x_q.dtype != torch.int8 or qweight.dtype != torch.int8:
        raise RuntimeError("x_q and qweight must be int8")
    if a_scales.dtype != torch.float32 or w_scales.dtype != torch.float32:
        raise RuntimeError("a_scales and w_scales must be float32")
    if out_dtype not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"W8A8 output dtype must be float16/bfloat16, got {out_dtype}")
    if x_q.dim() != 2 or qweight.dim() != 2:
        raise RuntimeError("x_q and qweight must be 2D")
    if x_q.shape[-1] != qweight.shape[-1]:
        raise RuntimeError(f"Incompatible shapes: x_q[-1]={x_q.shape[-1]} vs qweight[-1]={qweight.shape[-1]}")
    if a_scales.dim() != 1 or a_scales.numel() != x_q.shape[0]:
        raise RuntimeError("a_scales must be 1D with one value per input row")
    if w_scales.dim() != 1 or w_scales.numel() != qweight.shape[0]:
        raise RuntimeError("w_scales must be 1D with one value per output channel")
    if bias is not None and (bias.dim() != 1 or bias.numel() != qweight.shape[0]):
        raise RuntimeError("bias must be 1D with one value per output channel")


def native_w8a8_linear(x_q: torch.Tensor, a_scales: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                       bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """W8A8 GEMM on the gfx950 HIP kernels (reference: cuda.py:435-452)."""
    _validate_w8a8(x_q, a_scales, qweight, w_scales, bias, out_dtype)
    if not _on_gpu(x_q, a_scales, qweight, w_scales, bias):
        raise RuntimeError("native W8A8 backend requires GPU tensors")
    path = _hip.select_path(_hip.OP_W8A8, x_q.shape[0], qweight.shape[0], x_q.shape[1], out_dtype)
    _log_w8a8_backend_event_once(backend="native", phase=_get_phase(), path=path, x_q=x_q, qweight=qweight,
                                 out_dtype=out_dtype)
    if bias is not None:
        bias = bias.to(out_dtype).contiguous()
    return _hip.w8a8_gemm(x_q.contiguous(), a_scales.contiguous(), qweight.contiguous(), w_scales.contiguous(),
                          bias, out_dtype)


def w8a8_linear_fallback(x_q: torch.Tensor, a_scales: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                         bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """The reference's torch path (cuda.py:455-465): dequantize both operands in out_dtype, then F.linear."""
    x = x_q.to(out_dtype) * a_scales.to(out_dtype).unsqueeze(1)
    weight = qweight.to(out_dtype) * w_scales.to(out_dtype).unsqueeze(1)
    return F.linear(x, weight, bias)


def apply_w8a8_linear(x_q: torch.Tensor, a_scales: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                      bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16,
                      out_shape: tuple[int, ...] | None = None) -> torch.Tensor:
    """Dispatch of the W8A8 GEMM (reference: cuda.py:468-504)."""
    backend = _get_w8a8_backend_preference()
    if backend == "fallback" or not _on_gpu(x_q, a_scales, qweight, w_scales, bias):
        reason = "backend_forced_fallback" if backend == "fallback" else "cpu_tensors"
        _log_w8a8_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback", x_q=x_q,
                                     qweight=qweight, out_dtype=out_dtype, reason=reason)
        y = w8a8_linear_fallback(x_q, a_scales, qweight, w_scales, bias, out_dtype)
    else:
        _hip.load_library()  # a missing library is never hidden behind the torch path
        try:
            y = native_w8a8_linear(x_q, a_scales, qweight, w_scales, bias, out_dtype)
        except Exception as exc:
            if _strict_native():
                raise
            _log_w8a8_backend_event_once(backend="fallback", phase=_get_phase(), path="python_fallback", x_q=x_q,
                                         qweight=qweight, out_dtype=out_dtype,
                                         reason=f"native_unavailable {type(exc).__name__}: {exc}")
            y = w8a8_linear_fallback(x_q, a_scales, qweight, w_scales, bias, out_dtype)
    return y if out_shape is None else y.view(out_shape)


def native_w8a8_fused_linear(x: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                             bias: torch.Tensor | None = None) -> torch.Tensor:
    """Activation quantization + W8A8 GEMM in one C-ABI call (two kernels on the
    current stream); the int8 activations never round-trip through Python.
    Numerically identical to quantize_int8_per_row_dynamic + apply_w8a8_linear."""
    if not _on_gpu(x, qweight, w_scales, bias):
        raise RuntimeError("native W8A8 backend requires GPU tensors")
    n = qweight.shape[0]
    x_2d = x.contiguous().view(-1, x.shape[-1])
    if _should_log_w8a8_kernel_path():
        path = _hip.select_path(_hip.OP_W8A8, x_2d.shape[0], n, x_2d.shape[1], x.dtype)
        _log_w8a8_backend_event_once(backend="native", phase=_get_phase(), path=path, x_q=x_2d, qweight=qweight,
                                     out_dtype=x.dtype)
    if bias is not None:
        bias = bias.to(x.dtype).contiguous()
    y = _hip.w8a8_linear(x_2d, qweight.contiguous(), w_scales.contiguous(), bias)
    return y.view(*x.shape[:-1], n)
