"""ctypes binding of libtinyvllm_quant.so (include/tvq.h) plus thin torch-facing
wrappers that validate tensors, allocate outputs with torch's caching allocator
and launch on the current HIP stream.

This module replaces the reference's JIT-built pybind11 extensions
(nanovllm/quantization/cuda.py:146-222 loaders; csrc/*.cpp `forward` /
`select_path`). Nothing here computes on the CPU: if the library is missing or
a call fails, a RuntimeError is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libtinyvllm_quant.so"
ABI_VERSION = 5

OP_ACT_QUANT = 0
OP_W8A16 = 1
OP_W8A8 = 2

DTYPE_F16 = 0
DTYPE_BF16 = 1

_TORCH_TO_TVQ = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

# (name, restype, argtypes) for every symbol include/tvq.h declares.
_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SYMBOLS = (
    ("tvq_abi_version", _INT, ()),
    ("tvq_last_error", ctypes.c_char_p, ()),
    ("tvq_select_path", ctypes.c_char_p, (_INT, _I64, _I64, _I64, _INT)),
    ("tvq_act_quant", _INT, (_VP, _INT, _I64, _I64, ctypes.c_float, _VP, _VP, _VP)),
    ("tvq_w8a16_gemm", _INT, (_VP, _INT, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP, _I64, _VP)),
    ("tvq_w8a8_gemm", _INT, (_VP, _VP, _VP, _VP, _VP, _VP, _INT, _I64, _I64, _I64, _VP, _I64, _VP)),
    ("tvq_w8a8_gemm_i32", _INT, (_VP, _VP, _VP, _I64, _I64, _I64, _VP, _I64, _VP)),
    ("tvq_w8a16_gemm_rounded", _INT, (_VP, _INT, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP)),
    ("tvq_gemm_operand_floor", _INT, (_INT, _VP, _VP, _I64, _I64, _I64, _VP)),
    ("tvq_w8a8_linear", _INT, (_VP, _INT, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP, _VP, _VP, _I64, _VP)),
    ("tvq_gemm_workspace_bytes", _I64, ()),
    ("tvq_w8a8_linear_noalloc", _INT, (_VP, _INT, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP)),
    ("tvq_rmsnorm", _INT, (_VP, _VP, _VP, ctypes.c_float, _VP, _VP, _VP, _INT, _I64, _I64, _VP)),
    ("tvq_silu_mul", _INT, (_VP, _VP, _VP, _VP, _INT, _I64, _I64, _VP)),
    ("tvq_w8a8_gemm_glu", _INT, (_VP, _VP, _VP, _VP, _VP, _INT, _I64, _I64, _I64, _VP)),
    ("tvq_qk_norm_rope", _INT, (_VP, _I64, _VP, _VP, _VP, _VP, _VP, ctypes.c_float, _I64, _INT, _INT, _INT, _I64,
                                _VP, _VP, _VP, _VP, _VP, _I64, _I64, _INT, _VP)),
    ("tvq_prefill_attention", _INT, (_VP, _VP, _VP, _I64, _VP, _I64, _INT, _INT, _INT, ctypes.c_float, _VP, _INT,
                                     _VP)),
    ("tvq_decode_attention", _INT, (_VP, _I64, _VP, _I64, _VP, _I64, _VP, _VP, _VP, _VP, _I64, _INT, _INT, _INT, _I64,
                                    _I64, ctypes.c_float, _VP, _INT, _VP)),
    ("tvq_decode_attention_quant", _INT, (_VP, _I64, _VP, _I64, _VP, _I64, _VP, _VP, _VP, _VP, _I64, _INT, _INT, _INT,
                                          _I64, _I64, ctypes.c_float, _VP, _INT, _VP, _VP, ctypes.c_float, _VP, _I64,
                                          _VP)),
    ("tvq_prefill_attention_quant", _INT, (_VP, _VP, _VP, _I64, _VP, _I64, _INT, _INT, _INT, ctypes.c_float, _VP, _INT,
                                           _VP, _VP, ctypes.c_float, _VP, _I64, _VP)),
)


def library_path() -> Path:
    """Location of the built library: $TVQ_LIBRARY, else tiny-vllm_amd/lib/."""
    env = os.environ.get("TVQ_LIBRARY")
    if env:
        return Path(env)
    return Path(__file__).resolve().parents[2] / "lib" / LIB_NAME


_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


def load_library() -> ctypes.CDLL:
    """Load (once) and type the C ABI. Raises RuntimeError if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.is_file():
            raise RuntimeError(
                f"{LIB_NAME} not found at {path}; build it with `python tiny-vllm_amd/build.py` "
                "(or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:
            raise RuntimeError(f"failed to load {path}: {exc}") from exc
        for name, restype, argtypes in SYMBOLS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = list(argtypes)
        version = lib.tvq_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
        _LIB = lib
        return lib


def is_available() -> bool:
    try:
        load_library()
    except RuntimeError:
        return False
    return True


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().tvq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        _require(t.is_cuda, "all tensors must be on a ROCm (cuda) device")
        _require(t.is_contiguous(), "all tensors must be contiguous")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


_WORKSPACES: dict[int, torch.Tensor] = {}


def gemm_workspace(device: torch.device) -> torch.Tensor:
    """The device's split-K GEMM workspace: allocated zero-filled on first use
    and shared by every GEMM call on the device (the calls are ordered on the
    current stream; each leaves the workspace ready for the next). Allocate it
    before capturing HIP graphs, so captured and eager calls split alike."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WORKSPACES.get(idx)
    if ws is None:
        _require(not torch.cuda.is_current_stream_capturing(),
                 "the GEMM workspace must be allocated before HIP-graph capture (call gemm_workspace(device))")
        ws = torch.zeros(load_library().tvq_gemm_workspace_bytes(), dtype=torch.uint8, device=device)
        _WORKSPACES[idx] = ws
    return ws


_ATTN_COUNTERS: dict[int, torch.Tensor] = {}
ATTN_COUNTERS = 1 << 16  # row blocks (prefill) or sequences (decode) per quantizing attention call


def attn_counters(device: torch.device) -> torch.Tensor:
    """The device's counters for the attention kernels' fused o_proj
    quantization: zero-filled on first use, left zero by every call (calls
    are ordered on the current stream). Allocate before HIP-graph capture."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    c = _ATTN_COUNTERS.get(idx)
    if c is None:
        _require(not torch.cuda.is_current_stream_capturing(),
                 "the attention counters must be allocated before HIP-graph capture (call attn_counters(device))")
        c = torch.zeros(ATTN_COUNTERS, dtype=torch.int32, device=device)
        _ATTN_COUNTERS[idx] = c
    return c


def _ws(dev: torch.device, split_k: bool) -> tuple[int | None, int]:
    if not split_k:
        return None, 0
    ws = gemm_workspace(dev)
    return ws.data_ptr(), ws.numel()


def select_path(op: int, m: int, n: int, k: int, dtype: torch.dtype = torch.bfloat16) -> str:
    """Kernel path name for an op and shape (M-bucketed dispatch)."""
    res = load_library().tvq_select_path(op, m, n, k, _TORCH_TO_TVQ.get(dtype, DTYPE_BF16))
    _require(res is not None, f"invalid op {op}")
    return res.decode()


def act_quant(x: torch.Tensor, eps: float = 1e-8) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row dynamic int8 quantization of a 2-D bf16/fp16 tensor on the GPU."""
    lib = load_library()
    dev = _require_gpu(x)
    _require(x.dim() == 2, "x must be 2-D")
    _require(x.dtype in _TORCH_TO_TVQ, "x must be float16 or bfloat16")
    m, k = x.shape
    xq = torch.empty((m, k), dtype=torch.int8, device=dev)
    scales = torch.empty((m,), dtype=torch.float32, device=dev)
    if m == 0:
        return xq, scales
    _require(k > 0, "x must have K > 0")
    with torch.cuda.device(dev):
        rc = lib.tvq_act_quant(x.data_ptr(), _TORCH_TO_TVQ[x.dtype], m, k, eps, xq.data_ptr(), scales.data_ptr(),
                               _stream(dev))
    _check(rc, "tvq_act_quant")
    return xq, scales


def _check_weight(qweight: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None, k: int,
                  out_dtype: torch.dtype) -> int:
    _require(qweight.dim() == 2 and qweight.dtype == torch.int8, "qweight must be a 2-D int8 tensor")
    _require(qweight.shape[1] == k, f"Incompatible shapes: x[-1]={k} vs qweight[-1]={qweight.shape[1]}")
    n = qweight.shape[0]
    _require(scales.dim() == 1 and scales.dtype == torch.float32 and scales.numel() == n,
             "scales must be 1D float32 with one value per output channel")
    if bias is not None:
        _require(bias.dim() == 1 and bias.numel() == n, "bias must be 1D with one value per output channel")
        _require(bias.dtype == out_dtype, "bias dtype must match the output dtype")
    return n


def w8a16_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
               bias: torch.Tensor | None = None, split_k: bool = True) -> torch.Tensor:
    """y[M,N] = x[M,K] @ (qweight * scales[:,None])^T + bias, on the GPU."""
    lib = load_library()
    dev = _require_gpu(x, qweight, scales, bias)
    _require(x.dim() == 2, "x must be 2-D")
    _require(x.dtype in _TORCH_TO_TVQ, "x must be float16 or bfloat16")
    m, k = x.shape
    n = _check_weight(qweight, scales, bias, k, x.dtype)
    y = torch.empty((m, n), dtype=x.dtype, device=dev)
    if m == 0:
        return y
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a16_gemm(x.data_ptr(), _TORCH_TO_TVQ[x.dtype], qweight.data_ptr(), scales.data_ptr(),
                                _ptr(bias), y.data_ptr(), m, n, k, *_ws(dev, split_k), _stream(dev))
    _check(rc, "tvq_w8a16_gemm")
    return y


def w8a16_gemm_rounded(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
                       bias: torch.Tensor | None = None) -> torch.Tensor:
    """W8A16 with the reference kernel's rounding: y = x @ wd^T + bias with
    wd = T(T(qweight) * T(scales)[:,None]) in the activation dtype T."""
    lib = load_library()
    dev = _require_gpu(x, qweight, scales, bias)
    _require(x.dim() == 2, "x must be 2-D")
    _require(x.dtype in _TORCH_TO_TVQ, "x must be float16 or bfloat16")
    m, k = x.shape
    n = _check_weight(qweight, scales, bias, k, x.dtype)
    y = torch.empty((m, n), dtype=x.dtype, device=dev)
    if m == 0:
        return y
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a16_gemm_rounded(x.data_ptr(), _TORCH_TO_TVQ[x.dtype], qweight.data_ptr(), scales.data_ptr(),
                                        _ptr(bias), y.data_ptr(), m, n, k, _stream(dev))
    _check(rc, "tvq_w8a16_gemm_rounded")
    return y


def gemm_operand_floor(op: int, x: torch.Tensor, qweight: torch.Tensor) -> None:
    """Measurement: the operand stream alone of the DMA GEMM tiles the library
    would launch for (op, x, qweight); writes nothing."""
    lib = load_library()
    dev = _require_gpu(x, qweight)
    m, k = x.shape
    n = qweight.shape[0]
    with torch.cuda.device(dev):
        rc = lib.tvq_gemm_operand_floor(op, x.data_ptr(), qweight.data_ptr(), m, n, k, _stream(dev))
    _check(rc, "tvq_gemm_operand_floor")


def w8a8_gemm(x_q: torch.Tensor, a_scales: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
              bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16,
              split_k: bool = True) -> torch.Tensor:
    """y = ((x_q @ qweight^T) * a_scales[:,None]) * w_scales[None,:] + bias, int32 accumulation."""
    lib = load_library()
    dev = _require_gpu(x_q, a_scales, qweight, w_scales, bias)
    _require(out_dtype in _TORCH_TO_TVQ, "out_dtype must be float16 or bfloat16")
    _require(x_q.dim() == 2 and x_q.dtype == torch.int8, "x_q must be a 2-D int8 tensor")
    m, k = x_q.shape
    _require(a_scales.dim() == 1 and a_scales.dtype == torch.float32 and a_scales.numel() == m,
             "a_scales must be 1D float32 with one value per input row")
    n = _check_weight(qweight, w_scales, bias, k, out_dtype)
    y = torch.empty((m, n), dtype=out_dtype, device=dev)
    if m == 0:
        return y
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a8_gemm(x_q.data_ptr(), a_scales.data_ptr(), qweight.data_ptr(), w_scales.data_ptr(),
                               _ptr(bias), y.data_ptr(), _TORCH_TO_TVQ[out_dtype], m, n, k, *_ws(dev, split_k),
                               _stream(dev))
    _check(rc, "tvq_w8a8_gemm")
    return y


GLU_BLOCK = 32  # rows per gate / up block of tvq_w8a8_gemm_glu's weight layout


def glu_interleave(qweight: torch.Tensor, w_scales: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Regroup gate_up rows [gate (I) ; up (I)] into 32-row blocks gate_b, up_b
    (new row 64b + 32h + k <- old row h*I + 32b + k), the weight layout of
    w8a8_gemm_glu. I must be a multiple of 32."""
    n2 = qweight.shape[0]
    _require(n2 % (2 * GLU_BLOCK) == 0, "gate_up rows must be a multiple of 64")
    idx = torch.arange(n2, device=qweight.device).view(2, n2 // (2 * GLU_BLOCK), GLU_BLOCK).transpose(0, 1).reshape(-1)
    return qweight.index_select(0, idx).contiguous(), w_scales.index_select(0, idx).contiguous()


def w8a8_gemm_glu(x_q: torch.Tensor, a_scales: torch.Tensor, qweight_glu: torch.Tensor, w_scales_glu: torch.Tensor,
                  out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """silu(gate) * up of the W8A8 gate_up projection, [M, I], with the
    weights in glu_interleave layout; bit-identical to w8a8_gemm followed by
    silu_mul."""
    lib = load_library()
    dev = _require_gpu(x_q, a_scales, qweight_glu, w_scales_glu)
    _require(out_dtype in _TORCH_TO_TVQ, "out_dtype must be float16 or bfloat16")
    _require(x_q.dim() == 2 and x_q.dtype == torch.int8 and x_q.is_contiguous(), "x_q must be a contiguous 2-D int8 tensor")
    m, k = x_q.shape
    _require(a_scales.dim() == 1 and a_scales.dtype == torch.float32 and a_scales.numel() == m,
             "a_scales must be 1D float32 with one value per input row")
    n2 = _check_weight(qweight_glu, w_scales_glu, None, k, out_dtype)
    y = torch.empty((m, n2 // 2), dtype=out_dtype, device=dev)
    if m == 0:
        return y
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a8_gemm_glu(x_q.data_ptr(), a_scales.data_ptr(), qweight_glu.data_ptr(),
                                   w_scales_glu.data_ptr(), y.data_ptr(), _TORCH_TO_TVQ[out_dtype], m, n2, k,
                                   _stream(dev))
    _check(rc, "tvq_w8a8_gemm_glu")
    return y


def w8a8_gemm_i32(x_q: torch.Tensor, qweight: torch.Tensor, split_k: bool = True) -> torch.Tensor:
    """The exact int32 accumulator x_q @ qweight^T of the W8A8 path."""
    lib = load_library()
    dev = _require_gpu(x_q, qweight)
    _require(x_q.dim() == 2 and x_q.dtype == torch.int8, "x_q must be a 2-D int8 tensor")
    _require(qweight.dim() == 2 and qweight.dtype == torch.int8, "qweight must be a 2-D int8 tensor")
    m, k = x_q.shape
    _require(qweight.shape[1] == k, "x_q and qweight shapes do not align")
    n = qweight.shape[0]
    y = torch.empty((m, n), dtype=torch.int32, device=dev)
    if m == 0:
        return y
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a8_gemm_i32(x_q.data_ptr(), qweight.data_ptr(), y.data_ptr(), m, n, k, *_ws(dev, split_k),
                                   _stream(dev))
    _check(rc, "tvq_w8a8_gemm_i32")
    return y


def w8a8_linear(x: torch.Tensor, qweight: torch.Tensor, w_scales: torch.Tensor,
                bias: torch.Tensor | None = None, split_k: bool = True) -> torch.Tensor:
    """Fused per-token activation quantization + W8A8 GEMM; output in x.dtype."""
    lib = load_library()
    dev = _require_gpu(x, qweight, w_scales, bias)
    _require(x.dim() == 2, "x must be 2-D")
    _require(x.dtype in _TORCH_TO_TVQ, "x must be float16 or bfloat16")
    m, k = x.shape
    n = _check_weight(qweight, w_scales, bias, k, x.dtype)
    y = torch.empty((m, n), dtype=x.dtype, device=dev)
    if m == 0:
        return y
    xq = torch.empty((m, k), dtype=torch.int8, device=dev)
    a_s = torch.empty((m,), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = lib.tvq_w8a8_linear(x.data_ptr(), _TORCH_TO_TVQ[x.dtype], qweight.data_ptr(), w_scales.data_ptr(),
                                 _ptr(bias), y.data_ptr(), m, n, k, xq.data_ptr(), a_s.data_ptr(),
                                 *_ws(dev, split_k), _stream(dev))
    _check(rc, "tvq_w8a8_linear")
    return y


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
            out: bool = True, quant: bool = False):
    """RMSNorm of each row of x (after adding `residual`, which is then
    updated in place to the sum), on the GPU. Returns (y or None,
    (xq, a_scales) or None): y in x.dtype when `out`, the per-token int8
    codes and scales of y when `quant`."""
    lib = load_library()
    dev = _require_gpu(x, weight, residual)
    _require(x.dim() == 2 and x.is_contiguous(), "x must be a contiguous 2-D tensor")
    _require(x.dtype in _TORCH_TO_TVQ, "x must be float16 or bfloat16")
    _require(out or quant, "rmsnorm needs an output")
    m, k = x.shape
    _require(weight.dim() == 1 and weight.numel() == k and weight.dtype == x.dtype and weight.is_contiguous(),
             "weight must be a contiguous 1-D tensor of x's dtype and length K")
    if residual is not None:
        _require(residual.shape == x.shape and residual.dtype == x.dtype and residual.is_contiguous(),
                 "residual must match x")
    y = torch.empty_like(x) if out else None
    q = (torch.empty((m, k), dtype=torch.int8, device=dev), torch.empty((m,), dtype=torch.float32, device=dev)) \
        if quant else None
    if m == 0:
        return y, q
    with torch.cuda.device(dev):
        rc = lib.tvq_rmsnorm(x.data_ptr(), _ptr(residual), weight.data_ptr(), eps, _ptr(y),
                             q[0].data_ptr() if q else None, q[1].data_ptr() if q else None,
                             _TORCH_TO_TVQ[x.dtype], m, k, _stream(dev))
    _check(rc, "tvq_rmsnorm")
    return y, q


def silu_mul(gate_up: torch.Tensor, out: bool = True, quant: bool = False):
    """silu(gate_up[:, :I]) * gate_up[:, I:] on the GPU. Returns (y or None,
    (xq, a_scales) or None) as rmsnorm."""
    lib = load_library()
    dev = _require_gpu(gate_up)
    _require(gate_up.dim() == 2 and gate_up.is_contiguous(), "gate_up must be a contiguous 2-D tensor")
    _require(gate_up.dtype in _TORCH_TO_TVQ, "gate_up must be float16 or bfloat16")
    _require(gate_up.shape[1] % 2 == 0, "gate_up must have an even number of columns")
    _require(out or quant, "silu_mul needs an output")
    m, i = gate_up.shape[0], gate_up.shape[1] // 2
    y = torch.empty((m, i), dtype=gate_up.dtype, device=dev) if out else None
    q = (torch.empty((m, i), dtype=torch.int8, device=dev), torch.empty((m,), dtype=torch.float32, device=dev)) \
        if quant else None
    if m == 0:
        return y, q
    with torch.cuda.device(dev):
        rc = lib.tvq_silu_mul(gate_up.data_ptr(), _ptr(y), q[0].data_ptr() if q else None,
                              q[1].data_ptr() if q else None, _TORCH_TO_TVQ[gate_up.dtype], m, i, _stream(dev))
    _check(rc, "tvq_silu_mul")
    return y, q


def decode_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                     v_cache: torch.Tensor, slots: torch.Tensor, lens: torch.Tensor, scale: float,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Append k_new/v_new [B, Hkv, D] at position lens-1 of each sequence's
    cache slot and return softmax(scale q K^T) V for q [B, Hq, D]. The token
    dimension of q / k_new / v_new may be strided (views of a packed qkv)."""
    lib = load_library()
    dev = q.device
    for t in (q, k_new, v_new):
        _require(t.is_cuda and t.dim() == 3 and t.stride(2) == 1 and t.stride(1) == t.shape[2],
                 "q / k_new / v_new must be [B, H, D] with contiguous heads")
    for t in (k_cache, v_cache, slots, lens):
        _require(t.is_cuda and t.is_contiguous(), "cache / slots / lens must be contiguous GPU tensors")
    _require(slots.dtype == torch.int32 and lens.dtype == torch.int32, "slots and lens must be int32")
    b, hq, d = q.shape
    hkv = k_new.shape[1]
    _require(k_cache.dim() == 4 and k_cache.shape[1] == hkv and k_cache.shape[3] == d and
             v_cache.shape == k_cache.shape, "caches must be [slots, Hkv, max_len, D]")
    _require(q.dtype in _TORCH_TO_TVQ and k_cache.dtype == q.dtype, "dtype mismatch")
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=dev)
    if b == 0:
        return out
    with torch.cuda.device(dev):
        rc = lib.tvq_decode_attention(q.data_ptr(), q.stride(0), k_new.data_ptr(), k_new.stride(0), v_new.data_ptr(),
                                      v_new.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), slots.data_ptr(),
                                      lens.data_ptr(), b, hq, hkv, d, k_cache.shape[0], k_cache.shape[2], scale,
                                      out.data_ptr(),
                                      _TORCH_TO_TVQ[q.dtype], _stream(dev))
    _check(rc, "tvq_decode_attention")
    return out


def qk_norm_rope(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 q_weight: torch.Tensor | None, k_weight: torch.Tensor | None, eps: float, num_heads: int,
                 num_kv_heads: int, head_dim: int, k_cache: torch.Tensor | None = None,
                 v_cache: torch.Tensor | None = None, slots: torch.Tensor | None = None
                 ) -> tuple[torch.Tensor, torch.Tensor]:
    """q/k of a packed qkv [T, >= (Hq+Hkv)*D] (row-contiguous): per-head
    RMSNorm (when weights are given) and rotate-half rotary embedding.
    Returns q [T, Hq, D], k [T, Hkv, D]. With caches [S, Hkv, L, D] and
    per-token int64 slots, each token's key and value (the heads after the
    keys in qkv) are also stored at (slot, position)."""
    lib = load_library()
    dev = qkv.device
    _require(qkv.is_cuda and qkv.dim() == 2 and qkv.stride(1) == 1, "qkv must be a row-contiguous 2-D GPU tensor")
    _require(qkv.dtype in _TORCH_TO_TVQ, "qkv must be float16 or bfloat16")
    _require(positions.is_cuda and positions.dtype == torch.int64 and positions.is_contiguous(),
             "positions must be contiguous int64 on the GPU")
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32 and cos.is_contiguous() and
             sin.is_contiguous() and cos.shape == sin.shape and cos.shape[1] == head_dim // 2,
             "cos / sin must be contiguous fp32 [max_pos, head_dim/2]")
    for w in (q_weight, k_weight):
        _require(w is None or (w.dtype == qkv.dtype and w.is_contiguous() and w.numel() == head_dim),
                 "norm weights must be contiguous [head_dim] of qkv's dtype")
    t = qkv.shape[0]
    q = torch.empty((t, num_heads, head_dim), dtype=qkv.dtype, device=dev)
    k = torch.empty((t, num_kv_heads, head_dim), dtype=qkv.dtype, device=dev)
    if t == 0:
        return q, k
    store = k_cache is not None
    if store:
        _require(v_cache is not None and slots is not None, "k_cache, v_cache and slots go together")
        _require(k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape and
                 k_cache.dim() == 4 and k_cache.shape[1] == num_kv_heads and k_cache.shape[3] == head_dim and
                 k_cache.dtype == qkv.dtype, "caches must be contiguous [slots, Hkv, max_len, D] of qkv's dtype")
        _require(slots.is_cuda and slots.dtype == torch.int64 and slots.is_contiguous() and slots.numel() == t,
                 "slots must be contiguous int64 [T] on the GPU")
    with torch.cuda.device(dev):
        rc = lib.tvq_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                  _ptr(q_weight), _ptr(k_weight), eps, t, num_heads, num_kv_heads, head_dim,
                                  cos.shape[0], q.data_ptr(), k.data_ptr(), _ptr(k_cache), _ptr(v_cache),
                                  _ptr(slots), k_cache.shape[0] if store else 0, k_cache.shape[2] if store else 0,
                                  _TORCH_TO_TVQ[qkv.dtype], _stream(dev))
    _check(rc, "tvq_qk_norm_rope")
    return q, k


PREFILL_BLOCK_Q = 64  # TVQ_PREFILL_BLOCK_Q in include/tvq.h


def prefill_blocks(offsets_lens: list[tuple[int, int]], block_q: int = PREFILL_BLOCK_Q) -> torch.Tensor:
    """Host-side block table for prefill_attention: one (token offset,
    length, first query) row per PREFILL_BLOCK_Q-query block, blocks with the
    most keys first (they take longest)."""
    rows = [(off, n, q0) for off, n in offsets_lens for q0 in range(0, n, block_q)]
    rows.sort(key=lambda x: -x[2])
    return torch.tensor(rows, dtype=torch.int32).reshape(-1, 3)


def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, blocks: torch.Tensor,
                      scale: float) -> torch.Tensor:
    """Causal attention of packed prompts: q [T, Hq, D], k [T, Hkv, D]
    contiguous, v [T, Hkv, D] with contiguous heads (token stride free);
    blocks from prefill_blocks, on the GPU."""
    lib = load_library()
    dev = q.device
    _require(q.is_cuda and q.is_contiguous() and k.is_contiguous(), "q and k must be contiguous GPU tensors")
    _require(v.is_cuda and v.dim() == 3 and v.stride(2) == 1 and v.stride(1) == v.shape[2],
             "v must be [T, Hkv, D] with contiguous heads")
    _require(blocks.is_cuda and blocks.dtype == torch.int32 and blocks.is_contiguous() and blocks.dim() == 2,
             "blocks must be a contiguous int32 [n, 3] GPU tensor")
    _require(q.dtype in _TORCH_TO_TVQ and k.dtype == q.dtype and v.dtype == q.dtype, "dtype mismatch")
    t, hq, d = q.shape
    out = torch.empty_like(q)
    if blocks.shape[0] == 0:
        return out
    with torch.cuda.device(dev):
        rc = lib.tvq_prefill_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0), blocks.data_ptr(),
                                       blocks.shape[0], hq, k.shape[1], d, scale, out.data_ptr(),
                                       _TORCH_TO_TVQ[q.dtype], _stream(dev))
    _check(rc, "tvq_prefill_attention")
    return out


def prefill_attention_quant(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, blocks: torch.Tensor,
                            scale: float, eps: float = 1e-8) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """prefill_attention, with o_proj's per-token int8 quantization of the
    output in the same launch: returns (out, xq [T, Hq*D], a_scales [T]),
    the codes bit-identical to act_quant(out.view(T, -1), eps)."""
    lib = load_library()
    dev = q.device
    _require(q.is_cuda and q.is_contiguous() and k.is_contiguous(), "q and k must be contiguous GPU tensors")
    _require(v.is_cuda and v.dim() == 3 and v.stride(2) == 1 and v.stride(1) == v.shape[2],
             "v must be [T, Hkv, D] with contiguous heads")
    _require(blocks.is_cuda and blocks.dtype == torch.int32 and blocks.is_contiguous() and blocks.dim() == 2,
             "blocks must be a contiguous int32 [n, 3] GPU tensor")
    _require(q.dtype in _TORCH_TO_TVQ and k.dtype == q.dtype and v.dtype == q.dtype, "dtype mismatch")
    t, hq, d = q.shape
    out = torch.empty_like(q)
    xq = torch.empty((t, hq * d), dtype=torch.int8, device=dev)
    a_s = torch.empty((t,), dtype=torch.float32, device=dev)
    if blocks.shape[0] == 0:
        return out, xq, a_s
    cnt = attn_counters(dev)
    with torch.cuda.device(dev):
        rc = lib.tvq_prefill_attention_quant(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0), blocks.data_ptr(),
                                             blocks.shape[0], hq, k.shape[1], d, scale, out.data_ptr(),
                                             _TORCH_TO_TVQ[q.dtype], xq.data_ptr(), a_s.data_ptr(), eps,
                                             cnt.data_ptr(), cnt.numel(), _stream(dev))
    _check(rc, "tvq_prefill_attention_quant")
    return out, xq, a_s


def decode_attention_quant(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_cache: torch.Tensor,
                           v_cache: torch.Tensor, slots: torch.Tensor, lens: torch.Tensor, scale: float,
                           eps: float = 1e-8, out: torch.Tensor | None = None
                           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """decode_attention, with o_proj's per-token int8 quantization of the
    output in the same launch: returns (out, xq [B, Hq*D], a_scales [B])."""
    lib = load_library()
    dev = q.device
    for t in (q, k_new, v_new):
        _require(t.is_cuda and t.dim() == 3 and t.stride(2) == 1 and t.stride(1) == t.shape[2],
                 "q / k_new / v_new must be [B, H, D] with contiguous heads")
    for t in (k_cache, v_cache, slots, lens):
        _require(t.is_cuda and t.is_contiguous(), "cache / slots / lens must be contiguous GPU tensors")
    _require(slots.dtype == torch.int32 and lens.dtype == torch.int32, "slots and lens must be int32")
    b, hq, d = q.shape
    hkv = k_new.shape[1]
    _require(k_cache.dim() == 4 and k_cache.shape[1] == hkv and k_cache.shape[3] == d and
             v_cache.shape == k_cache.shape, "caches must be [slots, Hkv, max_len, D]")
    _require(q.dtype in _TORCH_TO_TVQ and k_cache.dtype == q.dtype, "dtype mismatch")
    if out is None:
        out = torch.empty((b, hq, d), dtype=q.dtype, device=dev)
    xq = torch.empty((b, hq * d), dtype=torch.int8, device=dev)
    a_s = torch.empty((b,), dtype=torch.float32, device=dev)
    if b == 0:
        return out, xq, a_s
    cnt = attn_counters(dev)
    with torch.cuda.device(dev):
        rc = lib.tvq_decode_attention_quant(q.data_ptr(), q.stride(0), k_new.data_ptr(), k_new.stride(0),
                                            v_new.data_ptr(), v_new.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
                                            slots.data_ptr(), lens.data_ptr(), b, hq, hkv, d, k_cache.shape[0],
                                            k_cache.shape[2], scale, out.data_ptr(), _TORCH_TO_TVQ[q.dtype],
                                            xq.data_ptr(), a_s.data_ptr(), eps, cnt.data_ptr(), cnt.numel(),
                                            _stream(dev))
    _check(rc, "tvq_decode_attention_quant")
    return out, xq, a_s
