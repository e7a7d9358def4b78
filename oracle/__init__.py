"""CPU oracle for tiny-vLLM's quantized-linear path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package, and only as the checker (or, for the
baseline, as the timed CPU restatement of the reference's torch path). The
product path (tiny-vllm_amd/) never imports it.

Two independent restatements of the same arithmetic:
  * numpy / torch-CPU functions in this file;
  * C functions in tvq_oracle.c (liboracle.so, built by oracle/Makefile).
Each function cites the reference code it restates. tests/test_oracle.py pins
them against closed-form special cases, against each other, against brute
force on tiny inputs and against invariants.

Parity status per function (see tests/test_oracle.py):
  quantize_rows            pinned (closed forms, ties, zero rows, torch, C)
  gemm_i32                 pinned (brute force, C vs numpy, invariants)
  gemm_i32_blas            pinned (equal to gemm_i32 / C at +-127 extremes)
  w8a8_epilogue_bf16       pinned (fp64 bound, sign/zero cases, C vs numpy)
  w8a16_torch_path         pinned against the exact fp64 product (bound)
  w8a8_torch_path          pinned against the exact fp64 product (bound)
  w8a16_f64 / w8a8_f64     pinned (brute force on tiny inputs, C vs numpy)
  w8a16_rounded_weights    pinned (CPU torch running the reference's expression,
                           bit for bit; power-of-two scales; known answers; C)
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "liboracle.so"

EPS = np.float32(1e-8)


# --------------------------------------------------------------------------
# bf16 / fp16 bit helpers (numpy)
# --------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact bf16 -> fp32 widening."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (c10::BFloat16 semantics)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return bits.astype(np.uint16).view(np.float16).astype(np.float32)


def to_f32(bits: np.ndarray, is_bf16: bool) -> np.ndarray:
    return bf16_bits_to_f32(bits) if is_bf16 else f16_bits_to_f32(bits)


# --------------------------------------------------------------------------
# numpy restatement
# --------------------------------------------------------------------------

def quantize_rows(x_f32: np.ndarray, eps: np.float32 = EPS) -> tuple[np.ndarray, np.ndarray]:
    """Row-wise symmetric int8 quantization.

    Restates quantize_int8_per_row_dynamic (nanovllm/quantization/utils.py:28-32)
    and quantize_int8_per_channel (utils.py:21-25):
        s = max(amax_row(|x|) / 127, eps)        fp32, IEEE round-to-nearest
        q = clamp(round_half_even(x / s), -127, 127)
    """
    x = np.asarray(x_f32, dtype=np.float32)
    amax = np.max(np.abs(x), axis=1) if x.shape[1] > 0 else np.zeros(x.shape[0], np.float32)
    s = np.maximum(amax / np.float32(127.0), np.float32(eps)).astype(np.float32)
    q = np.clip(np.rint(x / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def gemm_i32(xq: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact accumulator sum_k xq[m,k]*w[n,k] (w8a8_gemm.cu:336-375), via int64."""
    acc = xq.astype(np.int64) @ w.astype(np.int64).T
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def gemm_i32_blas(xq: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The same exact accumulator through a float64 BLAS product, for shapes
    too large for the scalar loops: every product is an integer of magnitude
    <= 127*127 and every partial sum stays below 2**31 << 2**53, so each
    float64 addition is exact whatever order the BLAS sums in."""
    acc = np.asarray(xq, np.float64) @ np.asarray(w, np.float64).T
    assert np.abs(acc).max(initial=0) < 2**31
    return acc.astype(np.int32)


def w8a8_epilogue_f32(acc: np.ndarray, a_s: np.ndarray, w_s: np.ndarray) -> np.ndarray:
    """(float(acc) * a_s[m]) * w_s[n] in fp32, each product rounded (w8a8_gemm.cu:387-389),
    no bias (+0.0 added, as the reference adds a zero bias tile)."""
    p = acc.astype(np.float32) * a_s.astype(np.float32)[:, None]
    return (p * w_s.astype(np.float32)[None, :] + np.float32(0.0)).astype(np.float32)


def w8a8_epilogue_bf16(acc: np.ndarray, a_s: np.ndarray, w_s: np.ndarray) -> np.ndarray:
    return f32_to_bf16_bits(w8a8_epilogue_f32(acc, a_s, w_s))


def w8a16_f64(x_f32: np.ndarray, q: np.ndarray, s: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """Exact-arithmetic W8A16 product (x @ q^T) * s + b in float64."""
    y = (x_f32.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
    if bias is not None:
        y = y + bias.astype(np.float64)[None, :]
    return y


def w8a16_rounded_weights(q: np.ndarray, s: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    """The reference kernel's dequantized weight T(T(q) * T(s)) as float32
    values (int8_weight_only_gemm.cu:401-411; the torch path's
    qweight.to(T) * scales.to(T)[:, None], cuda.py:293-300). T(q) is exact, and
    the product of two T values is exact in fp64, so one rounding to T gives
    the rounded multiply."""
    if is_bf16:
        sr = bf16_bits_to_f32(f32_to_bf16_bits(s.astype(np.float32)))
        prod = (q.astype(np.float32) * sr[:, None]).astype(np.float32)
        return bf16_bits_to_f32(f32_to_bf16_bits(prod))
    with np.errstate(over="ignore"):  # overflow to +-inf is the IEEE result
        sr = s.astype(np.float16).astype(np.float32)
        return (q.astype(np.float32) * sr[:, None]).astype(np.float16).astype(np.float32)


def w8a16_rounded_f64(x_f32: np.ndarray, wd_f32: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """Exact x @ wd^T + b in float64 for the rounded-dequant mode."""
    y = x_f32.astype(np.float64) @ wd_f32.astype(np.float64).T
    if bias is not None:
        y = y + bias.astype(np.float64)[None, :]
    return y


def w8a8_f64(xq: np.ndarray, a_s: np.ndarray, w: np.ndarray, w_s: np.ndarray,
             bias: np.ndarray | None = None) -> np.ndarray:
    """Exact-arithmetic W8A8 product acc * a_s[m] * w_s[n] + b in float64."""
    acc = gemm_i32(xq, w).astype(np.float64)
    y = acc * a_s.astype(np.float64)[:, None] * w_s.astype(np.float64)[None, :]
    if bias is not None:
        y = y + bias.astype(np.float64)[None, :]
    return y


# --------------------------------------------------------------------------
# The reference's torch path, restated with CPU torch (the library, not the
# reference's code): these are what the reference computes when its native
# backend is not used.
# --------------------------------------------------------------------------

def w8a16_torch_path(x, qweight, scales, bias=None):
    """int8_weight_only_linear_fallback (nanovllm/quantization/cuda.py:293-300):
    weight = bf16(bf16(q) * bf16(s)), y = F.linear(x, weight, bias)."""
    import torch
    import torch.nn.functional as F
    weight = qweight.to(x.dtype) * scales.to(x.dtype).unsqueeze(1)
    return F.linear(x, weight, bias)


def w8a8_torch_path(x_q, a_scales, qweight, w_scales, bias=None, out_dtype=None):
    """w8a8_linear_fallback (nanovllm/quantization/cuda.py:455-465)."""
    import torch
    import torch.nn.functional as F
    out_dtype = out_dtype or torch.float16
    x = x_q.to(out_dtype) * a_scales.to(out_dtype).unsqueeze(1)
    weight = qweight.to(out_dtype) * w_scales.to(out_dtype).unsqueeze(1)
    return F.linear(x, weight, bias)


def w8a16_fp32_scale_torch(x, qweight, scales, bias=None):
    """The GPU kernels' W8A16 numerics in torch: fp32 sum of x * int8 (exact
    products), per-channel fp32 scale and bias once per output, one rounding
    to x.dtype. Differs from the reference torch path only in not rounding
    the dequantized weight to bf16 (int8_weight_only_gemm.cu:397-413 rounds)."""
    import torch
    y = (x.float() @ qweight.float().T) * scales.float()[None, :]
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)


def w8a8_fp32_scale_torch(x_q, a_scales, qweight, w_scales, bias=None, out_dtype=None):
    """The GPU kernels' W8A8 numerics in torch: exact integer accumulator,
    (float(acc) * a_s) * w_s + b in fp32 (w8a8_gemm.cu:387-390 order), one
    rounding to the output dtype."""
    import torch
    acc = (x_q.to(torch.int64) @ qweight.to(torch.int64).T).float()
    y = acc * a_scales.float()[:, None] * w_scales.float()[None, :]
    if bias is not None:
        y = y + bias.float()
    return y.to(out_dtype or torch.bfloat16)


def rmsnorm_ref(x_f32: np.ndarray, w_f32: np.ndarray, eps: float, res_f32: np.ndarray | None = None,
                is_bf16: bool = True):
    """RMSNorm of layernorm.py:16-40 with its roundings, statistics in fp64.
    x, w, residual are the (exactly representable) fp32 values of bf16/fp16
    inputs. Returns (y, new_residual or None) as fp32 arrays of rounded values:
      h = fp32(x + res)  (one fp32 rounding, as torch's fp32 add)
      r = 1/sqrt(mean(h^2) + eps)  (fp64 here; fp32 on the device)
      y = rnd(fp32(rnd(fp32(h*r)) * w))"""
    rnd = (lambda a: bf16_bits_to_f32(f32_to_bf16_bits(a))) if is_bf16 else \
        (lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32))
    h = np.asarray(x_f32, np.float32)
    new_res = None
    if res_f32 is not None:
        h = (h + np.asarray(res_f32, np.float32)).astype(np.float32)
        new_res = rnd(h)
    hd = h.astype(np.float64)
    r = 1.0 / np.sqrt((hd * hd).mean(axis=-1, keepdims=True) + eps)
    y1 = rnd((hd * r).astype(np.float32))
    y = rnd((y1 * np.asarray(w_f32, np.float32)).astype(np.float32))
    return y, new_res


def silu_mul_ref(gu_f32: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    """SiluAndMul (activation.py:11-14) in fp64, one rounding to bf16/fp16."""
    rnd = (lambda a: bf16_bits_to_f32(f32_to_bf16_bits(a))) if is_bf16 else \
        (lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32))
    g, u = np.split(np.asarray(gu_f32, np.float64), 2, axis=-1)
    return rnd((g / (1.0 + np.exp(-g)) * u).astype(np.float32))


def quantize_rows_torch(x):
    """quantize_int8_per_row_dynamic (utils.py:28-32) in CPU torch."""
    import torch
    xf = x.float()
    s = xf.abs().amax(dim=1).div(127.0).clamp_min(1e-8)
    q = torch.round(xf / s.unsqueeze(1)).clamp(-127, 127).to(torch.int8)
    return q, s.to(torch.float32)


# --------------------------------------------------------------------------
# C restatement (liboracle.so)
# --------------------------------------------------------------------------

_C = None


def build_c(force: bool = False) -> Path:
    """Compile tvq_oracle.c with the committed Makefile (also when the built
    library is older than the source)."""
    src = ORACLE_DIR / "tvq_oracle.c"
    stale = LIB_PATH.is_file() and LIB_PATH.stat().st_mtime < src.stat().st_mtime
    if force or stale or not LIB_PATH.is_file():
        cmd = ["make", "-C", str(ORACLE_DIR)] + (["-B"] if force else [])
        subprocess.run(cmd, check=True, capture_output=True)
    return LIB_PATH


def c_lib() -> ctypes.CDLL:
    global _C
    if _C is None:
        build_c()
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.oracle_act_quant.argtypes = [vp, i32, i64, i64, ctypes.c_float, vp, vp]
        lib.oracle_quant_f32.argtypes = [vp, i64, i64, ctypes.c_float, vp, vp]
        lib.oracle_gemm_i32.argtypes = [vp, vp, i64, i64, i64, vp]
        lib.oracle_w8a8_epilogue.argtypes = [vp, vp, vp, vp, i64, i64, vp, vp]
        lib.oracle_w8a16_f64.argtypes = [vp, i32, vp, vp, vp, i64, i64, i64, vp]
        lib.oracle_f32_to_bf16.argtypes = [vp, i64, vp]
        lib.oracle_w8a16_rounded_weights.argtypes = [vp, vp, i32, i64, i64, vp]
        lib.oracle_f32_to_f16.argtypes = [vp, i64, vp]
        lib.oracle_quant_code_sweep.argtypes = [i32, ctypes.c_float, i32, ctypes.POINTER(ctypes.c_int64)]
        lib.oracle_quant_code_sweep.restype = ctypes.c_int64
        for f in (lib.oracle_act_quant, lib.oracle_quant_f32, lib.oracle_gemm_i32, lib.oracle_w8a8_epilogue,
                  lib.oracle_w8a16_f64, lib.oracle_f32_to_bf16, lib.oracle_w8a16_rounded_weights,
                  lib.oracle_f32_to_f16):
            f.restype = None
        _C = lib
    return _C


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def c_act_quant(x_bits: np.ndarray, is_bf16: bool = True, eps: float = 1e-8) -> tuple[np.ndarray, np.ndarray]:
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, k = x_bits.shape
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    c_lib().oracle_act_quant(_p(x_bits), int(is_bf16), m, k, eps, _p(q), _p(s))
    return q, s


def c_quant_f32(x: np.ndarray, eps: float = 1e-8) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty((m,), np.float32)
    c_lib().oracle_quant_f32(_p(x), m, k, eps, _p(q), _p(s))
    return q, s


def c_gemm_i32(xq: np.ndarray, w: np.ndarray) -> np.ndarray:
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = xq.shape
    n = w.shape[0]
    assert w.shape[1] == k
    acc = np.empty((m, n), np.int32)
    c_lib().oracle_gemm_i32(_p(xq), _p(w), m, n, k, _p(acc))
    return acc


def c_w8a8_epilogue(acc: np.ndarray, a_s: np.ndarray, w_s: np.ndarray,
                    bias_f32: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Returns (bf16 bits, fp32 values) of (float(acc)*a_s)*w_s + bias (fma)."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    a_s = np.ascontiguousarray(a_s, dtype=np.float32)
    w_s = np.ascontiguousarray(w_s, dtype=np.float32)
    if bias_f32 is not None:
        bias_f32 = np.ascontiguousarray(bias_f32, dtype=np.float32)
    m, n = acc.shape
    yb = np.empty((m, n), np.uint16)
    yf = np.empty((m, n), np.float32)
    c_lib().oracle_w8a8_epilogue(_p(acc), _p(a_s), _p(w_s), _p(bias_f32), m, n, _p(yb), _p(yf))
    return yb, yf


def c_w8a16_f64(x_bits: np.ndarray, q: np.ndarray, s: np.ndarray, bias_f32: np.ndarray | None = None,
                is_bf16: bool = True) -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    if bias_f32 is not None:
        bias_f32 = np.ascontiguousarray(bias_f32, dtype=np.float32)
    m, k = x_bits.shape
    n = q.shape[0]
    y = np.empty((m, n), np.float64)
    c_lib().oracle_w8a16_f64(_p(x_bits), int(is_bf16), _p(q), _p(s), _p(bias_f32), m, n, k, _p(y))
    return y


def c_w8a16_rounded_weights(q: np.ndarray, s: np.ndarray, is_bf16: bool = True) -> np.ndarray:
    """C restatement of w8a16_rounded_weights: the T bits of T(T(q) * T(s))."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    n, k = q.shape
    out = np.empty((n, k), np.uint16)
    c_lib().oracle_w8a16_rounded_weights(_p(q), _p(s), int(is_bf16), n, k, _p(out))
    return out


def c_quant_code_sweep(is_bf16: bool, variant: int = 0, eps: float = 1e-8) -> tuple[int, int]:
    """(mismatches, pairs) of the divide-free per-token code against
    rint(x / s) over every finite non-negative 16-bit (x <= amax) pair
    (oracle_quant_code_sweep)."""
    pairs = ctypes.c_int64(0)
    bad = c_lib().oracle_quant_code_sweep(int(is_bf16), eps, variant, ctypes.byref(pairs))
    return int(bad), int(pairs.value)


def c_f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    c_lib().oracle_f32_to_f16(_p(x), x.size, _p(out))
    return out


def c_f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    c_lib().oracle_f32_to_bf16(_p(x), x.size, _p(out))
    return out


# --------------------------------------------------------------------------
# Error metrics (the tolerance contract: rel-L2 <= 1e-2 and
# max-abs <= 2e-2 * max|ref|; bench_quant_quality.py:171-182 reports the same
# rel-L2 metric).
# --------------------------------------------------------------------------

def rel_l2(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / den) if den > 0 else float(np.linalg.norm(y - ref))


def max_abs_ratio(y: np.ndarray, ref: np.ndarray) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max(initial=0.0)
    diff = np.abs(y - ref).max(initial=0.0)
    return float(diff / den) if den > 0 else float(diff)


REL_L2_TOL = 1e-2
MAX_ABS_TOL = 2e-2
