"""CPU tests of the C ABI (no GPU compute) and of the Python dispatch layer.

* the library loads and exports every symbol include/tvq.h declares;
* argument validation and error reporting work without touching the GPU;
* path selection is the documented M-bucketed table;
* the nanovllm.quantization API keeps the reference's classes, parameter
  names/dtypes/shapes, environment switches and log format
  (nanovllm/quantization/{base,int8,w8a8,cuda}.py), and the torch path it
  falls back to on request matches the oracle.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols() -> list[str]:
    text = (ROOT / "include" / "tvq.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(tvq_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    syms = _declared_symbols()
    for name in ("tvq_abi_version", "tvq_last_error", "tvq_select_path", "tvq_act_quant", "tvq_w8a16_gemm",
                 "tvq_w8a8_gemm", "tvq_w8a8_gemm_i32", "tvq_w8a8_linear", "tvq_rmsnorm", "tvq_silu_mul",
                 "tvq_gemm_workspace_bytes", "tvq_w8a16_gemm_rounded", "tvq_gemm_operand_floor"):
        assert name in syms


def test_library_exports_every_declared_symbol(hiplib):
    from nanovllm.quantization import _hip
    lib = ctypes.CDLL(str(_hip.library_path()))
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert {n for n, _, _ in _hip.SYMBOLS} == set(_declared_symbols())


def test_abi_version_and_errors_without_gpu(hiplib):
    assert hiplib.tvq_abi_version() == 5
    assert hiplib.tvq_gemm_workspace_bytes() >= 32 << 20  # stream-K: two 64x256 fp32 images per CU
    assert hiplib.tvq_w8a16_gemm(None, 7, None, None, None, None, 1, 1, 16, None, 0, None) == -1
    assert b"dtype" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a16_gemm(None, 1, None, None, None, None, 1, 1, 16, None, 0, None) == -1
    assert b"null pointer" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a16_gemm(None, 1, None, None, None, None, 1, 1, 16, 0x1010, 1 << 20, None) == -1
    assert b"256-byte aligned" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a8_gemm(None, None, None, None, None, None, 1, 1, 0, 16, None, 0, None) == -1
    assert b"invalid shape" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a8_gemm_i32(None, None, None, 1, 1, 1 << 40, None, 0, None) == -2
    assert b"2^31" in hiplib.tvq_last_error()
    assert hiplib.tvq_act_quant(None, 1, 4, 16, -1.0, None, None, None) == -1
    # rounded-dequant W8A16: same validation as tvq_w8a16_gemm
    assert hiplib.tvq_w8a16_gemm_rounded(None, 9, None, None, None, None, 1, 1, 16, None) == -1
    assert b"dtype" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a16_gemm_rounded(None, 1, None, None, None, None, 1, 1, 16, None) == -1
    assert b"null pointer" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a16_gemm_rounded(None, 1, None, None, None, None, 0, 8, 16, None) == 0
    # operand floor: op check, then the DMA tiles' shape rule, before any launch
    assert hiplib.tvq_gemm_operand_floor(0, 0x1000, 0x1000, 4, 8, 128, None) == -1
    assert b"op must be" in hiplib.tvq_last_error()
    assert hiplib.tvq_gemm_operand_floor(2, 0x1000, 0x1000, 4, 8, 96, None) == -2
    assert b"K % 128" in hiplib.tvq_last_error()
    assert hiplib.tvq_gemm_operand_floor(1, 0x1008, 0x1000, 4, 8, 128, None) == -2
    assert hiplib.tvq_gemm_operand_floor(2, None, 0x1000, 4, 8, 128, None) == -1
    # attention with the fused o_proj quantization: its own arguments are checked first
    assert hiplib.tvq_prefill_attention_quant(None, None, None, 0, None, 2, 16, 8, 128, 0.1, None, 1, None, None,
                                              1e-8, None, 0, None) == -1
    assert b"null xq" in hiplib.tvq_last_error()
    assert hiplib.tvq_prefill_attention_quant(None, None, None, 0, None, 2, 16, 8, 128, 0.1, None, 1, 0x1000,
                                              0x1000, 1e-8, 0x1000, 1, None) == -1
    assert b"counters hold 1" in hiplib.tvq_last_error()
    assert hiplib.tvq_decode_attention_quant(None, 0, None, 0, None, 0, None, None, None, None, 3, 16, 8, 128, 4,
                                             64, 0.1, None, 1, 0x1000, 0x1000, 0.0, 0x1000, 8, None) == -1
    assert b"eps" in hiplib.tvq_last_error()
    assert hiplib.tvq_decode_attention_quant(None, 0, None, 0, None, 0, None, None, None, None, 3, 16, 8, 128, 4,
                                             64, 0.1, None, 1, 0x1001, 0x1000, 1e-8, 0x1000, 8, None) == -2
    assert hiplib.tvq_decode_attention_quant(None, 0, None, 0, None, 0, None, None, None, None, 0, 16, 8, 128, 4,
                                             64, 0.1, None, 1, None, None, 1e-8, None, 0, None) == 0
    assert hiplib.tvq_rmsnorm(None, None, None, 1e-6, None, None, None, 1, 4, 16, None) == -1
    assert b"null pointer" in hiplib.tvq_last_error()
    assert hiplib.tvq_rmsnorm(1, None, 1, 1e-6, None, None, None, 1, 4, 16, None) == -1
    assert b"needs an output" in hiplib.tvq_last_error()
    assert hiplib.tvq_silu_mul(1, None, 1, None, 1, 4, 16, None) == -1
    assert b"without a_scales" in hiplib.tvq_last_error()
    assert hiplib.tvq_silu_mul(1, 1, None, None, 1, 0, 16, None) == 0
    assert hiplib.tvq_w8a8_gemm_glu(None, None, None, None, None, 1, 4, 128, 128, None) == -1
    assert b"null pointer" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a8_gemm_glu(16, 16, 16, 16, 16, 1, 4, 96, 128, None) == -2
    assert b"N2 % 64" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a8_gemm_glu(16, 16, 16, 16, 16, 1, 4, 128, 100, None) == -2
    assert hiplib.tvq_w8a8_gemm_glu(16, 16, 16, 16, 8, 1, 4, 128, 128, None) == -2
    assert b"16-byte aligned" in hiplib.tvq_last_error()
    assert hiplib.tvq_w8a8_gemm_glu(None, None, None, None, None, 1, 0, 128, 128, None) == 0
    # M == 0 is a valid no-op that launches nothing
    assert hiplib.tvq_w8a16_gemm(None, 1, None, None, None, None, 0, 8, 16, None, 0, None) == 0
    assert hiplib.tvq_last_error() == b""


def test_select_path_buckets(hiplib):
    from nanovllm.quantization import _hip
    sp = _hip.select_path
    assert sp(_hip.OP_ACT_QUANT, 4, 0, 1024) == "act_quant_vec"
    assert sp(_hip.OP_ACT_QUANT, 4, 0, 100) == "act_quant_scalar"
    assert sp(_hip.OP_W8A16, 1, 4096, 1024) == "gemv_dot2_f16x"          # M <= 2, K % 1024 == 0
    assert sp(_hip.OP_W8A8, 2, 4096, 12288) == "gemv_dot4_i8"
    assert sp(_hip.OP_W8A8, 3, 4096, 12288) == "skinny_mfma_i8_m16"
    assert sp(_hip.OP_W8A8, 1, 4096, 1040) == "skinny_mfma_i8_m16"     # K % 1024 != 0
    assert sp(_hip.OP_W8A8, 1, 4096, 16384) == "skinny_mfma_i8_m16"    # K > 12288
    assert sp(_hip.OP_W8A16, 16, 4096, 1024) == "skinny_mfma_f16x_m16"
    assert sp(_hip.OP_W8A16, 64, 4096, 1024) == "dma_mfma_f16x_32x64"     # 16 < M <= 64: DMA tiles
    # split-K shapes (M <= 64, N < 16384, K >= 2048) take 64x64 tiles above M = 32; without a
    # device the name carries no "_splitk" (the split count depends on the CU count)
    assert sp(_hip.OP_W8A16, 64, 4096, 12288) == "dma_mfma_f16x_64x64"
    assert sp(_hip.OP_W8A8, 48, 4096, 4096) == "dma_mfma_i8_64x64"
    assert sp(_hip.OP_W8A16, 32, 4096, 4096) == "dma_mfma_f16x_32x64"
    assert sp(_hip.OP_W8A8, 17, 6144, 1024) == "dma_mfma_i8_32x64"
    assert sp(_hip.OP_W8A8, 64, 24576, 4096) == "dma_mfma_i8_64x128"     # wide N
    assert sp(_hip.OP_W8A16, 64, 24576, 4096) == "dma_mfma_f16x_64x128w8"
    assert sp(_hip.OP_W8A8, 16, 24576, 4096) == "dma_mfma_i8_32x64"     # 8 < M <= 16, >= 24 Mi weights
    assert sp(_hip.OP_W8A8, 16, 16384, 1024) == "stream_mfma_i8_m16"    # wide N, smaller weights
    assert sp(_hip.OP_W8A16, 12, 4096, 4096) == "skinny_mfma_f16x_m16"
    assert sp(_hip.OP_W8A8, 64, 6144, 1040) == "skinny_mfma_i8_m64"     # K % 128 != 0 keeps skinny
    assert sp(_hip.OP_W8A8, 8, 24576, 4096) == "skinny_mfma_i8_m16"     # M <= 8
    assert sp(_hip.OP_W8A8, 16, 24576, 4160) == "skinny_mfma_i8_m16"    # K % 256 != 0
    assert sp(_hip.OP_W8A8, 256, 4096, 1024) == "dma_mfma_i8_64x64"     # 64x64 tiles fill the CUs
    assert sp(_hip.OP_W8A8, 192, 4096, 1024) == "dma_mfma_i8_32x64"
    assert sp(_hip.OP_W8A8, 8192, 1024, 3072) == "dma_mfma_i8_256x128"
    assert sp(_hip.OP_W8A8, 8192, 6144, 1024) == "dma_mfma_i8_256x256"
    assert sp(_hip.OP_W8A16, 8192, 1024, 3072) == "dma_mfma_f16x_128x256"
    assert sp(_hip.OP_W8A8, 300, 1000, 1040).startswith("tiled_")         # K % 128 != 0
    assert sp(_hip.OP_W8A8, 8, 33, 40) == "generic_simt"
    with pytest.raises(RuntimeError):
        sp(9, 1, 1, 1)


def test_select_path_opt_in_switches(hiplib, monkeypatch):
    """TVQ_PREFILL_W4 swaps the 8-wave prefill tiles for the 4-wave ones;
    TVQ_STREAMK moves decode-size DMA shapes onto the widest decode tiles
    (the "_streamk" suffix needs a device: it depends on the CU count)."""
    from nanovllm.quantization import _hip
    sp = _hip.select_path
    monkeypatch.setenv("TVQ_PREFILL_W4", "1")
    assert sp(_hip.OP_W8A8, 8192, 6144, 1024) == "dma_mfma_i8_256x256w4"
    assert sp(_hip.OP_W8A16, 8192, 1024, 3072) == "dma_mfma_f16x_128x256w4"
    assert sp(_hip.OP_W8A8, 8192, 1024, 3072) == "dma_mfma_i8_256x128"     # fewer than 256 such tiles
    assert sp(_hip.OP_W8A8, 256, 4096, 1024) == "dma_mfma_i8_64x64"        # decode sizes unchanged
    monkeypatch.delenv("TVQ_PREFILL_W4")
    monkeypatch.setenv("TVQ_STREAMK", "1")
    assert sp(_hip.OP_W8A16, 64, 4096, 12288) == "dma_mfma_f16x_64x256"     # instead of split-K 64x64
    assert sp(_hip.OP_W8A16, 64, 24576, 4096) == "dma_mfma_f16x_64x256"     # instead of 64x128w8
    assert sp(_hip.OP_W8A8, 48, 4096, 4096) == "dma_mfma_i8_64x128"
    assert sp(_hip.OP_W8A16, 32, 4096, 4096) == "dma_mfma_f16x_32x256"
    assert sp(_hip.OP_W8A16, 17, 4096, 4096) == "dma_mfma_f16x_32x256"
    assert sp(_hip.OP_W8A8, 16, 24576, 4096) == "dma_mfma_i8_32x64"
    assert sp(_hip.OP_W8A8, 256, 4096, 1024) == "dma_mfma_i8_64x64"        # M > 64 unchanged
    assert sp(_hip.OP_W8A16, 1, 4096, 1024) == "gemv_dot2_f16x"            # the GEMV keeps M <= 2
    assert sp(_hip.OP_W8A16, 16, 4096, 1024) == "dma_mfma_f16x_16x128"     # M <= 16: 16-row tiles
    assert sp(_hip.OP_W8A16, 3, 24576, 4096) == "dma_mfma_f16x_16x128"
    assert sp(_hip.OP_W8A8, 8, 24576, 4096) == "dma_mfma_i8_32x64"
    assert sp(_hip.OP_W8A8, 8, 4096, 1040) == "skinny_mfma_i8_m16"        # K % 128 != 0 keeps skinny


# ------------------------------------------------------------------ Python API

class _Layer(torch.nn.Module):
    pass


def test_quant_method_parameters_match_reference_layout():
    from nanovllm.quantization import Int8WeightOnlyQuantMethod, W8A8QuantMethod
    lay = _Layer()
    Int8WeightOnlyQuantMethod().create_weights(lay, 1024, 4096)
    assert lay.qweight.dtype == torch.int8 and tuple(lay.qweight.shape) == (4096, 1024)
    assert lay.scales.dtype == torch.float32 and tuple(lay.scales.shape) == (4096,)
    assert not lay.qweight.requires_grad and not lay.scales.requires_grad
    assert Int8WeightOnlyQuantMethod().quantize_activation(torch.zeros(2, 4)) is None
    lay2 = _Layer()
    W8A8QuantMethod().create_weights(lay2, 3072, 1024)
    assert lay2.qweight.dtype == torch.int8 and tuple(lay2.qweight.shape) == (1024, 3072)
    assert lay2.w_scales.dtype == torch.float32 and tuple(lay2.w_scales.shape) == (1024,)
    assert not hasattr(lay2, "scales")


def _cpu_layer(method, n, k, seed=0):
    x = torch.randn(3, 5, k, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(seed + 1)) * 0.02).to(torch.bfloat16)
    q, s = oracle.quantize_rows(w.float().numpy())
    lay = _Layer()
    method.create_weights(lay, k, n)
    lay.qweight.data.copy_(torch.from_numpy(q))
    getattr(lay, "scales", getattr(lay, "w_scales", None)).data.copy_(torch.from_numpy(s))
    lay.bias = None
    return lay, x, torch.from_numpy(q), torch.from_numpy(s)


def test_cpu_tensors_take_reference_torch_path_and_log(monkeypatch, capsys):
    from nanovllm.quantization import Int8WeightOnlyQuantMethod, W8A8QuantMethod, cuda
    monkeypatch.setenv("NANOVLLM_INT8_LOG_PATH", "1")
    monkeypatch.setenv("NANOVLLM_W8A8_LOG_PATH", "1")
    cuda._LOGGED_KERNEL_EVENTS.clear()
    lay, x, q, s = _cpu_layer(Int8WeightOnlyQuantMethod(), 64, 128)
    y = Int8WeightOnlyQuantMethod().apply(x, lay)
    assert tuple(y.shape) == (3, 5, 64) and y.dtype == torch.bfloat16
    assert torch.equal(y, oracle.w8a16_torch_path(x, q, s))
    lay8, x8, q8, s8 = _cpu_layer(W8A8QuantMethod(), 64, 128, seed=3)
    y8 = W8A8QuantMethod().apply(x8, lay8)
    xq, a_s = oracle.quantize_rows_torch(x8.reshape(-1, 128))
    ref = oracle.w8a8_torch_path(xq, a_s, q8, s8, None, torch.bfloat16).view(3, 5, 64)
    assert torch.equal(y8, ref)
    out = capsys.readouterr().out.strip().splitlines()
    assert out[0].startswith("[nanovllm.int8] backend=fallback phase=decode path=python_fallback "
                             "x_dtype=torch.bfloat16 x_shape=(3, 5, 128) qweight_shape=(64, 128)")
    assert out[0].endswith("reason=cpu_tensors")
    assert out[1].startswith("[nanovllm.w8a8] backend=fallback phase=decode path=python_fallback "
                             "out_dtype=torch.bfloat16 x_q_shape=(15, 128) qweight_shape=(64, 128)")
    # one-shot: the same event is not logged twice
    Int8WeightOnlyQuantMethod().apply(x, lay)
    assert capsys.readouterr().out == ""


def test_backend_env_parsing(monkeypatch):
    from nanovllm.quantization import cuda
    for val, want in (("native", "native"), ("FALLBACK", "fallback"), (" cutlass ", "cutlass"), ("auto", "auto"),
                      ("bogus", "native"), ("", "native")):
        monkeypatch.setenv("NANOVLLM_INT8_BACKEND", val)
        assert cuda._get_backend_preference() == want
    for val, want in (("native", "native"), ("fallback", "fallback"), ("cutlass", "native")):
        monkeypatch.setenv("NANOVLLM_W8A8_BACKEND", val)
        assert cuda._get_w8a8_backend_preference() == want
    for val, want in (("", False), ("0", False), ("off", False), ("1", True), ("yes", True)):
        monkeypatch.setenv("NANOVLLM_INT8_LOG_PATH", val)
        assert cuda._should_log_kernel_path() is want


def test_forced_fallback_logs_reason(monkeypatch, capsys):
    from nanovllm.quantization import cuda
    monkeypatch.setenv("NANOVLLM_INT8_BACKEND", "fallback")
    monkeypatch.setenv("NANOVLLM_INT8_LOG_PATH", "1")
    cuda._LOGGED_KERNEL_EVENTS.clear()
    from nanovllm.utils.context import step_context
    with step_context(True):
        lay, x, q, s = _cpu_layer(__import__("nanovllm.quantization", fromlist=["x"]).Int8WeightOnlyQuantMethod(),
                                  32, 64)
        cuda.apply_int8_weight_only_linear(x, lay.qweight, lay.scales)
    line = capsys.readouterr().out.strip()
    assert "backend=fallback phase=prefill path=python_fallback" in line
    assert line.endswith("reason=backend_forced_fallback")


def test_native_entry_points_refuse_cpu_tensors():
    """The native path never silently computes on the CPU."""
    from nanovllm.quantization import cuda
    lay, x, q, s = _cpu_layer(__import__("nanovllm.quantization", fromlist=["x"]).Int8WeightOnlyQuantMethod(), 32, 64)
    with pytest.raises(RuntimeError):
        cuda.native_int8_weight_only_linear(x, q, s)
    xq, a_s = oracle.quantize_rows_torch(x.reshape(-1, 64))
    with pytest.raises(RuntimeError):
        cuda.native_w8a8_linear(xq, a_s, q, s, None, torch.bfloat16)


def test_validation_messages_match_reference():
    from nanovllm.quantization import cuda
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    q = torch.zeros(8, 32, dtype=torch.int8)
    s = torch.zeros(8)
    with pytest.raises(RuntimeError, match="Incompatible shapes"):
        cuda.native_int8_weight_only_linear(x, q, s)
    with pytest.raises(RuntimeError, match="scales must be 1D"):
        cuda.native_int8_weight_only_linear(x[:, :32], q, torch.zeros(7))
    with pytest.raises(RuntimeError, match="bias must be 1D"):
        cuda.native_int8_weight_only_linear(x[:, :32], q, s, torch.zeros(3))
    xq = torch.zeros(2, 32, dtype=torch.int8)
    with pytest.raises(RuntimeError, match="a_scales must be 1D"):
        cuda.native_w8a8_linear(xq, torch.zeros(3), q, s, None, torch.bfloat16)
    with pytest.raises(RuntimeError, match="output dtype"):
        cuda.native_w8a8_linear(xq, torch.zeros(2), q, s, None, torch.float32)


def test_utils_quantizers_match_oracle():
    from nanovllm.quantization.utils import (is_qwen3_int8_target_weight, quantize_int8_per_channel,
                                             quantize_int8_per_row_dynamic)
    w = (torch.randn(64, 256, generator=torch.Generator().manual_seed(1)) * 0.02).to(torch.bfloat16)
    q, s = quantize_int8_per_channel(w)
    q_o, s_o = oracle.quantize_rows(w.float().numpy())
    np.testing.assert_array_equal(q.numpy(), q_o)
    np.testing.assert_array_equal(s.numpy(), s_o)
    q2, s2 = quantize_int8_per_row_dynamic(w)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    assert is_qwen3_int8_target_weight("model.layers.0.mlp.down_proj.weight")
    assert not is_qwen3_int8_target_weight("model.layers.0.input_layernorm.weight")


def test_prefill_block_size_matches_header():
    """The host block table and the kernel agree on the query block size."""
    import re
    from pathlib import Path
    from nanovllm.quantization import _hip
    hdr = (Path(__file__).resolve().parents[1] / "include" / "tvq.h").read_text()
    assert int(re.search(r"#define TVQ_PREFILL_BLOCK_Q (\d+)", hdr).group(1)) == _hip.PREFILL_BLOCK_Q
    rows = _hip.prefill_blocks([(0, 130), (130, 64)]).tolist()
    assert sorted(r[2] for r in rows if r[0] == 0) == list(range(0, 130, _hip.PREFILL_BLOCK_Q))


def test_glu_interleave_layout():
    """Row 64b + 32h + k of the regrouped gate_up weights is old row h*I + 32b + k."""
    from nanovllm.quantization import _hip
    i, k = 96, 8
    qw = torch.arange(2 * i * k, dtype=torch.int32).view(2 * i, k).to(torch.int8)
    rows = torch.arange(2 * i, dtype=torch.float32)
    q2, s2 = _hip.glu_interleave(qw, rows)
    for b in range(i // 32):
        for h in range(2):
            for kk in range(32):
                assert s2[64 * b + 32 * h + kk].item() == h * i + 32 * b + kk
    assert torch.equal(q2, qw[s2.long()])
    with pytest.raises(Exception):
        _hip.glu_interleave(qw[:96], rows[:96])


def _pretend_native(monkeypatch, cuda):
    """Route CPU tensors into the native branch, whose call then raises."""
    monkeypatch.setattr(cuda, "_on_gpu", lambda *t: True)
    monkeypatch.setattr(cuda._hip, "load_library", lambda: None)

    def boom(*a, **k):
        raise RuntimeError("tvq_w8a16_gemm failed (code -2): unsupported")
    monkeypatch.setattr(cuda, "native_int8_weight_only_linear", boom)
    monkeypatch.setattr(cuda, "native_w8a8_linear", boom)


def test_native_failure_falls_back_like_reference(monkeypatch, capsys):
    """Default dispatch (reference cuda.py:344-356, 487-503): a native failure is
    logged once as native_unavailable and the torch path computes the result."""
    from nanovllm.quantization import cuda, Int8WeightOnlyQuantMethod
    monkeypatch.delenv("NANOVLLM_NATIVE_STRICT", raising=False)
    monkeypatch.setenv("NANOVLLM_INT8_LOG_PATH", "1")
    monkeypatch.setenv("NANOVLLM_W8A8_LOG_PATH", "1")
    monkeypatch.setenv("NANOVLLM_INT8_BACKEND", "native")
    monkeypatch.setenv("NANOVLLM_W8A8_BACKEND", "native")
    cuda._LOGGED_KERNEL_EVENTS.clear()
    _pretend_native(monkeypatch, cuda)
    lay, x, q, s = _cpu_layer(Int8WeightOnlyQuantMethod(), 32, 64)
    y = cuda.apply_int8_weight_only_linear(x, q, s)
    assert torch.equal(y, cuda.int8_weight_only_linear_fallback(x, q, s))
    xq, a_s = oracle.quantize_rows_torch(x.reshape(-1, 64))
    y8 = cuda.apply_w8a8_linear(xq, a_s, q, s, None, torch.bfloat16)
    assert torch.equal(y8, cuda.w8a8_linear_fallback(xq, a_s, q, s, None, torch.bfloat16))
    out = capsys.readouterr().out.strip().splitlines()
    assert len(out) == 2
    assert all("backend=fallback" in l and "path=python_fallback" in l for l in out)
    assert all("reason=native_unavailable RuntimeError: tvq_w8a16_gemm failed" in l for l in out)


def test_strict_switch_reraises_native_failure(monkeypatch):
    """NANOVLLM_NATIVE_STRICT=1 (set by tests, smoke and bench) re-raises."""
    from nanovllm.quantization import cuda, Int8WeightOnlyQuantMethod
    monkeypatch.setenv("NANOVLLM_NATIVE_STRICT", "1")
    monkeypatch.setenv("NANOVLLM_INT8_BACKEND", "native")
    monkeypatch.setenv("NANOVLLM_W8A8_BACKEND", "native")
    _pretend_native(monkeypatch, cuda)
    lay, x, q, s = _cpu_layer(Int8WeightOnlyQuantMethod(), 32, 64)
    with pytest.raises(RuntimeError, match="unsupported"):
        cuda.apply_int8_weight_only_linear(x, q, s)
    xq, a_s = oracle.quantize_rows_torch(x.reshape(-1, 64))
    with pytest.raises(RuntimeError, match="unsupported"):
        cuda.apply_w8a8_linear(xq, a_s, q, s, None, torch.bfloat16)


def test_missing_library_is_never_hidden(monkeypatch):
    """A missing HIP library raises even without the strict switch."""
    from nanovllm.quantization import cuda, Int8WeightOnlyQuantMethod
    monkeypatch.delenv("NANOVLLM_NATIVE_STRICT", raising=False)
    monkeypatch.setenv("NANOVLLM_INT8_BACKEND", "native")
    monkeypatch.setattr(cuda, "_on_gpu", lambda *t: True)
    monkeypatch.setattr(cuda._hip, "_LIB", None)
    monkeypatch.setenv("TVQ_LIBRARY", "/nonexistent/libtinyvllm_quant.so")
    lay, x, q, s = _cpu_layer(Int8WeightOnlyQuantMethod(), 32, 64)
    with pytest.raises(RuntimeError, match="not found"):
        cuda.apply_int8_weight_only_linear(x, q, s)


def test_noalloc_linear_rejects_sizes_beyond_its_scratch(hiplib):
    """The size limits are checked before any device work (no GPU needed)."""
    big_k = 1024
    m = (8 << 20) // big_k + 1  # one row past TVQ_NOALLOC_MAX_XQ_BYTES
    rc = hiplib.tvq_w8a8_linear_noalloc(None, 1, None, None, None, None, m, 64, big_k, None)
    assert rc == -2
    assert b"scratch maximum" in hiplib.tvq_last_error()
    rc = hiplib.tvq_w8a8_linear_noalloc(None, 1, None, None, None, None, 65537, 64, 16, None)
    assert rc == -2
    assert hiplib.tvq_w8a8_linear_noalloc(None, 1, None, None, None, None, -1, 64, 16, None) == -1


def test_rounded_dequant_switch(monkeypatch):
    """NANOVLLM_INT8_DEQUANT_ROUNDING selects the reference kernel's rounding
    only for 'reference' / 'activation'; anything else keeps the fp32 scale."""
    from nanovllm.quantization import cuda
    for value, want in (("reference", True), ("Activation", True), ("fp32", False), ("", False), ("bf16x", False)):
        monkeypatch.setenv("NANOVLLM_INT8_DEQUANT_ROUNDING", value)
        assert cuda._rounded_dequant() is want
    monkeypatch.delenv("NANOVLLM_INT8_DEQUANT_ROUNDING")
    assert cuda._rounded_dequant() is False
