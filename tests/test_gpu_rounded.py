"""GPU parity of the W8A16 rounded-dequant mode (tvq_w8a16_gemm_rounded) and
the operand-floor measurement entry (tvq_gemm_operand_floor).

Rounded dequant reproduces the reference kernel's rounding
(int8_weight_only_gemm.cu:397-413, the same expression as the torch path,
cuda.py:293-300): each weight becomes wd = T(T(q) * T(s)) before an fp32 dot
product, and the epilogue adds only the bias. Bars:
* against the exact float64 product x @ wd^T + b (oracle.w8a16_rounded_f64 on
  oracle.w8a16_rounded_weights): within one rounding of the output type plus
  the fp32 summation bound K * 2^-23 * sum|x * wd|;
* against the reference's torch path run by CPU torch (oracle.w8a16_torch_path):
  within the same bound doubled (both sides reassociate the fp32 sum), and
  within rel-L2 <= 1e-2, max-abs <= 2e-2 * max|ref|.
Shapes cover every DMA tile configuration (K % 128 == 0), the generic kernel
(K % 128 != 0, an unaligned view), bf16 and fp16, with and without bias.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import f32, make_activations, make_weights

pytestmark = pytest.mark.gpu


def _case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(y, x, q, s, bias, dtype, rows=None):
    is_bf = dtype == torch.bfloat16
    xs = x if rows is None else x[rows]
    ys = y if rows is None else y[rows]
    wd = oracle.w8a16_rounded_weights(q.numpy(), s.numpy(), is_bf16=is_bf)
    b = None if bias is None else f32(bias)
    y64 = oracle.w8a16_rounded_f64(f32(xs), wd, b)
    mag = np.abs(f32(xs)).astype(np.float64) @ np.abs(wd).astype(np.float64).T
    k = x.shape[1]
    ulp = 2.0 ** -8 if is_bf else 2.0 ** -11
    bound = np.abs(y64) * ulp + mag * (k * 2.0 ** -23) + 1e-30
    err = np.abs(f32(ys).astype(np.float64) - y64)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"
    ref = oracle.w8a16_torch_path(xs, q, s, bias)
    err_t = np.abs(f32(ys).astype(np.float64) - f32(ref).astype(np.float64))
    assert np.all(err_t <= 2 * bound + np.abs(y64) * ulp), f"max excess vs torch path {np.max(err_t - 2 * bound)}"
    assert oracle.rel_l2(f32(ys), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(ys), f32(ref)) <= oracle.MAX_ABS_TOL


SHAPES = [
    (1, 4096, 1024),      # 32x64 tiles
    (16, 6144, 1024),
    (64, 6144, 1024),     # config 1's shape
    (64, 24576, 1024),    # 64x128 (8 waves)
    (200, 1000, 384),     # ragged M and N, 64x64
    (300, 2048, 256),     # M > 256: 64x128
    (2048, 1024, 1024),   # 128x256
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_rounded_dequant_dma_tiles(gpu, hiplib, m, n, k, dtype):
    from nanovllm.quantization import _hip
    _case(test="rounded_dma", m=m, n=n, k=k, dtype=dtype)
    x = make_activations(m, k, seed=m + n, dtype=dtype, outlier_frac=0.0)
    q, s = make_weights(n, k, seed=k)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(3)) * 0.1).to(dtype) if m % 2 == 0 else None
    y = _hip.w8a16_gemm_rounded(x.to(gpu), q.to(gpu), s.to(gpu), None if bias is None else bias.to(gpu)).cpu()
    rows = None if m <= 256 else np.r_[0:64, m - 64:m]
    _check(y, x, q, s, bias, dtype, rows)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,n,k", [(7, 96, 40), (33, 130, 80), (5, 64, 1000)])
def test_rounded_dequant_generic(gpu, hiplib, m, n, k, dtype):
    from nanovllm.quantization import _hip
    _case(test="rounded_generic", m=m, n=n, k=k, dtype=dtype)
    x = make_activations(m, k, seed=k, dtype=dtype, outlier_frac=0.0)
    q, s = make_weights(n, k, seed=n)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(4)) * 0.1).to(dtype)
    y = _hip.w8a16_gemm_rounded(x.to(gpu), q.to(gpu), s.to(gpu), bias.to(gpu)).cpu()
    _check(y, x, q, s, bias, dtype)


def test_rounded_dequant_unaligned_view(gpu, hiplib):
    """A contiguous view 2 bytes into its storage takes the generic kernel."""
    from nanovllm.quantization import _hip
    _case(test="rounded_unaligned")
    m, n, k = 9, 256, 1024
    xb = make_activations(m * k + 1, 1, seed=2, dtype=torch.bfloat16, outlier_frac=0.0).view(-1)
    q, s = make_weights(n, k, seed=9)
    xg = xb.to(gpu)[1:].view(m, k)
    assert xg.data_ptr() % 16 != 0
    y = _hip.w8a16_gemm_rounded(xg, q.to(gpu), s.to(gpu)).cpu()
    _check(y, xb[1:].view(m, k), q, s, None, torch.bfloat16)


def test_rounded_dequant_through_dispatch(gpu, hiplib, monkeypatch):
    """NANOVLLM_INT8_DEQUANT_ROUNDING=reference routes apply_int8_weight_only_linear
    to the rounded kernel; the default keeps the fp32-scale kernels."""
    from nanovllm.quantization import _hip
    from nanovllm.quantization.cuda import apply_int8_weight_only_linear
    _case(test="rounded_dispatch")
    x = make_activations(6, 1024, seed=1, dtype=torch.bfloat16, outlier_frac=0.0).view(3, 2, 1024)
    q, s = make_weights(512, 1024, seed=2)
    xg, qg, sg = x.to(gpu), q.to(gpu), s.to(gpu)
    monkeypatch.setenv("NANOVLLM_INT8_DEQUANT_ROUNDING", "reference")
    y_r = apply_int8_weight_only_linear(xg, qg, sg)
    assert y_r.shape == (3, 2, 512)
    assert torch.equal(y_r.view(6, 512), _hip.w8a16_gemm_rounded(xg.view(6, 1024), qg, sg))
    monkeypatch.setenv("NANOVLLM_INT8_DEQUANT_ROUNDING", "fp32")
    y_f = apply_int8_weight_only_linear(xg, qg, sg)
    assert torch.equal(y_f.view(6, 512), _hip.w8a16_gemm(xg.view(6, 1024), qg, sg))
    _check(y_r.view(6, 512).cpu(), x.view(6, 1024), q, s, None, torch.bfloat16)


@pytest.mark.parametrize("op,m,n,k", [(2, 256, 4096, 1024), (2, 8192, 1024, 3072), (2, 64, 24576, 1024),
                                      (1, 64, 6144, 1024), (1, 4096, 1024, 1024)])
def test_operand_floor_runs_and_writes_nothing(gpu, hiplib, op, m, n, k):
    """The measurement entry launches the tiles' operand stream only: it
    returns OK, leaves a guard buffer after the operands untouched and rejects
    shapes the DMA tiles cannot take."""
    from nanovllm.quantization import _hip
    _case(test="operand_floor", op=op, m=m, n=n, k=k)
    dt = torch.int8 if op == 2 else torch.bfloat16
    x = torch.ones(m, k, dtype=dt, device=gpu)
    q = torch.ones(n, k, dtype=torch.int8, device=gpu)
    guard = torch.full((1 << 16,), 7, dtype=torch.int32, device=gpu)
    _hip.gemm_operand_floor(op, x, q)
    torch.cuda.synchronize()
    assert torch.all(guard == 7)
    with pytest.raises(RuntimeError, match="K % 128"):
        _hip.gemm_operand_floor(op, torch.ones(m, 96, dtype=dt, device=gpu), torch.ones(n, 96, dtype=torch.int8,
                                                                                           device=gpu))
