"""GPU parity of the fused producer kernels (tvq_rmsnorm, tvq_silu_mul)
against the oracle (oracle.rmsnorm_ref / silu_mul_ref, which restate
layernorm.py:16-40 and activation.py:11-14).

Bar:
  * new residual (x + residual rounded): bit-exact;
  * y: bit-exact on >= 99 % of elements and otherwise one rounding flip
    away from the oracle (the device takes fp32 statistics and expf where
    the oracle uses fp64): within 1 ulp for silu_mul, 2 ulps for rmsnorm,
    whose first rounding is then scaled by the weight (< 2);
  * fused int8 codes and scales: bit-exact against act-quant of the kernel's
    own y (tvq_act_quant and the oracle's quantize_rows), i.e. exactly what
    the reference's W8A8QuantMethod.quantize_activation would produce from
    that y; the quant-only and y-only variants give the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import f32, make_activations

pytestmark = pytest.mark.gpu


def _log_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _ulp(ref: np.ndarray, dtype) -> np.ndarray:
    mant = 7 if dtype == torch.bfloat16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(ref), 1e-30)))
    sub = -126 if dtype == torch.bfloat16 else -14
    return np.exp2(np.maximum(e, sub) - mant)


def _check_y(y: torch.Tensor, ref: np.ndarray, dtype, ulps: float = 1.0):
    got = f32(y)
    diff = np.abs(got - ref)
    assert np.all(diff <= _ulp(ref, dtype) * ulps * 1.0001), float(diff.max())
    assert np.mean(got == ref) >= 0.99


def _check_codes(y: torch.Tensor, q):
    from nanovllm.quantization import _hip
    xq, s = q
    rq, rs = _hip.act_quant(y)
    assert torch.equal(xq, rq) and torch.equal(s, rs)
    oq, os_ = oracle.quantize_rows(f32(y))
    np.testing.assert_array_equal(xq.cpu().numpy(), oq)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


def _placed(t: torch.Tensor, misalign: bool) -> torch.Tensor:
    """t on the GPU, optionally at an address that is not 16-byte aligned."""
    if not misalign:
        return t.cuda()
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device="cuda")
    out = buf[1:].view(t.shape)
    out.copy_(t.cuda())
    return out


# M picks the threads per row: < 512 four waves, 512..1023 two waves, >= 1024 one wave
RMS_SHAPES = [(1, 1024), (7, 1024), (300, 1024), (64, 128), (33, 4096), (4, 2048), (5, 5000), (9, 1003), (1, 8),
              (600, 2048), (513, 4096), (1030, 1024), (1500, 3072)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", RMS_SHAPES)
@pytest.mark.parametrize("with_res", [False, True])
def test_rmsnorm(hiplib, shape, dtype, with_res):
    from nanovllm.quantization import _hip
    m, k = shape
    _log_case(test="rmsnorm", m=m, k=k, dtype=dtype, res=with_res)
    x = make_activations(m, k, seed=m * 7 + k, dtype=dtype)
    r = make_activations(m, k, seed=m * 11 + k + 1, dtype=dtype, outlier_frac=0.0) if with_res else None
    w = (torch.rand(k, generator=torch.Generator().manual_seed(k)) + 0.5).to(dtype)
    if m >= 3:
        x[1].zero_()
        if r is not None:
            r[1].zero_()           # all-zero row: y = 0, scale = eps
    eps = 1e-6
    y_ref, res_ref = oracle.rmsnorm_ref(f32(x), f32(w), eps, None if r is None else f32(r),
                                        is_bf16=dtype == torch.bfloat16)
    misalign = k % 8 != 0 or k > 4096
    xd, wd = _placed(x, misalign), w.cuda()
    rd = _placed(r, misalign) if r is not None else None
    y, q = _hip.rmsnorm(xd, wd, eps, rd, out=True, quant=True)
    torch.cuda.synchronize()
    _check_y(y, y_ref, dtype, ulps=2.0)  # a flip in the first rounding, scaled by w < 2
    if r is not None:
        np.testing.assert_array_equal(f32(rd), res_ref)
    _check_codes(y, q)
    # quant-only and y-only variants agree bit for bit (residual re-supplied)
    rd2 = _placed(r, misalign) if r is not None else None
    _, q2 = _hip.rmsnorm(xd, wd, eps, rd2, out=False, quant=True)
    rd3 = _placed(r, misalign) if r is not None else None
    y3, _ = _hip.rmsnorm(xd, wd, eps, rd3, out=True, quant=False)
    assert torch.equal(q2[0], q[0]) and torch.equal(q2[1], q[1]) and torch.equal(y3, y)
    if r is not None:
        assert torch.equal(rd2, rd) and torch.equal(rd3, rd)


SILU_SHAPES = [(1, 3072), (64, 3072), (513, 3072), (16, 768), (3, 4096), (5, 6000), (7, 1003), (2, 8),
               (1030, 3072), (700, 1024)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SILU_SHAPES)
def test_silu_mul(hiplib, shape, dtype):
    from nanovllm.quantization import _hip
    m, i = shape
    _log_case(test="silu_mul", m=m, i=i, dtype=dtype)
    gu = make_activations(m, 2 * i, seed=m * 3 + i, dtype=dtype, outlier_frac=0.0) * 3
    if m >= 2:
        gu[1].zero_()
    ref = oracle.silu_mul_ref(f32(gu), is_bf16=dtype == torch.bfloat16)
    g = _placed(gu, i % 8 != 0 or i > 4096)
    y, q = _hip.silu_mul(g, out=True, quant=True)
    torch.cuda.synchronize()
    _check_y(y, ref, dtype)
    _check_codes(y, q)
    _, q2 = _hip.silu_mul(g, out=False, quant=True)
    y3, _ = _hip.silu_mul(g, out=True, quant=False)
    assert torch.equal(q2[0], q[0]) and torch.equal(q2[1], q[1]) and torch.equal(y3, y)


def test_rmsnorm_prefill_size_bandwidth_sanity(hiplib):
    """Full prefill size (M=8192, K=1024, residual + codes): properties only."""
    from nanovllm.quantization import _hip
    m, k = 8192, 1024
    x = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    r = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(k, device="cuda", dtype=torch.bfloat16)
    r0 = r.clone()
    y, q = _hip.rmsnorm(x, w, 1e-6, r, out=True, quant=True)
    assert torch.equal(r, (x.float() + r0.float()).bfloat16())
    rq, rs = _hip.act_quant(y)
    assert torch.equal(q[0], rq) and torch.equal(q[1], rs)
    # rows have unit RMS after normalisation (weight 1): mean(y^2) ~ 1
    ms = y.float().pow(2).mean(-1)
    assert torch.all((ms - 1).abs() < 2e-2)
