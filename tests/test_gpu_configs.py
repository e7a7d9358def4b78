"""GPU parity at the benchmark configurations' exact shapes.

* config 1: W8A16 gate_up of Qwen3-0.6B, M=64, N=6144, K=1024, generated as
  the config states (seed 0, X ~ N(0,1), W ~ N(0,0.02) quantized per channel);
* config 2: the QKV shape N=4096, K=1024 at M in {1, 16, 64, 256, 512}, W8A8
  and W8A16, against the oracle (not the HIP path against itself);
* config 4: the four 8B-like projections at M in {1, 64, 512}, checked in
  full, and at M in {4096, 16384} on sampled rows (always the last one) plus
  the last output column of every row.

Bars: W8A8 int32 accumulators and bf16 outputs bit-exact against the oracle's
restatement of the reference kernel (w8a8_gemm.cu:336-390), and within rel-L2
<= 1e-2, max-abs <= 2e-2*max|ref| of the reference's torch path
(cuda.py:455-465) where that path is cheap enough on the CPU; W8A16 within the
same tolerance of its torch path (cuda.py:293-300) and within a bf16-rounding
bound of the exact product, evaluated with a float64 BLAS product.
"""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, f32, make_activations, make_weights

pytestmark = pytest.mark.gpu

QWEN8B = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096), "down": (4096, 12288)}


def _dev():
    return torch.device("cuda", 0)


def _log_case(**kw):
    print("CASE", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@functools.lru_cache(maxsize=2)
def _weights(n, k, seed):
    q, s = make_weights(n, k, seed=seed)
    return q, s, q.to(_dev()), s.to(_dev())


def _w8a8_check_rows(y_rows, x_rows, q, s, torch_path: bool):
    """y_rows (CPU bf16) of tvq_w8a8_linear against the oracle on x_rows."""
    xq, a_s = oracle.c_act_quant(bits16(x_rows))
    acc = oracle.gemm_i32_blas(xq, q.numpy())
    yb_ref, _ = oracle.c_w8a8_epilogue(acc, a_s, s.numpy())
    np.testing.assert_array_equal(bits16(y_rows), yb_ref)
    if torch_path:
        ref = oracle.w8a8_torch_path(torch.from_numpy(xq), torch.from_numpy(a_s), q, s, None, torch.bfloat16)
        assert oracle.rel_l2(f32(y_rows), f32(ref)) <= oracle.REL_L2_TOL
        assert oracle.max_abs_ratio(f32(y_rows), f32(ref)) <= oracle.MAX_ABS_TOL


def _w8a16_check_rows(y_rows, x_rows, q, s, torch_path: bool):
    """Bound vs the exact product (float64 BLAS) and, optionally, tolerance vs
    the reference's torch path."""
    xf = f32(x_rows).astype(np.float64)
    qf = q.numpy().astype(np.float64)
    sd = s.numpy().astype(np.float64)[None, :]
    y64 = (xf @ qf.T) * sd
    mag = (np.abs(xf) @ np.abs(qf).T) * sd
    k = x_rows.shape[1]
    bound = np.abs(y64) * 2.0 ** -8 + mag * (k * 2.0 ** -23) + 1e-30
    err = np.abs(f32(y_rows).astype(np.float64) - y64)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"
    assert oracle.rel_l2(f32(y_rows), y64) <= oracle.REL_L2_TOL
    if torch_path:
        ref = oracle.w8a16_torch_path(x_rows, q, s)
        assert oracle.rel_l2(f32(y_rows), f32(ref)) <= oracle.REL_L2_TOL
        assert oracle.max_abs_ratio(f32(y_rows), f32(ref)) <= oracle.MAX_ABS_TOL


# ---------------------------------------------------------------- config 1

def test_config1_w8a16_gate_up_m64_exact_recipe(hiplib):
    """Config 1 exactly as BASELINE states it: torch.manual_seed(0); X bf16
    [64,1024] ~ N(0,1); W bf16 [6144,1024] ~ N(0,0.02) -> per-channel int8."""
    from nanovllm.quantization import _hip
    m, n, k = 64, 6144, 1024
    _log_case(test="config1", m=m, n=n, k=k, path=_hip.select_path(_hip.OP_W8A16, m, n, k))
    torch.manual_seed(0)
    x = torch.randn(m, k).to(torch.bfloat16)
    w = (torch.randn(n, k) * 0.02).to(torch.bfloat16)
    q_np, s_np = oracle.quantize_rows(f32(w))
    q, s = torch.from_numpy(q_np), torch.from_numpy(s_np)
    y = _hip.w8a16_gemm(x.to(_dev()), q.to(_dev()), s.to(_dev()))
    _w8a16_check_rows(y.cpu(), x, q, s, torch_path=True)
    # the C restatement of the exact product agrees as well
    y64 = oracle.c_w8a16_f64(bits16(x), q_np, s_np)
    assert oracle.rel_l2(f32(y.cpu()), y64) < 4e-3


# ---------------------------------------------------------------- config 2

@pytest.mark.parametrize("m", [1, 16, 64, 256, 512])
@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
def test_config2_qkv_sweep(hiplib, mode, m):
    """The QKV shape with the config's 1 % outlier columns x20, every M of
    the decode-batch sweep, against the oracle."""
    from nanovllm.quantization import _hip
    n, k = 4096, 1024
    op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
    _log_case(test="config2", mode=mode, m=m, path=_hip.select_path(op, m, n, k))
    x = make_activations(m, k, seed=1000 + m)
    q, s, qd, sd = _weights(n, k, 77)
    if mode == "w8a8":
        y = _hip.w8a8_linear(x.to(_dev()), qd, sd).cpu()
        _w8a8_check_rows(y, x, q, s, torch_path=True)
        # the int32 accumulator itself, through the same path selection
        xq, _ = oracle.c_act_quant(bits16(x))
        acc = _hip.w8a8_gemm_i32(torch.from_numpy(xq).to(_dev()), qd)
        np.testing.assert_array_equal(acc.cpu().numpy(), oracle.c_gemm_i32(xq, q.numpy()))
    else:
        y = _hip.w8a16_gemm(x.to(_dev()), qd, sd).cpu()
        _w8a16_check_rows(y, x, q, s, torch_path=True)


# ---------------------------------------------------------------- config 4

@pytest.mark.parametrize("m", [1, 64, 512])
@pytest.mark.parametrize("proj", list(QWEN8B))
@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
def test_config4_8b_decode_full(hiplib, mode, proj, m):
    """All four 8B-like projections at decode/mid M, every output checked."""
    from nanovllm.quantization import _hip
    n, k = QWEN8B[proj]
    op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
    _log_case(test="config4", mode=mode, proj=proj, m=m, path=_hip.select_path(op, m, n, k))
    x = make_activations(m, k, seed=n + k + m, outlier_frac=0.01 if mode == "w8a8" else 0.0)
    q, s, qd, sd = _weights(n, k, n + k)
    if mode == "w8a8":
        y = _hip.w8a8_linear(x.to(_dev()), qd, sd).cpu()
        _w8a8_check_rows(y, x, q, s, torch_path=m <= 64)
    else:
        y = _hip.w8a16_gemm(x.to(_dev()), qd, sd).cpu()
        _w8a16_check_rows(y, x, q, s, torch_path=m <= 64)


@pytest.mark.parametrize("m", [4096, 16384])
@pytest.mark.parametrize("proj", list(QWEN8B))
@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
def test_config4_8b_prefill_sampled(hiplib, mode, proj, m):
    """The 8B-like projections at prefill M: 24 sampled rows plus the first and
    last, every column; and the last output column of every row."""
    from nanovllm.quantization import _hip
    n, k = QWEN8B[proj]
    op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
    _log_case(test="config4_prefill", mode=mode, proj=proj, m=m, path=_hip.select_path(op, m, n, k))
    x = make_activations(m, k, seed=n + k + m, outlier_frac=0.01 if mode == "w8a8" else 0.0)
    q, s, qd, sd = _weights(n, k, n + k)
    rows = np.unique(np.concatenate([np.random.default_rng(m + n).choice(m, 24, replace=False), [0, m - 1]]))
    ridx = torch.from_numpy(rows)
    xd = x.to(_dev())
    y = _hip.w8a8_linear(xd, qd, sd) if mode == "w8a8" else _hip.w8a16_gemm(xd, qd, sd)
    del xd
    y_rows = y[ridx.to(_dev())].cpu()
    y_col = y[:, -1:].cpu()
    del y
    assert torch.isfinite(y_rows.float()).all()
    if mode == "w8a8":
        _w8a8_check_rows(y_rows, x[ridx], q, s, torch_path=False)
        _w8a8_check_rows(y_col, x, q[-1:], s[-1:], torch_path=False)
    else:
        _w8a16_check_rows(y_rows, x[ridx], q, s, torch_path=False)
        _w8a16_check_rows(y_col, x, q[-1:], s[-1:], torch_path=False)
