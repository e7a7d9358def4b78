"""BASELINE.json's GEMM configurations at their exact shapes, run through the
kernel sources on the CPU emulation (tests/cpu_emu) and the same C ABI as
on the GPU, checked against the oracle to the GPU tests' bar:

  cfg1  W8A16 gate_up, M=64, N=6144, K=1024
  cfg2  W8A8 qkv, N=4096, K=1024, M in {1, 16, 64, 256, 512}: act-quant
        codes / scales, int32 accumulators and bf16 outputs bit-exact
  cfg3  prefill M=8192 (16 ragged sequences of 100-1024 tokens, zero
        padding) for down (K=3072), o (K=2048) and gate_up (N=6144), W8A8 and
        W8A16: 48 sampled rows (and the last) exact / in bound, padding rows
        zero, every output finite
  cfg4  Qwen3-8B-like projections at M=1 (the decode GEMV) and M=64 (the
        DMA tiles, split-K where the shape splits), W8A8 and W8A16 (W8A16
        outputs wider than 8192 checked on 1024 sampled channels)

Inputs follow BASELINE: X ~ N(0,1) (W8A8: 1% outlier columns x20), W ~
N(0, 0.02) quantized per output channel. The emulation does not time
anything; tests/test_gpu_configs.py holds the same shapes for the GPU.

TVQ_EMU_RACE=1 (with EMU_DMA=late) runs the same cases on the race-checking
build (tests/cpu_emu/racecheck.h), single-threaded, and fails a case that
produces a race report.
"""
from __future__ import annotations

import functools
import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, f32, make_activations, make_weights, ragged_prefill_rows

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "cpu_emu"))
import emu  # noqa: E402

if not Path(emu.CLANG).exists():  # pragma: no cover
    pytest.skip("host clang of the ROCm toolchain not found", allow_module_level=True)


RACE = os.environ.get("TVQ_EMU_RACE") == "1"


@pytest.fixture(scope="module")
def lib():
    return emu.load(race=RACE)


@pytest.fixture(autouse=True)
def _no_race_reports(lib):
    before = lib.tvq_emu_race_reports() if RACE else 0
    yield
    if RACE:
        assert lib.tvq_emu_race_reports() == before, "race report(s): see stderr"


_WS = {}


@functools.lru_cache(maxsize=4)
def _weights(n, k, seed):
    """Quantized weights, generated once per shape for every mode and M."""
    return make_weights(n, k, seed=seed)


def _ws(lib):
    if "ws" not in _WS:
        n = lib.tvq_gemm_workspace_bytes()
        raw = torch.zeros(n + 256, dtype=torch.uint8)
        off = (-raw.data_ptr()) % 256
        _WS["raw"], _WS["ws"] = raw, raw[off:off + n]
    return _WS["ws"]


def _w8a8_linear(lib, x, q, s):
    m, k = x.shape
    n = q.shape[0]
    y = torch.empty(m, n, dtype=torch.bfloat16)
    xq = torch.empty(m, k, dtype=torch.int8)
    xs = torch.empty(m)
    ws = _ws(lib)
    rc = lib.tvq_w8a8_linear(x.data_ptr(), 1, q.data_ptr(), s.data_ptr(), None, y.data_ptr(), m, n, k, xq.data_ptr(),
                             xs.data_ptr(), ws.data_ptr(), ws.numel(), None)
    assert rc == 0, lib.tvq_last_error()
    return y, xq, xs


def _w8a16(lib, x, q, s):
    m, k = x.shape
    n = q.shape[0]
    y = torch.empty(m, n, dtype=torch.bfloat16)
    ws = _ws(lib)
    rc = lib.tvq_w8a16_gemm(x.data_ptr(), 1, q.data_ptr(), s.data_ptr(), None, y.data_ptr(), m, n, k, ws.data_ptr(),
                            ws.numel(), None)
    assert rc == 0, lib.tvq_last_error()
    return y


def _check_w8a8(y, xq, xs, x, q, s, rows=None):
    """Codes and scales exact against the oracle, accumulator-exact output
    through the restated epilogue, torch-path tolerance."""
    r = slice(None) if rows is None else torch.as_tensor(rows)
    xr = x[r]
    rq, rs = oracle.c_act_quant(bits16(xr))
    np.testing.assert_array_equal(xq[r].numpy(), rq)
    np.testing.assert_array_equal(xs[r].numpy().view(np.uint32), rs.view(np.uint32))
    yb, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(rq, q.numpy()), rs, s.numpy())
    np.testing.assert_array_equal(bits16(y[r]), yb)
    ref = oracle.w8a8_torch_path(torch.from_numpy(rq), torch.from_numpy(rs), q, s, None, torch.bfloat16)
    assert oracle.rel_l2(f32(y[r]), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(y[r]), f32(ref)) <= oracle.MAX_ABS_TOL


def _check_w8a16(y, x, q, s):
    if q.shape[0] > 8192:  # the fp64 oracle on 1024 sampled output channels
        cols = torch.as_tensor(np.sort(np.random.default_rng(1).choice(q.shape[0], 1024, replace=False)))
        y, q, s = y[:, cols], q[cols], s[cols]
    ref = oracle.w8a16_torch_path(x, q, s)
    assert oracle.rel_l2(f32(y), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(y), f32(ref)) <= oracle.MAX_ABS_TOL
    y64 = oracle.c_w8a16_f64(bits16(x), q.numpy(), s.numpy(), None, is_bf16=True)
    mag = (np.abs(f32(x)).astype(np.float64) @ np.abs(q.numpy()).astype(np.float64).T) * s.numpy()[None, :]
    bound = np.abs(y64) * 2.0 ** -8 + mag * (x.shape[1] * 2.0 ** -23) + 1e-30
    assert np.all(np.abs(f32(y).astype(np.float64) - y64) <= bound)


def test_cfg1_w8a16_gate_up_m64(lib):
    m, n, k = 64, 6144, 1024
    x = make_activations(m, k, seed=0, outlier_frac=0.0)
    q, s = make_weights(n, k, seed=1)
    _check_w8a16(_w8a16(lib, x, q, s), x, q, s)


@pytest.mark.parametrize("m", [1, 16, 64, 256, 512])
def test_cfg2_w8a8_qkv(lib, m):
    n, k = 4096, 1024
    x = make_activations(m, k, seed=m)
    q, s = make_weights(n, k, seed=2)
    y, xq, xs = _w8a8_linear(lib, x, q, s)
    _check_w8a8(y, xq, xs, x, q, s)


def _prefill_x(k, seed, outliers):
    lens = ragged_prefill_rows(8192, 16, 100, 1024, seed=seed)
    x = make_activations(8192, k, seed=seed, outlier_frac=0.01 if outliers else 0.0)
    x[sum(lens):].zero_()  # padding rows
    return x, sum(lens)


@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
@pytest.mark.parametrize("nk", [(1024, 3072), (1024, 2048), (6144, 1024)], ids=["down", "o", "gate_up"])
def test_cfg3_prefill_m8192(lib, mode, nk):
    n, k = nk
    x, used = _prefill_x(k, seed=n + k, outliers=mode == "w8a8")
    q, s = _weights(n, k, k)
    rows = np.sort(np.random.default_rng(0).choice(used, 47, replace=False)).tolist() + [8191]
    if mode == "w8a8":
        y, xq, xs = _w8a8_linear(lib, x, q, s)
        _check_w8a8(y, xq, xs, x, q, s, rows)
    else:
        y = _w8a16(lib, x, q, s)
        _check_w8a16(y[torch.as_tensor(rows)], x[torch.as_tensor(rows)], q, s)
    assert torch.isfinite(y.float()).all()
    assert (y[used:].float() == 0).all()


CFG4 = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096), "down": (4096, 12288)}


@pytest.mark.parametrize("proj", list(CFG4))
@pytest.mark.parametrize("m", [1, 64])
@pytest.mark.parametrize("mode", ["w8a8", "w8a16"])
def test_cfg4_8b_projections(lib, proj, mode, m):
    n, k = CFG4[proj]
    x = make_activations(m, k, seed=n + m, outlier_frac=0.01 if mode == "w8a8" else 0.0)
    q, s = _weights(n, k, k + 5)
    if mode == "w8a8":
        y, xq, xs = _w8a8_linear(lib, x, q, s)
        _check_w8a8(y, xq, xs, x, q, s)
    else:
        _check_w8a16(_w8a16(lib, x, q, s), x, q, s)
