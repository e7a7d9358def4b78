"""Parity of the kernel sources on the CPU: tiny-vllm_amd/csrc compiled for the
host against the gfx950 emulation in tests/cpu_emu (MFMA, LDS DMA,
cross-lane operations and barriers emulated; see tests/cpu_emu/hip/hip_runtime.h),
called through the same C ABI and Python wrappers as on the GPU, and checked
against the oracle to the GPU tests' bar:

  * act-quant codes and scales, W8A8 int32 accumulators and W8A8 outputs
    (the restated reference epilogue): bit-exact;
  * W8A16 (default and rounded dequant): within the GPU tests' bounds;
  * producers, gate_up+SiLU epilogue, q/k-norm + rotary, attention: the
    GPU tests' bounds (the emulation's exp2 / rcp are libm's, about an ulp
    from the hardware's).

What this does not show: timing, the GPU memory model across XCDs (the
emulation's memory is coherent), and the hardware's exp2 / rcp rounding.
Here one workgroup runs at a time and each LDS DMA lands when issued; child
processes rerun a case of every family with 32 workgroups interleaved in
random order, DMA landing at the latest permitted time, and on an
AddressSanitizer build. Every DMA
tile configuration is reached at small shapes through a hook compiled into
the emulation build only (TVQ_TEST_HOOKS), and small CU counts (EMU_CUS) make
the persistent grid walk several tiles per workgroup.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, f32, make_activations, make_weights

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "cpu_emu"))
import emu  # noqa: E402

if not Path(emu.CLANG).exists():  # pragma: no cover
    pytest.skip("host clang of the ROCm toolchain not found", allow_module_level=True)

# DmaCfg indices (gemm_dma.hip)
CFG = dict(kI8_256x256=0, kI8_256x128=1, kI8_64x64=2, kI8_64x128=3, kI8_32x64=4, kH_128x256=5, kH_64x128=6,
           kH_64x64=7, kH_32x64=8, kH_64x128w8=9, kI8_256x256w4=10, kH_128x256w4=11, kH_16x128=12,
           kH_64x256=13, kH_32x256=14)
I8_CFGS = [c for c in CFG if c.startswith("kI8")]
H_CFGS = [c for c in CFG if c.startswith("kH")]


@pytest.fixture(scope="module")
def elib():
    return emu.load()


class _NoDevice:
    def __init__(self, *a, **k):
        pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


_WS = {}


def _workspace(lib):
    if "ws" not in _WS:
        n = lib.tvq_gemm_workspace_bytes()
        raw = torch.zeros(n + 256, dtype=torch.uint8)
        off = (-raw.data_ptr()) % 256
        _WS["raw"] = raw
        _WS["ws"] = raw[off:off + n]
    return _WS["ws"]


@pytest.fixture
def hip(elib, monkeypatch):
    """nanovllm.quantization._hip running on the emulated library with CPU tensors."""
    from nanovllm.quantization import _hip
    monkeypatch.setattr(_hip, "load_library", lambda: elib)
    monkeypatch.setattr(_hip, "_require_gpu", lambda *ts: torch.device("cpu"))
    monkeypatch.setattr(_hip, "_stream", lambda dev: None)
    monkeypatch.setattr(_hip, "gemm_workspace", lambda dev: _workspace(elib))
    monkeypatch.setattr(torch.cuda, "device", _NoDevice)
    monkeypatch.setenv("EMU_CUS", "256")
    return _hip


@contextlib.contextmanager
def forced_cfg(elib, name):
    v = ctypes.c_int.in_dll(elib, "tvq_test_force_dma_cfg")
    old = v.value
    v.value = CFG[name]
    try:
        yield
    finally:
        v.value = old


def _w8a8_inputs(m, n, k, seed):
    x = make_activations(m, k, seed=seed)
    xq, a_s = oracle.c_act_quant(bits16(x))
    q, w_s = make_weights(n, k, seed=seed + 1)
    return xq, a_s, q.numpy(), w_s.numpy()


def _w8a16_check(y, x, q, s, bias=None):
    """As the GPU tests: the torch-path tolerance and a bf16-rounding bound vs fp64."""
    ref = oracle.w8a16_torch_path(x, q, s, bias)
    assert oracle.rel_l2(f32(y), f32(ref)) <= oracle.REL_L2_TOL
    assert oracle.max_abs_ratio(f32(y), f32(ref)) <= oracle.MAX_ABS_TOL
    y64 = oracle.c_w8a16_f64(bits16(x), q.numpy(), s.numpy(), None if bias is None else f32(bias),
                             is_bf16=x.dtype == torch.bfloat16)
    mag = (np.abs(f32(x)).astype(np.float64) @ np.abs(q.numpy()).astype(np.float64).T) * s.numpy()[None, :]
    half_ulp = 2.0 ** -8 if x.dtype == torch.bfloat16 else 2.0 ** -11
    bound = np.abs(y64) * half_ulp + mag * (x.shape[1] * 2.0 ** -23) + 1e-30
    err = np.abs(f32(y).astype(np.float64) - y64)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


# ---------------------------------------------------------------- act-quant

ACT_SHAPES = [(1, 1024), (3, 1024), (64, 1024), (33, 4096), (5, 12288), (2, 8), (7, 24), (9, 100), (1, 1),
              (511, 256), (600, 128), (1030, 64), (3, 24), (2, 16384)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", ACT_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_act_quant_bit_exact(hip, shape, dtype):
    m, k = shape
    x = make_activations(m, k, seed=m * 131 + k, dtype=dtype)
    if m >= 3:
        x[1].zero_()
        x[2] = x[2] * 1e-30 if dtype == torch.bfloat16 else x[2] * 1e-6
    q_ref, s_ref = oracle.c_act_quant(bits16(x), is_bf16=dtype == torch.bfloat16)
    xq, s = hip.act_quant(x)
    np.testing.assert_array_equal(s.numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(xq.numpy(), q_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_act_quant_and_rmsnorm_codes_near_ties(hip, dtype):
    rng = np.random.default_rng(5)
    rows = []
    for _ in range(96):
        amax = np.float32(rng.uniform(0.5, 40.0))
        s = max(np.float32(amax / np.float32(127.0)), np.float32(1e-8))
        k = rng.integers(-126, 126, 255).astype(np.float32)
        t = (k + np.float32(0.5)) * s * (1 + rng.integers(-4, 5, 255) * np.float32(2.0 ** -23))
        rows.append(np.concatenate([[amax], t]).astype(np.float32))
    x = torch.from_numpy(np.stack(rows)).to(dtype)
    q_ref, s_ref = oracle.c_act_quant(bits16(x), is_bf16=dtype == torch.bfloat16)
    xq, sc = hip.act_quant(x)
    np.testing.assert_array_equal(sc.numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(xq.numpy(), q_ref)
    y, q = hip.rmsnorm(x, torch.ones(256, dtype=dtype), 1e-6, out=True, quant=True)
    rq, rs = oracle.c_act_quant(bits16(y), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(q[0].numpy(), rq)
    np.testing.assert_array_equal(q[1].numpy().view(np.uint32), rs.view(np.uint32))


# ---------------------------------------------------------------- W8A8 / W8A16, default dispatch

GEMM_SHAPES = [(1, 256, 1024), (2, 128, 2048), (1, 64, 9216), (3, 128, 1024), (16, 200, 1024), (17, 100, 1024),
               (5, 96, 1040), (7, 33, 40), (64, 128, 3072), (33, 256, 4096), (48, 256, 1024), (65, 256, 1024),
               (129, 136, 80), (300, 130, 2048), (256, 512, 1024), (2, 136, 3072), (12, 16384, 128)]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_w8a8_accumulator_bit_exact(hip, shape):
    m, n, k = shape
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m + n + k)
    acc = hip.w8a8_gemm_i32(torch.from_numpy(xq), torch.from_numpy(q))
    np.testing.assert_array_equal(acc.numpy(), oracle.c_gemm_i32(xq, q))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_w8a8_output_bit_exact(hip, shape, out_dtype):
    m, n, k = shape
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=3 * m + n + k)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(m)).to(out_dtype) if m % 2 else None
    y = hip.w8a8_gemm(torch.from_numpy(xq), torch.from_numpy(a_s), torch.from_numpy(q), torch.from_numpy(w_s),
                      bias, out_dtype)
    yb_ref, yf_ref = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q), a_s, w_s, None if bias is None else f32(bias))
    if out_dtype == torch.bfloat16:
        np.testing.assert_array_equal(bits16(y), yb_ref)
    else:
        np.testing.assert_array_equal(bits16(y), yf_ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_w8a16_output(hip, shape, dtype):
    m, n, k = shape
    x = make_activations(m, k, seed=m * 7 + n + k, dtype=dtype, outlier_frac=0.0)
    q, s = make_weights(n, k, seed=m + 2 * n + k)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(n)).to(dtype) if m % 3 == 0 else None
    y = hip.w8a16_gemm(x, q, s, bias)
    _w8a16_check(y, x, q, s, bias)


@pytest.mark.parametrize("fam", ["gemv", "skinny", "stream", "dma"])
def test_forced_families_agree(hip, monkeypatch, fam):
    """TVQ_GEMM_PATH forces a kernel family on shapes it supports: every
    family gives the oracle's exact W8A8 accumulators and a W8A16 output in
    bounds on the same inputs."""
    monkeypatch.setenv("TVQ_GEMM_PATH", fam)
    shapes = {"gemv": [(1, 64, 2048), (2, 100, 1024)], "skinny": [(1, 64, 1024), (9, 96, 256), (16, 64, 2048)],
              "stream": [(9, 16384, 256), (40, 16448, 256)], "dma": [(3, 128, 1024), (40, 256, 512)]}[fam]
    for m, n, k in shapes:
        xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m * n)
        acc = hip.w8a8_gemm_i32(torch.from_numpy(xq), torch.from_numpy(q))
        np.testing.assert_array_equal(acc.numpy(), oracle.c_gemm_i32(xq, q))
        x = make_activations(m, k, seed=m + k, outlier_frac=0.0)
        qq, s = make_weights(n, k, seed=n)
        _w8a16_check(hip.w8a16_gemm(x, qq, s), x, qq, s)


# ---------------------------------------------------------------- every DMA tile configuration

def _dma_cases(tile_m, tile_n):
    # ragged M and N (partial tiles) and a whole-tile case; K of 1..3 stages of 128 plus 8
    return [(tile_m + tile_m // 2 + 3, 2 * tile_n + 40, 384), (tile_m, tile_n, 1024), (max(1, tile_m // 3), 24, 256)]


TILE = {c: (int(c.split("_")[1].split("x")[0]), int(c.split("x")[1].rstrip("w48"))) for c in CFG}


@pytest.mark.parametrize("cus", [256, 3, 12])
@pytest.mark.parametrize("cfg", I8_CFGS)
def test_dma_w8a8_every_config(hip, elib, monkeypatch, cfg, cus):
    """Each W8A8 DMA tile with ragged edges, bit-exact accumulators and
    outputs; with 3 CUs the persistent grid walks several tiles per
    workgroup (the next tile's stages go out before the current epilogue);
    12 CUs round the grid down to whole rounds of the 8 XCDs."""
    monkeypatch.setenv("EMU_CUS", str(cus))
    bm, bn = TILE[cfg]
    with forced_cfg(elib, cfg):
        for m, n, k in _dma_cases(bm, bn):
            xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=m + n)
            acc = hip.w8a8_gemm_i32(torch.from_numpy(xq), torch.from_numpy(q), split_k=False)
            np.testing.assert_array_equal(acc.numpy(), oracle.c_gemm_i32(xq, q))
            bias = torch.randn(n, generator=torch.Generator().manual_seed(k)).to(torch.bfloat16)
            y = hip.w8a8_gemm(torch.from_numpy(xq), torch.from_numpy(a_s), torch.from_numpy(q),
                              torch.from_numpy(w_s), bias, torch.bfloat16, split_k=False)
            yb_ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q), a_s, w_s, f32(bias))
            np.testing.assert_array_equal(bits16(y), yb_ref)


@pytest.mark.parametrize("cus", [256, 3, 12])
@pytest.mark.parametrize("cfg", H_CFGS)
def test_dma_w8a16_every_config(hip, elib, monkeypatch, cfg, cus):
    monkeypatch.setenv("EMU_CUS", str(cus))
    bm, bn = TILE[cfg]
    with forced_cfg(elib, cfg):
        for m, n, k in _dma_cases(bm, bn):
            for dtype in (torch.bfloat16, torch.float16):
                x = make_activations(m, k, seed=m + k, dtype=dtype, outlier_frac=0.0)
                q, s = make_weights(n, k, seed=n + k)
                bias = torch.randn(n, generator=torch.Generator().manual_seed(m)).to(dtype)
                _w8a16_check(hip.w8a16_gemm(x, q, s, bias, split_k=False), x, q, s, bias)


@pytest.mark.parametrize("cfg", ["kH_64x64", "kH_128x256", "kH_16x128", "kH_64x128w8"])
def test_dma_rounded_dequant(hip, elib, cfg):
    """The rounded-dequant mode on DMA tiles: within one output rounding plus
    the fp32 summation bound of the exact product of the rounded weights."""
    bm, bn = TILE[cfg]
    with forced_cfg(elib, cfg):
        for m, n, k in _dma_cases(bm, bn):
            for dtype in (torch.bfloat16, torch.float16):
                x = make_activations(m, k, seed=m, dtype=dtype, outlier_frac=0.0)
                q, s = make_weights(n, k, seed=n)
                y = hip.w8a16_gemm_rounded(x, q, s)
                wdf = oracle.w8a16_rounded_weights(q.numpy(), s.numpy(), is_bf16=dtype == torch.bfloat16)
                y64 = oracle.w8a16_rounded_f64(f32(x), wdf)
                mag = np.abs(f32(x)).astype(np.float64) @ np.abs(wdf).astype(np.float64).T
                half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
                bound = np.abs(y64) * half_ulp + mag * (k * 2.0 ** -23) + 1e-30
                assert np.all(np.abs(f32(y).astype(np.float64) - y64) <= bound)


def test_operand_floor_runs_and_writes_nothing(hip, elib):
    for op, m, n, k in [(2, 256, 512, 1024), (1, 64, 256, 2048), (2, 40, 128, 384), (1, 300, 256, 256)]:
        x = torch.ones(m, k, dtype=torch.int8 if op == 2 else torch.bfloat16)
        q = torch.ones(n, k, dtype=torch.int8)
        before = (x.clone(), q.clone())
        hip.gemm_operand_floor(op, x, q)
        assert torch.equal(x, before[0]) and torch.equal(q, before[1])


# ---------------------------------------------------------------- split-K and stream-K

SPLIT_SHAPES = [(1, 64, 4096), (5, 128, 8192), (33, 96, 4096), (64, 128, 2048), (17, 256, 12288)]


@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_split_k_matches_unsplit(hip, monkeypatch, shape):
    """Split-K (the DMA tiles at decode M with a workspace): bit-identical
    W8A8 accumulators and outputs, W8A16 within the bound, counters zero
    afterwards."""
    monkeypatch.setenv("TVQ_GEMM_PATH", "dma")
    m, n, k = shape
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=k + m)
    t = [torch.from_numpy(v) for v in (xq, a_s, q, w_s)]
    y1 = hip.w8a8_gemm(*t, None, torch.bfloat16, split_k=True)
    y0 = hip.w8a8_gemm(*t, None, torch.bfloat16, split_k=False)
    assert torch.equal(y1.view(torch.int16), y0.view(torch.int16))
    np.testing.assert_array_equal(hip.w8a8_gemm_i32(t[0], t[2]).numpy(), oracle.c_gemm_i32(xq, q))
    x = make_activations(m, k, seed=m, outlier_frac=0.0)
    qq, s = make_weights(n, k, seed=n)
    _w8a16_check(hip.w8a16_gemm(x, qq, s, split_k=True), x, qq, s)
    assert int(_workspace(hip.load_library())[:65536].view(torch.int32).abs().sum()) == 0


STREAMK_SHAPES = [(1, 512, 1024), (16, 384, 2048), (17, 640, 1024), (33, 1280, 512), (64, 1152, 1024), (8, 200, 384)]


@pytest.mark.parametrize("cus", [8, 5])
@pytest.mark.parametrize("shape", STREAMK_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_streamk_matches_oracle(hip, monkeypatch, shape, cus):
    """Stream-K (TVQ_STREAMK=1, opt-in): every CU takes an equal share of the
    tiles' k-stages; with a few emulated CUs a workgroup's range cuts tiles
    into several contributors. Exact W8A8, W8A16 within the bound, counters
    zero afterwards."""
    monkeypatch.setenv("TVQ_STREAMK", "1")
    monkeypatch.setenv("TVQ_STREAMK_MIN", "2")
    monkeypatch.setenv("EMU_CUS", str(cus))
    m, n, k = shape
    assert "streamk" in hip.select_path(hip.OP_W8A8, m, n, k) or m <= 2
    xq, a_s, q, w_s = _w8a8_inputs(m, n, k, seed=n + k)
    np.testing.assert_array_equal(hip.w8a8_gemm_i32(torch.from_numpy(xq), torch.from_numpy(q)).numpy(),
                                  oracle.c_gemm_i32(xq, q))
    y = hip.w8a8_gemm(*(torch.from_numpy(v) for v in (xq, a_s, q, w_s)), None, torch.bfloat16)
    yb_ref, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q), a_s, w_s)
    np.testing.assert_array_equal(bits16(y), yb_ref)
    for dtype in (torch.bfloat16, torch.float16):
        x = make_activations(m, k, seed=m, dtype=dtype, outlier_frac=0.0)
        qq, s = make_weights(n, k, seed=n)
        _w8a16_check(hip.w8a16_gemm(x, qq, s), x, qq, s)
    assert int(_workspace(hip.load_library())[:65536].view(torch.int32).abs().sum()) == 0


# ---------------------------------------------------------------- fused linear, no-alloc entry

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_w8a8_linear_and_noalloc(hip, elib, dtype):
    for m, n, k in [(1, 256, 1024), (8, 128, 2048), (64, 128, 3072), (300, 256, 1024), (4, 64, 40)]:
        x = make_activations(m, k, seed=m + k, dtype=dtype)
        q, w_s = make_weights(n, k, seed=n)
        y = hip.w8a8_linear(x, q, w_s)
        xq, a_s = hip.act_quant(x)
        y2 = hip.w8a8_gemm(xq, a_s, q, w_s, None, dtype)
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
        y3 = torch.empty_like(y)
        rc = elib.tvq_w8a8_linear_noalloc(x.data_ptr(), hip._TORCH_TO_TVQ[dtype], q.data_ptr(), w_s.data_ptr(), None,
                                          y3.data_ptr(), m, n, k, None)
        assert rc == 0, elib.tvq_last_error()
        assert torch.equal(y.view(torch.int16), y3.view(torch.int16))


# ---------------------------------------------------------------- producers and the gate_up epilogue

def _ulp(ref, dtype):
    mant = 7 if dtype == torch.bfloat16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(ref), 1e-30)))
    return np.exp2(np.maximum(e, -126 if dtype == torch.bfloat16 else -14) - mant)


RMS_SHAPES = [(1, 1024), (7, 1024), (64, 128), (33, 4096), (5, 5000), (9, 1003), (1, 8), (600, 256), (1030, 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", RMS_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_rmsnorm_and_codes(hip, shape, dtype):
    m, k = shape
    x = make_activations(m, k, seed=m + k, dtype=dtype)
    res = make_activations(m, k, seed=m + k + 1, dtype=dtype)
    w = (torch.rand(k, generator=torch.Generator().manual_seed(k)) + 0.5).to(dtype)
    r0 = res.clone()
    y, q = hip.rmsnorm(x, w, 1e-6, residual=res, out=True, quant=True)
    y_ref, r_ref = oracle.rmsnorm_ref(f32(x), f32(w), 1e-6, f32(r0), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(f32(res), r_ref)
    diff = np.abs(f32(y) - y_ref)
    assert np.all(diff <= 2 * _ulp(y_ref, dtype) * 1.0001)
    rq, rs = oracle.c_act_quant(bits16(y), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(q[0].numpy(), rq)
    np.testing.assert_array_equal(q[1].numpy().view(np.uint32), rs.view(np.uint32))


SILU_SHAPES = [(1, 3072), (7, 3072), (64, 64), (33, 1000), (600, 256), (1030, 96)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SILU_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_silu_mul_and_codes(hip, shape, dtype):
    m, i = shape
    gu = make_activations(m, 2 * i, seed=m + i, dtype=dtype)
    y, q = hip.silu_mul(gu, out=True, quant=True)
    ref = oracle.silu_mul_ref(f32(gu), is_bf16=dtype == torch.bfloat16)
    assert np.all(np.abs(f32(y) - ref) <= _ulp(ref, dtype) * 1.0001)
    rq, rs = oracle.c_act_quant(bits16(y), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(q[0].numpy(), rq)
    np.testing.assert_array_equal(q[1].numpy().view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,i,k", [(1, 64, 128), (300, 160, 384), (513, 96, 256)])
def test_gemm_glu_matches_gemm_then_silu_mul(hip, m, i, k, dtype):
    from nanovllm.quantization.utils import quantize_int8_per_channel
    x = make_activations(m, k, seed=m + i, dtype=dtype)
    w = torch.randn(2 * i, k, generator=torch.Generator().manual_seed(k)) * 0.02
    qw, ws = quantize_int8_per_channel(w)
    ws = ws.float()
    xq, xs = hip.act_quant(x)
    ref = hip.w8a8_gemm(xq, xs, qw, ws, out_dtype=dtype, split_k=False)
    yref, _ = hip.silu_mul(ref, out=True, quant=False)
    q2, s2 = hip.glu_interleave(qw, ws)
    y = hip.w8a8_gemm_glu(xq, xs, q2, s2, out_dtype=dtype)
    assert torch.equal(y, yref)


# ---------------------------------------------------------------- q/k-norm + rotary, attention

def _rope_ref(qkv, pos, cos, sin, qw, kw, eps, hq, hkv, d):
    t = qkv.shape[0]
    q = qkv[:, : hq * d].reshape(t, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].reshape(t, hkv, d)

    def norm(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w

    def rot(x):
        c, s = cos[pos].unsqueeze(1), sin[pos].unsqueeze(1)
        x1, x2 = x.float().chunk(2, -1)
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), -1).to(x.dtype)

    if qw is not None:
        q, k = norm(q, qw), norm(k, kw)
    return rot(q), rot(k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("t,hq,hkv", [(1, 16, 8), (37, 16, 8)])
def test_qk_norm_rope_and_kv_store(elib, dtype, t, hq, hkv):
    d, max_pos, n_slots, max_len = 128, 256, 3, 64
    g = torch.Generator().manual_seed(t + hq)
    qkv = (torch.randn(t, (hq + 2 * hkv) * d, generator=g) * 2).to(dtype)
    pairs = torch.randperm(n_slots * max_len, generator=g)[:t]   # distinct (slot, position), as the engine's
    pos = pairs % max_len
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=torch.float) / d))
    fr = torch.outer(torch.arange(max_pos, dtype=torch.float), inv)
    cos, sin = fr.cos().contiguous(), fr.sin().contiguous()
    qw = (torch.rand(d, generator=g) + 0.5).to(dtype)
    kw = (torch.rand(d, generator=g) + 0.5).to(dtype)
    slots = pairs // max_len
    kc = torch.zeros(n_slots, hkv, max_len, d, dtype=dtype)
    vc = torch.zeros_like(kc)
    q = torch.empty(t, hq, d, dtype=dtype)
    k = torch.empty(t, hkv, d, dtype=dtype)
    rc = elib.tvq_qk_norm_rope(qkv.data_ptr(), qkv.stride(0), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                               qw.data_ptr(), kw.data_ptr(), 1e-6, t, hq, hkv, d, max_pos, q.data_ptr(), k.data_ptr(),
                               kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), n_slots, max_len,
                               1 if dtype == torch.bfloat16 else 0, None)
    assert rc == 0, elib.tvq_last_error()
    rq, rk = _rope_ref(qkv, pos, cos, sin, qw, kw, 1e-6, hq, hkv, d)
    for got, ref in ((q, rq), (k, rk)):
        gf, rf = got.float(), ref.float()
        ulp = torch.exp2(torch.floor(torch.log2(rf.abs().clamp_min(1e-30))) - (7 if dtype == torch.bfloat16 else 10))
        head_ulp = rf.abs().amax(-1, keepdim=True) * 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
        assert torch.all((gf - rf).abs() <= 2.0001 * ulp + head_ulp + 1e-6)
    v = qkv[:, (hq + hkv) * d:].reshape(t, hkv, d)
    for i in range(t):
        sl, p = int(slots[i]), int(pos[i])
        assert torch.equal(kc[sl, :, p], k[i]) and torch.equal(vc[sl, :, p], v[i])


def _decode_ref(q, kc, vc, slots, lens, scale):
    out = []
    hq, hkv = q.shape[1], kc.shape[1]
    for b in range(q.shape[0]):
        n = int(lens[b])
        k = kc[int(slots[b]), :, :n].float().repeat_interleave(hq // hkv, 0)
        v = vc[int(slots[b]), :, :n].float().repeat_interleave(hq // hkv, 0)
        p = torch.softmax((q[b].float()[:, None, :] @ k.transpose(1, 2)).squeeze(1) * scale, -1)
        out.append((p[:, None, :] @ v).squeeze(1))
    return torch.stack(out)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4)])
def test_decode_attention(elib, hq, hkv):
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(hq * 10 + hkv)
    n_slots, max_len, d = 5, 80, 128
    kc = torch.randn(n_slots, hkv, max_len, d, generator=g).to(dtype)
    vc = torch.randn(n_slots, hkv, max_len, d, generator=g).to(dtype)
    lens_l, slots_l = [1, 2, 17, 33, 80], [3, 0, 4, 1, 2]
    b = len(lens_l)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g).to(dtype)
    q = qkv[:, : hq * d].view(b, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].view(b, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    slots = torch.tensor(slots_l, dtype=torch.int32)
    lens = torch.tensor(lens_l, dtype=torch.int32)
    exp_k, exp_v = kc.clone(), vc.clone()
    for i in range(b):
        exp_k[slots_l[i], :, lens_l[i] - 1] = k[i]
        exp_v[slots_l[i], :, lens_l[i] - 1] = v[i]
    out = torch.empty(b, hq, d, dtype=dtype)
    rc = elib.tvq_decode_attention(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
                                   kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), lens.data_ptr(), b, hq, hkv, d,
                                   n_slots, max_len, d ** -0.5, out.data_ptr(), 1, None)
    assert rc == 0, elib.tvq_last_error()
    assert torch.equal(kc, exp_k) and torch.equal(vc, exp_v)
    ref = _decode_ref(q, exp_k, exp_v, slots, lens, d ** -0.5)
    assert (out.float() - ref).abs().max().item() <= 1e-2 * ref.abs().max().item() + 1e-3


def _prefill_ref(q, k, v, lens, scale):
    out = torch.empty_like(q, dtype=torch.float32)
    hq, hkv = q.shape[1], k.shape[1]
    off = 0
    for n in lens:
        qq = q[off:off + n].float().transpose(0, 1)
        kk = k[off:off + n].float().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        vv = v[off:off + n].float().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        s = qq @ kk.transpose(1, 2) * scale
        s.masked_fill_(torch.ones(n, n, dtype=torch.bool).triu(1), float("-inf"))
        out[off:off + n] = (torch.softmax(s, -1) @ vv).transpose(0, 1)
        off += n
    return out


@pytest.mark.parametrize("hq,hkv", [(4, 2), (8, 2), (2, 2), (6, 2), (24, 4)])   # GQA ratios 2, 4, 1, 3, 6
def test_prefill_attention(hip, elib, hq, hkv):
    """GQA ratio 2 and 4: the 32-query DMA kernel; 1 and 3: the 16-query one."""
    dtype = torch.bfloat16
    lens = [1, 5, 64, 65, 129]
    t, d = sum(lens), 128
    g = torch.Generator().manual_seed(hq + hkv)
    q = torch.randn(t, hq, d, generator=g).to(dtype)
    k = torch.randn(t, hkv, d, generator=g).to(dtype)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(dtype)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    offs, o = [], 0
    for n in lens:
        offs.append((o, n))
        o += n
    blocks = hip.prefill_blocks(offs)
    out = torch.empty_like(q)
    rc = elib.tvq_prefill_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0), blocks.data_ptr(),
                                    blocks.shape[0], hq, hkv, d, d ** -0.5, out.data_ptr(), 1, None)
    assert rc == 0, elib.tvq_last_error()
    ref = _prefill_ref(q, k, v, lens, d ** -0.5)
    err = (out.float() - ref).abs()
    assert err.max().item() <= 1.5e-2 * ref.abs().amax() + 1e-3
    assert ((out.float() - ref).norm() / ref.norm()).item() < 8e-3


# ---------------------------------------------------------------- attention with o_proj's quantization fused

def _counters(n=64):
    return torch.zeros(n, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(4, 2), (8, 2), (2, 2), (6, 2), (24, 4), (32, 8)])   # 32 heads: 4096-wide rows
def test_prefill_attention_quant(hip, elib, hq, hkv, dtype):
    """The quantizing prefill attention writes the same output as the plain
    kernel, and int8 codes / scales bit-identical to act-quant of that
    output; the counters are zero afterwards (two calls in a row, the second
    smaller)."""
    d = 128
    for lens in ([1, 5, 64, 65, 129], [3, 70]):
        t = sum(lens)
        g = torch.Generator().manual_seed(hq + hkv + t)
        q = torch.randn(t, hq, d, generator=g).to(dtype)
        k = torch.randn(t, hkv, d, generator=g).to(dtype)
        qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(dtype)
        v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
        offs, o = [], 0
        for n in lens:
            offs.append((o, n))
            o += n
        blocks = hip.prefill_blocks(offs)
        dt = hip._TORCH_TO_TVQ[dtype]
        ref = torch.empty_like(q)
        assert elib.tvq_prefill_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0), blocks.data_ptr(),
                                          blocks.shape[0], hq, hkv, d, d ** -0.5, ref.data_ptr(), dt, None) == 0
        out = torch.empty_like(q)
        xq = torch.full((t, hq * d), 77, dtype=torch.int8)
        xs = torch.full((t,), -1.0)
        cnt = _counters()
        rc = elib.tvq_prefill_attention_quant(q.data_ptr(), k.data_ptr(), v.data_ptr(), v.stride(0),
                                              blocks.data_ptr(), blocks.shape[0], hq, hkv, d, d ** -0.5,
                                              out.data_ptr(), dt, xq.data_ptr(), xs.data_ptr(), 1e-8,
                                              cnt.data_ptr(), cnt.numel(), None)
        assert rc == 0, elib.tvq_last_error()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        rq, rs = oracle.c_act_quant(bits16(ref.view(t, -1)), is_bf16=dtype == torch.bfloat16)
        np.testing.assert_array_equal(xq.numpy(), rq)
        np.testing.assert_array_equal(xs.numpy().view(np.uint32), rs.view(np.uint32))
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4), (32, 8)])   # 32 heads: 4096-wide rows
def test_decode_attention_quant(elib, hq, hkv, dtype):
    """The quantizing decode attention: same output and cache update as the
    plain kernel, codes and scales bit-identical to act-quant of the output,
    an invalid sequence's row quantized from its zero output, counters zero
    afterwards."""
    g = torch.Generator().manual_seed(hq * 3 + hkv)
    n_slots, max_len, d = 5, 80, 128
    kc0 = torch.randn(n_slots, hkv, max_len, d, generator=g).to(dtype)
    vc0 = torch.randn(n_slots, hkv, max_len, d, generator=g).to(dtype)
    lens_l, slots_l = [1, 2, 17, 33, 80, 0], [3, 0, 4, 1, 2, 1]   # the last sequence is invalid (length 0)
    b = len(lens_l)
    qkv = torch.randn(b, (hq + 2 * hkv) * d, generator=g).to(dtype)
    q = qkv[:, : hq * d].view(b, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].view(b, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(b, hkv, d)
    slots = torch.tensor(slots_l, dtype=torch.int32)
    lens = torch.tensor(lens_l, dtype=torch.int32)
    dt = 1 if dtype == torch.bfloat16 else 0
    outs = []
    for quant in (False, True):
        kc, vc = kc0.clone(), vc0.clone()
        out = torch.empty(b, hq, d, dtype=dtype)
        args = (q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), kc.data_ptr(),
                vc.data_ptr(), slots.data_ptr(), lens.data_ptr(), b, hq, hkv, d, n_slots, max_len, d ** -0.5,
                out.data_ptr(), dt)
        if quant:
            xq = torch.full((b, hq * d), 5, dtype=torch.int8)
            xs = torch.full((b,), -1.0)
            cnt = _counters()
            rc = elib.tvq_decode_attention_quant(*args, xq.data_ptr(), xs.data_ptr(), 1e-8, cnt.data_ptr(),
                                                 cnt.numel(), None)
        else:
            rc = elib.tvq_decode_attention(*args, None)
        assert rc == 0, elib.tvq_last_error()
        outs.append((out, kc, vc))
    (o0, k0, v0), (o1, k1, v1) = outs
    assert torch.equal(o0.view(torch.int16), o1.view(torch.int16))
    assert torch.equal(k0, k1) and torch.equal(v0, v1)
    rq, rs = oracle.c_act_quant(bits16(o0.view(b, -1)), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(xq.numpy(), rq)
    np.testing.assert_array_equal(xs.numpy().view(np.uint32), rs.view(np.uint32))
    assert int(cnt.abs().sum()) == 0


# ---------------------------------------------------------------- child-process modes

def test_kernels_in_child_modes():
    """Four child processes, run concurrently, each a case of every family:

      * the AddressSanitizer build (global buffers sized exactly, LDS a fresh
        allocation per workgroup): any out-of-bounds access aborts;
      * 32 workgroups resident at once, in a seeded random order, stalled at
        random so that they drift apart, with every LDS DMA landing only at
        its wave's vmcnt wait (the latest the hardware may complete it): a
        stage wait that waits too little, a cross-wave dependency without a
        barrier, or a cross-workgroup handoff that assumes an arrival order
        breaks parity (a stage wait weakened by one stage gives wrong
        accumulators in this mode and none in the default one; picking the
        attention rows' quantizer by head index instead of by the arrival
        counter gives wrong codes with 32 resident workgroups);
      * the same interleaving with a second seed and DMA landing at issue;
      * the race-checking build (tests/cpu_emu/racecheck.h), DMA landing at
        its wave's wait: no access may conflict with one the GPU does not
        order it against (tests/test_cpu_emu_race.py shows what it catches)."""
    sys.path.insert(0, str(ROOT / "tests" / "cpu_emu"))
    import build as emu_build
    emu.ensure_built(asan=True)
    emu.ensure_built(race=True)
    emu.ensure_built()
    base = dict(os.environ, PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "tiny-vllm_amd")]))
    script = str(ROOT / "tests" / "cpu_emu" / "child_cases.py")
    runs = {
        "asan": ([script, "--asan"], dict(base, LD_PRELOAD=emu_build.asan_runtime(),
                                          ASAN_OPTIONS="detect_leaks=0:detect_stack_use_after_return=0:"
                                                       "abort_on_error=1")),
        "concurrent-late-dma": ([script], dict(base, EMU_DMA="late", EMU_SHUFFLE="1", EMU_CONCURRENT="32")),
        "concurrent": ([script], dict(base, EMU_SHUFFLE="2", EMU_CONCURRENT="32")),
        "race": ([script, "--race"], dict(base, EMU_DMA="late")),
    }
    procs = {k: subprocess.Popen([sys.executable, *a], env=e, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                 text=True) for k, (a, e) in runs.items()}
    failed = []
    for k, p in procs.items():
        out, err = p.communicate(timeout=900)
        if p.returncode != 0 or "all cases passed" not in out:
            failed.append(f"--- {k}: rc={p.returncode}\n{out[-2000:]}\n{emu.symbolize(err[-4000:])}")
    assert not failed, "\n".join(failed)
