"""Pins the oracle (CPU) before it is trusted as the checker.

The reference ships no unit tests, fixtures or golden vectors for this path,
so each oracle function is pinned by checks a plausible mistake would fail:
closed-form special cases, brute force on tiny inputs, agreement of the two
independent restatements (numpy and C), agreement with CPU torch running the
reference's own expressions, and invariants. Also checks the committed golden
fixtures (tests/golden/*.npz).
"""
from __future__ import annotations

import itertools
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import bits16, f32, make_activations, make_weights

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------ quantizer

def test_quant_zero_row_gives_eps_scale():
    q, s = oracle.quantize_rows(np.zeros((2, 16), np.float32))
    assert s.dtype == np.float32 and np.all(s == np.float32(1e-8))
    assert np.all(q == 0)


def test_quant_single_nonzero_maps_to_127():
    for v in (3.0, -0.001, 1e20, -7.5):
        x = np.zeros((1, 9), np.float32)
        x[0, 4] = v
        q, s = oracle.quantize_rows(x)
        assert q[0, 4] == (127 if v > 0 else -127)
        assert np.count_nonzero(q) == 1
        assert s[0] == np.float32(abs(np.float32(v)) / np.float32(127.0))


def test_quant_amax_element_is_127_for_all_magnitudes():
    rng = np.random.default_rng(0)
    for _ in range(200):
        x = rng.standard_normal((1, 64)).astype(np.float32) * np.float32(10.0 ** rng.uniform(-4, 20))  # amax/127 stays above eps
        q, _ = oracle.quantize_rows(x)
        i = np.argmax(np.abs(x[0]))
        assert abs(int(q[0, i])) == 127


def test_quant_ties_round_half_to_even():
    # amax = 127 -> s = 1 exactly, so q = rint(x)
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 100.5, -126.5, 8.5]], np.float32)
    q, s = oracle.quantize_rows(x)
    assert s[0] == 1.0
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 100, -126, 8]


def test_quant_power_of_two_scale_ties():
    # amax = 127 * 2^-3 -> s = 2^-3; x = (k + 0.5) * 2^-3 are exact ties
    s_exp = 2.0 ** -3
    ks = np.arange(-20, 20)
    x = np.concatenate([[127 * s_exp], (ks + 0.5) * s_exp]).astype(np.float32)[None, :]
    q, s = oracle.quantize_rows(x)
    assert s[0] == np.float32(s_exp)
    expect = [int(np.round(k + 0.5)) for k in ks]  # numpy round = half-even
    assert all(e % 2 == 0 for e in expect)
    assert q[0, 1:].tolist() == expect


def test_quant_never_produces_minus_128_and_clamps():
    x = np.array([[-1.0, 1.0, -0.999999, 0.3]], np.float32)
    q, _ = oracle.quantize_rows(x)
    assert q.min() >= -127
    x = np.full((3, 5), -2.0, np.float32)
    q, _ = oracle.quantize_rows(x)
    assert np.all(q == -127)


def test_quant_eps_floor():
    # amax/127 < eps -> s = eps; values then quantize against eps
    x = np.array([[1e-10, -5e-10, 0.0]], np.float32)
    q, s = oracle.quantize_rows(x)
    assert s[0] == np.float32(1e-8)
    assert q[0].tolist() == [0, 0, 0]
    for amax in (1.26e-6, 1.28e-6):  # amax/127 just below and just above eps
        x = np.array([[amax, 0.5e-8]], np.float32)
        q, s = oracle.quantize_rows(x)
        assert s[0] == max(np.float32(amax) / np.float32(127.0), np.float32(1e-8))


def test_quant_matches_brute_force_python():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((6, 33)) * rng.uniform(0.01, 100, (6, 1))).astype(np.float32)
    q, s = oracle.quantize_rows(x)
    for m in range(6):
        amax = max(abs(float(v)) for v in x[m])
        sc = np.float32(max(np.float32(amax) / np.float32(127.0), np.float32(1e-8)))
        assert s[m] == sc
        for k in range(33):
            t = float(np.float32(x[m, k]) / sc)  # fp32 divide
            r = round(t)  # Python round = half-even
            assert q[m, k] == max(-127, min(127, r))


def test_quant_numpy_matches_torch_reference_expression():
    for seed, (m, k) in enumerate([(64, 1024), (7, 4096), (3, 24)]):
        x = make_activations(m, k, seed=seed)
        q_t, s_t = oracle.quantize_rows_torch(x)
        q_n, s_n = oracle.quantize_rows(f32(x))
        np.testing.assert_array_equal(q_n, q_t.numpy())
        np.testing.assert_array_equal(s_n.view(np.uint32), s_t.numpy().view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_c_matches_numpy(dtype):
    for seed, (m, k) in enumerate([(64, 1024), (9, 3072), (5, 100), (1, 1)]):
        x = make_activations(m, k, seed=seed, dtype=dtype)
        if m > 2:
            x[1].zero_()
        q_c, s_c = oracle.c_act_quant(bits16(x), is_bf16=dtype == torch.bfloat16)
        q_n, s_n = oracle.quantize_rows(f32(x))
        np.testing.assert_array_equal(q_c, q_n)
        np.testing.assert_array_equal(s_c.view(np.uint32), s_n.view(np.uint32))


def test_quant_f32_c_matches_numpy():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((50, 300)) * 0.02).astype(np.float32)
    q_c, s_c = oracle.c_quant_f32(x)
    q_n, s_n = oracle.quantize_rows(x)
    np.testing.assert_array_equal(q_c, q_n)
    np.testing.assert_array_equal(s_c, s_n)


def test_dequant_reconstruction_bound():
    """|q*s - x| <= s/2 for every element (round-to-nearest invariant)."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((20, 512)) * 3).astype(np.float32)
    q, s = oracle.quantize_rows(x)
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 1e-6))


def test_f16_decoder_matches_numpy():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    fin = np.isfinite(bits.view(np.float16))
    x = bits.reshape(256, 256)
    q_c, s_c = oracle.c_act_quant(np.where(fin, bits, 0).astype(np.uint16).reshape(256, 256), is_bf16=False)
    q_n, s_n = oracle.quantize_rows(oracle.f16_bits_to_f32(np.where(fin, bits, 0).reshape(256, 256)))
    np.testing.assert_array_equal(q_c, q_n)
    np.testing.assert_array_equal(s_c, s_n)
    del x


# ------------------------------------------------------------ bf16 rounding

def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.0e38, -1e-40], np.float32)])
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(v), ref)
    np.testing.assert_array_equal(oracle.c_f32_to_bf16(v), ref)


# ------------------------------------------------------------ int32 accumulator

def test_gemm_i32_brute_force_tiny():
    rng = np.random.default_rng(6)
    for m, n, k in [(1, 1, 1), (2, 3, 5), (4, 7, 16), (3, 2, 33)]:
        a = rng.integers(-127, 128, (m, k)).astype(np.int8)
        b = rng.integers(-127, 128, (n, k)).astype(np.int8)
        expect = [[sum(int(a[i, t]) * int(b[j, t]) for t in range(k)) for j in range(n)] for i in range(m)]
        np.testing.assert_array_equal(oracle.gemm_i32(a, b), np.array(expect, np.int32))
        np.testing.assert_array_equal(oracle.c_gemm_i32(a, b), np.array(expect, np.int32))


def test_gemm_i32_extremes_and_identity():
    k = 12288  # largest K in the configs: |acc| <= 127^2 * K < 2^31
    a = np.full((2, k), 127, np.int8)
    a[1] = -127
    b = np.full((3, k), -127, np.int8)
    acc = oracle.c_gemm_i32(a, b)
    assert acc[0, 0] == -127 * 127 * k and acc[1, 0] == 127 * 127 * k
    eye = np.eye(16, dtype=np.int8)
    x = np.random.default_rng(7).integers(-127, 128, (5, 16)).astype(np.int8)
    np.testing.assert_array_equal(oracle.c_gemm_i32(x, eye), x.astype(np.int32))


def test_gemm_i32_c_matches_numpy_and_linearity():
    rng = np.random.default_rng(8)
    a = rng.integers(-60, 61, (37, 200)).astype(np.int8)
    a2 = rng.integers(-60, 61, (37, 200)).astype(np.int8)
    b = rng.integers(-127, 128, (29, 200)).astype(np.int8)
    c1 = oracle.c_gemm_i32(a, b)
    np.testing.assert_array_equal(c1, oracle.gemm_i32(a, b))
    c12 = oracle.c_gemm_i32((a.astype(np.int16) + a2).astype(np.int8), b)
    np.testing.assert_array_equal(c12, c1 + oracle.c_gemm_i32(a2, b))
    # transpose symmetry: (A B^T)^T = B A^T
    np.testing.assert_array_equal(oracle.c_gemm_i32(b, a), c1.T)


# ------------------------------------------------------------ W8A8 epilogue

def test_w8a8_epilogue_c_matches_numpy_and_fp64():
    rng = np.random.default_rng(9)
    acc = rng.integers(-(2 ** 28), 2 ** 28, (40, 50)).astype(np.int32)
    a_s = (rng.uniform(0.001, 1.0, 40)).astype(np.float32)
    w_s = (rng.uniform(1e-5, 1e-3, 50)).astype(np.float32)
    yb, yf = oracle.c_w8a8_epilogue(acc, a_s, w_s)
    np.testing.assert_array_equal(yf, oracle.w8a8_epilogue_f32(acc, a_s, w_s))
    np.testing.assert_array_equal(yb, oracle.w8a8_epilogue_bf16(acc, a_s, w_s))
    exact = acc.astype(np.float64) * a_s[:, None] * w_s[None, :]
    assert np.all(np.abs(yf - exact) <= np.abs(exact) * 2.0 ** -22)
    got = oracle.bf16_bits_to_f32(yb).astype(np.float64)
    assert np.all(np.abs(got - exact) <= np.abs(exact) * (2.0 ** -8 + 2.0 ** -21))


def test_w8a8_epilogue_zero_sign_and_order():
    acc = np.array([[0, -1, 1, 3]], np.int32)
    a_s = np.array([0.5], np.float32)
    w_s = np.array([2.0, -0.0, 4.0, 1.0 / 3.0], np.float32)
    yb, yf = oracle.c_w8a8_epilogue(acc, a_s, w_s)
    # (0*0.5)*2 + 0 = +0; (-1*0.5)*-0 = +0 then + 0 -> +0 bits
    assert yb[0, 0] == 0 and yb[0, 1] == 0
    assert yf[0, 2] == 2.0
    # order: (3*0.5)*(1/3) rounded per step in fp32
    assert yf[0, 3] == np.float32(np.float32(1.5) * np.float32(1.0 / 3.0))


def test_w8a8_epilogue_order_known_answers():
    """Vectors found by a CPU brute-force search where (acc*a_s)*w_s (the
    reference order, w8a8_gemm.cu:387-389) and acc*(a_s*w_s) round to
    different fp32 values and, for the first three, to different bf16 values.
    The expected bits are those of the reference order."""
    u = lambda v: np.array([v], np.uint32).view(np.float32)[0]
    cases = [  # acc, a_s bits, w_s bits, fp32 result (ref order), bf16 bits (ref order, other order)
        (589386, 1058899755, 972549179, 171.5, 17196, 17195),
        (297063, 1035536272, 1005178573, 191.5, 17216, 17215),
        (3299, 1058281226, 967378317, None, 16158, 16157),
    ]
    for acc_v, a_bits, w_bits, want_f, want_b, other_b in cases:
        a_s, w_s = u(a_bits), u(w_bits)
        yb, yf = oracle.c_w8a8_epilogue(np.array([[acc_v]], np.int32), np.array([a_s]), np.array([w_s]))
        ref = np.float32(np.float32(np.float32(acc_v) * a_s) * w_s)
        alt = np.float32(np.float32(acc_v) * np.float32(a_s * w_s))
        assert ref != alt  # the vector does separate the two orders
        assert yf[0, 0] == ref and yf[0, 0] != alt
        if want_f is not None:
            assert yf[0, 0] == np.float32(want_f)
        assert yb[0, 0] == want_b and yb[0, 0] != other_b
        # numpy restatement agrees
        assert oracle.w8a8_epilogue_f32(np.array([[acc_v]], np.int32), np.array([a_s]), np.array([w_s]))[0, 0] == ref


def test_w8a8_epilogue_bias_is_fused_fma():
    acc = np.array([[1 << 24 | 1]], np.int32)
    a_s = np.array([1.0], np.float32)
    w_s = np.array([1.0 + 2.0 ** -23], np.float32)
    bias = np.array([-float(np.float32((1 << 24 | 1)))], np.float32)
    _, yf = oracle.c_w8a8_epilogue(acc, a_s, w_s, bias)
    p = np.float64(np.float32(1 << 24 | 1))  # float(acc) rounds to 16777216
    assert yf[0, 0] == np.float32(p * (1.0 + 2.0 ** -23) + float(bias[0]))  # exact fma result


# ------------------------------------------------------------ torch paths

def test_w8a16_torch_path_close_to_exact():
    x = make_activations(32, 1024, seed=10, outlier_frac=0.0)
    q, s = make_weights(256, 1024, seed=11)
    y = oracle.w8a16_torch_path(x, q, s)
    y64 = oracle.w8a16_f64(f32(x), q.numpy(), s.numpy())
    assert oracle.rel_l2(f32(y), y64) < 5e-3
    y64c = oracle.c_w8a16_f64(bits16(x), q.numpy(), s.numpy())
    np.testing.assert_allclose(y64c, y64, rtol=1e-12, atol=1e-12)


def test_w8a16_f64_brute_force():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 5)).astype(np.float32)
    xb = oracle.f32_to_bf16_bits(x)
    xr = oracle.bf16_bits_to_f32(xb)
    q = rng.integers(-127, 128, (4, 5)).astype(np.int8)
    s = rng.uniform(0.01, 0.1, 4).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = oracle.c_w8a16_f64(xb, q, s, b)
    for i, j in itertools.product(range(3), range(4)):
        e = sum(float(xr[i, t]) * int(q[j, t]) for t in range(5)) * float(s[j]) + float(b[j])
        assert abs(y[i, j] - e) <= 1e-12 * max(1.0, abs(e))


def test_w8a8_torch_path_close_to_exact():
    x = make_activations(64, 1024, seed=13)
    xq, a_s = oracle.quantize_rows(f32(x))
    q, w_s = make_weights(128, 1024, seed=14)
    y = oracle.w8a8_torch_path(torch.from_numpy(xq), torch.from_numpy(a_s), q, w_s, None, torch.bfloat16)
    y64 = oracle.w8a8_f64(xq, a_s, q.numpy(), w_s.numpy())
    assert oracle.rel_l2(f32(y), y64) < 1e-2
    # and the bit-exact kernel epilogue is closer to exact than the torch path
    yb, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q.numpy()), a_s, w_s.numpy())
    assert oracle.rel_l2(oracle.bf16_bits_to_f32(yb), y64) <= oracle.rel_l2(f32(y), y64)


def test_fp32_scale_torch_models_match_exact_and_c_epilogue():
    """The model-level helpers restating the kernels' fp32-scale numerics:
    W8A8 equals the C epilogue up to the unfused bias-free fma (<= 1 bf16 ulp
    on ties of the two roundings); W8A16 is within fp32 summation error of
    the fp64 product."""
    x = make_activations(16, 512, seed=15)
    xq, a_s = oracle.quantize_rows(f32(x))
    q, w_s = make_weights(96, 512, seed=16)
    y = oracle.w8a8_fp32_scale_torch(torch.from_numpy(xq), torch.from_numpy(a_s), q, w_s, None, torch.bfloat16)
    yb, _ = oracle.c_w8a8_epilogue(oracle.c_gemm_i32(xq, q.numpy()), a_s, w_s.numpy())
    got, ref = f32(y), oracle.bf16_bits_to_f32(yb)
    assert np.mean(got == ref) > 0.999
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7)
    y16 = oracle.w8a16_fp32_scale_torch(x, q, w_s)
    y64 = oracle.w8a16_f64(f32(x), q.numpy(), w_s.numpy())
    assert np.all(np.abs(f32(y16) - y64) <= np.abs(y64) * 2.0 ** -8 + 1e-6 * np.abs(y64).max())


# ------------------------------------------------------------ producers

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_ref_matches_reference_torch_expression(dtype):
    """oracle.rmsnorm_ref against the reference's torch ops (layernorm.py:16-40)
    run by CPU torch: residual bit-exact, y within one ulp (fp64 vs fp32
    statistics), almost all bit-exact; plus closed-form special cases."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(64, 1024, generator=g).to(dtype)
    r = torch.randn(64, 1024, generator=g).to(dtype)
    w = (torch.rand(1024, generator=g) + 0.5).to(dtype)
    h = x.float() + r.float()
    res_t = h.to(dtype)
    y_t = (h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-6)).to(dtype) * w
    y, res = oracle.rmsnorm_ref(f32(x), f32(w), 1e-6, f32(r), is_bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(res, f32(res_t))
    assert np.mean(y == f32(y_t)) > 0.999
    # a constant row c normalises to sign(c) (eps negligible): y = w exactly
    yc, _ = oracle.rmsnorm_ref(np.full((1, 64), 3.0, np.float32), np.full(64, 0.75, np.float32), 0.0)
    assert np.all(yc == 0.75)
    # zero row -> zeros
    yz, _ = oracle.rmsnorm_ref(np.zeros((1, 16), np.float32), np.ones(16, np.float32), 1e-6)
    assert np.all(yz == 0)


def test_silu_mul_ref_matches_torch_and_closed_forms():
    g = torch.Generator().manual_seed(22)
    gu = (torch.randn(32, 2048, generator=g) * 3).bfloat16()
    a, b = gu.float().chunk(2, -1)
    y_t = (torch.nn.functional.silu(a) * b).bfloat16()
    y = oracle.silu_mul_ref(f32(gu))
    assert np.mean(y == f32(y_t)) > 0.999
    # gate | up = [0, ln 3 | 5, 1]: silu(0) * 5 = 0; silu(ln 3) * 1 = ln3 / (1 + 1/3) = 0.75 ln 3
    v = np.array([[0.0, np.log(3.0), 5.0, 1.0]], np.float32)
    out = oracle.silu_mul_ref(v)
    assert out[0, 0] == 0.0
    assert out[0, 1] == oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(np.float32(0.75 * np.log(3.0))))


# ------------------------------------------------------------ golden fixtures

def _golden_files():
    return sorted(GOLDEN.glob("*.npz"))


def test_golden_fixtures_present():
    assert _golden_files(), "tests/golden/*.npz missing; run tests/golden/make_golden.py"


@pytest.mark.parametrize("path", _golden_files(), ids=lambda p: p.stem)
def test_golden_fixture(path):
    d = np.load(path, allow_pickle=False)
    kind = str(d["kind"])
    if kind == "act_quant":
        q, s = oracle.c_act_quant(d["x_bits"], is_bf16=bool(d["is_bf16"]))
        np.testing.assert_array_equal(q, d["xq"])
        np.testing.assert_array_equal(s.view(np.uint32), d["a_scales"].view(np.uint32))
        q2, s2 = oracle.quantize_rows(oracle.to_f32(d["x_bits"], bool(d["is_bf16"])))
        np.testing.assert_array_equal(q2, d["xq"])
    elif kind == "w8a8":
        acc = oracle.c_gemm_i32(d["xq"], d["qweight"])
        np.testing.assert_array_equal(acc, d["acc"])
        yb, _ = oracle.c_w8a8_epilogue(acc, d["a_scales"], d["w_scales"])
        np.testing.assert_array_equal(yb, d["y_bits"])
    elif kind == "w8a16":
        y = oracle.c_w8a16_f64(d["x_bits"], d["qweight"], d["scales"])
        np.testing.assert_allclose(y, d["y_f64"], rtol=1e-12, atol=1e-12)
    elif kind == "kat":
        q, s = oracle.quantize_rows(d["x"])
        np.testing.assert_array_equal(q, d["q"])
        np.testing.assert_array_equal(s, d["s"])
    else:
        pytest.fail(f"unknown fixture kind {kind}")


def test_gemm_i32_blas_exact():
    """The float64-BLAS accumulator equals the integer loops bit for bit,
    including all-extreme rows at the largest K (|acc| = 127*127*12288)."""
    rng = np.random.default_rng(21)
    for m, n, k in ((7, 33, 40), (64, 96, 4096), (5, 17, 12288)):
        xq = rng.integers(-127, 128, (m, k)).astype(np.int8)
        w = rng.integers(-127, 128, (n, k)).astype(np.int8)
        xq[0] = 127
        w[0] = -127
        w[1] = 127
        got = oracle.gemm_i32_blas(xq, w)
        np.testing.assert_array_equal(got, oracle.c_gemm_i32(xq, w))
        np.testing.assert_array_equal(got, oracle.gemm_i32(xq, w))
        assert got[0, 0] == -127 * 127 * k and got[0, 1] == 127 * 127 * k


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rounded_weights_match_reference_expression(dtype):
    """w8a16_rounded_weights == CPU torch running the reference's dequant
    expression qweight.to(T) * scales.to(T)[:, None] (cuda.py:293-300), bit for
    bit, over scales spanning several binades and every int8 code."""
    rng = np.random.default_rng(11)
    q = np.tile(np.arange(-127, 128, dtype=np.int8), (64, 1))
    s = (rng.random(64) * 10.0 ** rng.integers(-5, 0, size=64)).astype(np.float32) + np.float32(1e-6)
    got = oracle.w8a16_rounded_weights(q, s, is_bf16=dtype == torch.bfloat16)
    ref = (torch.from_numpy(q).to(dtype) * torch.from_numpy(s).to(dtype)[:, None]).float().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rounded_weights_closed_forms():
    q = np.array([[-127, -1, 0, 1, 5, 127]], dtype=np.int8)
    # power-of-two scale: every product is exact in both types
    for bf in (True, False):
        wd = oracle.w8a16_rounded_weights(q, np.array([2.0 ** -10], np.float32), is_bf16=bf)
        assert np.array_equal(wd, q.astype(np.float32) * np.float32(2.0 ** -10))
    # q = 1 gives the rounded scale itself; 3 * bf16(1/3) rounds once more
    s = np.array([1.0 / 3.0], np.float32)
    wd = oracle.w8a16_rounded_weights(np.array([[1, 3]], np.int8), s, is_bf16=True)
    s_bf = np.float32(0.333984375)              # bf16(1/3) = 0x3EAB
    assert wd[0, 0] == s_bf
    assert wd[0, 1] == np.float32(1.0)          # 3 * 0.333984375 = 1.001953125 -> bf16 1.0
    wd16 = oracle.w8a16_rounded_weights(np.array([[3]], np.int8), s, is_bf16=False)
    assert wd16[0, 0] == np.float32(np.float16(3 * np.float32(np.float16(1.0 / 3.0))))


def test_rounded_f64_brute_force_tiny():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 7)).astype(np.float32)
    wd = rng.standard_normal((4, 7)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y = oracle.w8a16_rounded_f64(x, wd, b)
    for m in range(3):
        for n in range(4):
            assert y[m, n] == pytest.approx(sum(float(x[m, k]) * float(wd[n, k]) for k in range(7)) + float(b[n]),
                                            rel=1e-15, abs=1e-15)


@pytest.mark.parametrize("is_bf16", [True, False])
def test_rounded_weights_c_matches_numpy(is_bf16):
    """The two restatements of the rounded dequantization agree bit for bit."""
    rng = np.random.default_rng(21)
    q = rng.integers(-127, 128, size=(96, 255), dtype=np.int8)
    q[:, :255] = np.tile(np.arange(-127, 128, dtype=np.int8), (96, 1))
    s = (rng.random(96) * 10.0 ** rng.integers(-6, 1, size=96)).astype(np.float32)
    s[:4] = np.float32([2.0 ** -12, 1.0 / 3.0, 65504.0 / 127.0, 1e-7])
    bits = oracle.c_w8a16_rounded_weights(q, s, is_bf16=is_bf16)
    got = oracle.to_f32(bits, is_bf16)
    want = oracle.w8a16_rounded_weights(q, s, is_bf16=is_bf16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_c_f16_rounding_matches_numpy():
    """The C float -> half RNE (used by the rounded-dequant restatement) equals
    numpy's conversion on random values across the half range, the subnormal
    range, exact ties and overflow."""
    rng = np.random.default_rng(8)
    x = np.concatenate([
        (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 5, size=20000)).astype(np.float32),
        np.float32([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                    2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf]),
    ])
    got = oracle.c_f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("is_bf16", [True, False], ids=["bf16", "fp16"])
def test_divide_free_quant_code_is_exact_for_every_input(is_bf16):
    """The act-quant and producer kernels compute the per-token code without a
    divide (csrc/tvq_common.h quant_code: d = x*rs, one fma correction, rint).
    Over every finite non-negative 16-bit pair x <= amax (the code is odd in x)
    with s = max(amax/127, 1e-8), it must equal utils.py:28-32's
    rint(x / s) exactly; the plain rint(x * rs) must not (so the check can fail)."""
    bad, pairs = oracle.c_quant_code_sweep(is_bf16, variant=0)
    assert pairs == (532701120 if is_bf16 else 503856640)
    assert bad == 0
    plain_bad, _ = oracle.c_quant_code_sweep(is_bf16, variant=1)
    assert plain_bad > 1000
