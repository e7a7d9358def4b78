"""Writes the small golden fixtures under tests/golden/.

The reference ships no golden vectors, fixtures or known-answer tests for this
path (no tests/ directory at all), so these fixtures are of two kinds:

* kat_*.npz  known-answer vectors whose expected outputs are fixed by hand
  from the quantizer's definition (utils.py:21-32): exact ties, zero rows,
  saturating rows, eps-floored rows; independent of any implementation;
* act_quant_*.npz, w8a8_*.npz, w8a16_*.npz  seeded input/output vectors
  produced by the oracle (numpy restatement), frozen so that later changes to
  either oracle implementation are caught and the GPU path can be checked
  against stored outputs.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402


def kat() -> None:
    # Row 0: amax 127 -> s = 1 exactly; ties go to even.
    # Row 1: all zero -> s = eps (fp32(1e-8)), q = 0.
    # Row 2: amax 254 -> s = 2; x/s hits exact ties: 1/2 -> 0, 3/2 -> 2, 5/2 -> 2, -253/2 -> -126.
    # Row 3: amax/127 < eps -> s = eps; values quantize against 1e-8 (no ties).
    x = np.array([
        [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5],
        [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
        [254.0, 1.0, 3.0, 5.0, -1.0, -3.0, -253.0, 0.0],
        [5e-7, -5e-7, 3.1e-8, 1.4e-8, 0.0, 4e-9, -6e-9, 1.26e-6],
    ], np.float32)
    q = np.array([
        [127, 0, 2, 2, 0, -2, -2, 126],
        [0, 0, 0, 0, 0, 0, 0, 0],
        [127, 0, 2, 2, 0, -2, -126, 0],
        [50, -50, 3, 1, 0, 0, -1, 126],
    ], np.int8)
    eps = np.float32(1e-8)
    s = np.array([1.0, eps, 2.0, eps], np.float32)
    np.savez(HERE / "kat_quantizer.npz", kind="kat", x=x, q=q, s=s)


def seeded() -> None:
    rng = np.random.default_rng(20261201)
    # act-quant: bf16 and fp16 rows with outlier columns
    for name, is_bf16 in (("bf16", True), ("fp16", False)):
        x = rng.standard_normal((8, 96)).astype(np.float32)
        x[:, rng.choice(96, 3, replace=False)] *= 20
        x[3] = 0
        bits = oracle.f32_to_bf16_bits(x) if is_bf16 else x.astype(np.float16).view(np.uint16)
        q, s = oracle.quantize_rows(oracle.to_f32(bits, is_bf16))
        np.savez(HERE / f"act_quant_{name}.npz", kind="act_quant", x_bits=bits, is_bf16=is_bf16, xq=q, a_scales=s)
    # W8A8 GEMM: accumulators and bf16 outputs
    xb = oracle.f32_to_bf16_bits(rng.standard_normal((5, 128)).astype(np.float32))
    xq, a_s = oracle.quantize_rows(oracle.bf16_bits_to_f32(xb))
    w = (rng.standard_normal((24, 128)) * 0.02).astype(np.float32)
    qw, w_s = oracle.quantize_rows(w)
    acc = oracle.gemm_i32(xq, qw)
    y = oracle.w8a8_epilogue_bf16(acc, a_s, w_s)
    np.savez(HERE / "w8a8_small.npz", kind="w8a8", xq=xq, a_scales=a_s, qweight=qw, w_scales=w_s, acc=acc, y_bits=y)
    # W8A16: exact fp64 product
    xb = oracle.f32_to_bf16_bits(rng.standard_normal((3, 64)).astype(np.float32))
    w = (rng.standard_normal((16, 64)) * 0.02).astype(np.float32)
    qw, s = oracle.quantize_rows(w)
    y = oracle.w8a16_f64(oracle.bf16_bits_to_f32(xb), qw, s)
    np.savez(HERE / "w8a16_small.npz", kind="w8a16", x_bits=xb, qweight=qw, scales=s, y_f64=y)


if __name__ == "__main__":
    kat()
    seeded()
    print(sorted(p.name for p in HERE.glob("*.npz")))
