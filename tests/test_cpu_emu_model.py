"""The Qwen3 model's device path on the CPU emulation of the kernels (see
tests/cpu_emu/model_cases.py for the cases): prefill projections against the
oracle with every W8A8 projection fed fused codes (o_proj's from the
attention kernel), the gate_up GEMM with the SiLU epilogue bit-identical to
the unfused path, greedy KV-cache decode equal to recomputation, and the
device path close to the host path; at the test architecture and, for W8A8,
the 28-layer Qwen3-0.6B one. It runs in a child process: the script makes
every tensor of its process report is_cuda=True so that the model takes its
device path."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "cpu_emu"))
import emu  # noqa: E402

if not Path(emu.CLANG).exists():  # pragma: no cover
    pytest.skip("host clang of the ROCm toolchain not found", allow_module_level=True)


def test_model_device_path_on_emulated_kernels():
    emu.ensure_built()
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "tiny-vllm_amd")]))
    proc = subprocess.run([sys.executable, str(ROOT / "tests" / "cpu_emu" / "model_cases.py")], env=env,
                          capture_output=True, text=True, timeout=1200)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-5000:]
    assert "all cases passed" in proc.stdout
