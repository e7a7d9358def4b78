"""The CPU emulation's race checker (tests/cpu_emu/racecheck.h): the kernel
sources compiled with the compiler's memory-access instrumentation, every
access checked against the GPU's ordering rules (barrier intervals between
waves, no order between workgroups of a launch, lockstep within a wave, LDS
DMA from issue to its wave's wait).

  * probe kernels (tests/cpu_emu/race_probe): each kind of race is reported
    and its correctly synchronised twin is not, with DMA landing at issue
    and at the wave's wait;
  * three mutants of the product kernels, each a synchronisation bug: a
    dropped barrier in the producers' cross-wave row reduction, a DMA stage
    wait one stage too short (wrong values only when DMA lands late), the
    split-K partial images stored plainly instead of atomically (right
    values in every emulation mode: only the ordering is wrong). The
    race-checking run of their cases fails with reports.

The clean kernels run race-checked in tests/test_cpu_emu_kernels.py
(test_kernels_in_child_modes), every family, with no report allowed."""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
EMU = ROOT / "tests" / "cpu_emu"
sys.path.insert(0, str(EMU))
import build as emu_build  # noqa: E402
import emu  # noqa: E402

if not Path(emu.CLANG).exists():  # pragma: no cover
    pytest.skip("host clang of the ROCm toolchain not found", allow_module_level=True)

RACY = {0: "LDS across waves, no barrier", 3: "two workgroups, one word", 5: "plain write, atomic read elsewhere",
        7: "own DMA read before its wait", 9: "other wave reads DMA data, no barrier",
        11: "DMA refills a buffer another wave reads"}
SAFE = {1: "LDS across waves, barrier", 2: "LDS within a wave", 4: "two workgroups, atomics",
        6: "disjoint workgroups", 8: "own DMA read after the wait", 10: "other wave reads after a barrier",
        12: "refill after a barrier"}

_RUN_PROBES = """
import ctypes, json, sys
lib = ctypes.CDLL(sys.argv[1])
out = {}
for w in range(13):
    buf = (ctypes.c_int * 1024)(*range(1024))
    before = lib.tvq_emu_race_reports()
    assert lib.race_probe(w, buf) == 0
    out[w] = lib.tvq_emu_race_reports() - before
print(json.dumps(out))
"""


def _env(**kw) -> dict:
    return dict(os.environ, PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "tiny-vllm_amd")]), **kw)


def test_checker_reports_races_and_only_races():
    lib = emu_build.build(race=True, csrc=EMU / "race_probe", name="probe")
    for dma in ("late", "issue"):
        proc = subprocess.run([sys.executable, "-c", _RUN_PROBES, str(lib)], env=_env(EMU_DMA=dma),
                              capture_output=True, text=True, timeout=300)
        assert proc.returncode == 0, proc.stderr[-3000:]
        counts = {int(k): v for k, v in json.loads(proc.stdout.strip().splitlines()[-1]).items()}
        # with DMA landing at issue, a wave's own early read sees the data: no race
        racy = {k for k in RACY if not (dma == "issue" and k == 7)}
        missed = [RACY[k] for k in racy if counts[k] == 0]
        false = [f"{SAFE.get(k, RACY.get(k))}: {counts[k]}" for k in counts if k not in racy and counts[k]]
        assert not missed and not false, (dma, missed, false, emu.symbolize(proc.stderr)[-3000:])


MUTANTS = {
    # the producers' cross-wave reduction reads the other waves' partial sums without the barrier
    "barrier": ("producers.hip", "lds[threadIdx.x / kWave] = v;\n    __syncthreads();",
                "lds[threadIdx.x / kWave] = v;", "producers"),
    # the DMA pipeline waits for one stage fewer than the one it consumes
    "stage_wait": ("gemm_dma_kernel.h", "      wait_vm<LPW * A>();\n      return;",
                   "      wait_vm<LPW * A + LPW>();\n      return;", "dma"),
    # split-K partial images stored plainly: the last workgroup's reads are not ordered after them
    "splitk_store": ("gemm_dma_kernel.h",
                     "__hip_atomic_store(img(own, i, j, q, e), (E)acc[i][j][4 * q + e], __ATOMIC_RELAXED,\n"
                     "                                 __HIP_MEMORY_SCOPE_AGENT);",
                     "*img(own, i, j, q, e) = (E)acc[i][j][4 * q + e];", "gemm"),
}


def test_checker_catches_kernel_mutants(tmp_path):
    def make(key):
        f, old, new, _ = MUTANTS[key]
        src = tmp_path / key / "csrc"
        shutil.copytree(ROOT / "tiny-vllm_amd" / "csrc", src)
        text = (src / f).read_text()
        assert text.count(old) == 1, (key, "mutation site not found")
        (src / f).write_text(text.replace(old, new))
        return emu_build.build(race=True, csrc=src, name=f"mut_{key}", jobs=4)

    with ThreadPoolExecutor(len(MUTANTS)) as ex:
        libs = dict(zip(MUTANTS, ex.map(make, MUTANTS)))
    script = str(EMU / "child_cases.py")
    for key, lib in libs.items():
        proc = subprocess.run([sys.executable, script, "--race", "--lib", str(lib), "--only", MUTANTS[key][3]],
                              env=_env(EMU_DMA="late"), capture_output=True, text=True, timeout=600)
        assert proc.returncode != 0 and "emu race" in proc.stderr, (key, proc.stdout[-1000:], proc.stderr[-2000:])
