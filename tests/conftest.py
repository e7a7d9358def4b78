import os
import sys
from pathlib import Path

import pytest

# Native failures raise instead of falling back to the torch path, so no parity
# check can pass on the fallback.
os.environ.setdefault("NANOVLLM_NATIVE_STRICT", "1")

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "tiny-vllm_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


# TVQ_GPU_TESTS_ON_EMU=1: the -m gpu tests run on the CPU emulation of the
# kernels (tests/cpu_emu/gpu_on_emu.py), CPU tensors standing in for device
# ones; with TVQ_EMU_RACE=1 (and EMU_DMA=late) on its race-checking build,
# each test failing if it adds a race report.
ON_EMU = os.environ.get("TVQ_GPU_TESTS_ON_EMU") == "1"
EMU_RACE = ON_EMU and os.environ.get("TVQ_EMU_RACE") == "1"
if ON_EMU:
    sys.path.insert(0, str(ROOT / "tests" / "cpu_emu"))
    import emu
    import gpu_on_emu
    _EMU_LIB = emu.load(race=EMU_RACE)
    gpu_on_emu.install(_EMU_LIB)

    @pytest.fixture(autouse=True)
    def _emu_race_reports():
        before = _EMU_LIB.tvq_emu_race_reports() if EMU_RACE else 0
        yield
        if EMU_RACE:
            assert _EMU_LIB.tvq_emu_race_reports() == before, "race report(s) on stderr"


@pytest.fixture(scope="session")
def hiplib():
    """The built C-ABI library (built on demand if absent)."""
    from nanovllm.quantization import _hip
    if ON_EMU:
        return _hip.load_library()
    if not _hip.library_path().is_file():
        sys.path.insert(0, str(PKG))
        import build as tvq_build
        tvq_build.build()
    return _hip.load_library()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible ROCm device")
    return torch.device("cuda", 0)
