"""ctypes loader of the CPU-emulated kernel library (test infrastructure).

`load()` returns the library built by tests/cpu_emu/build.py from the
unchanged kernel sources, typed with the product's own symbol table, so a
test calls the same C ABI as on the GPU, with host (CPU torch) pointers."""
from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for _p in (str(ROOT), str(ROOT / "tiny-vllm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

_LIBS: dict[tuple, ctypes.CDLL] = {}
CLANG = "/opt/rocm/llvm/bin/clang++"


def lib_path(asan: bool = False, race: bool = False) -> Path:
    return HERE / "_build" / ("libtvq_emu_asan.so" if asan else "libtvq_emu_race.so" if race else "libtvq_emu.so")


def ensure_built(asan: bool = False, race: bool = False) -> Path:
    """Build the emulated library when it is missing or older than a kernel or emulation source."""
    import fcntl
    path = lib_path(asan, race)
    srcs = list((ROOT / "tiny-vllm_amd" / "csrc").iterdir()) + [
        HERE / f for f in ("emu_runtime.cpp", "racecheck.cpp", "racecheck.h", "hip/hip_runtime.h", "build.py")]
    (HERE / "_build").mkdir(exist_ok=True)
    with open(HERE / "_build" / ".lock", "w") as lk:   # one builder at a time (pytest -n workers)
        fcntl.flock(lk, fcntl.LOCK_EX)
        if not path.is_file() or path.stat().st_mtime < max(p.stat().st_mtime for p in srcs):
            sys.path.insert(0, str(HERE))
            import build as emu_build  # tests/cpu_emu/build.py
            emu_build.build(asan, race=race)
    return path


def load(asan: bool = False, race: bool = False) -> ctypes.CDLL:
    """The emulated library (built first when missing or stale), typed as the product's C ABI."""
    if (asan, race) in _LIBS:
        return _LIBS[(asan, race)]
    lib = load_file(ensure_built(asan, race))
    _LIBS[(asan, race)] = lib
    return lib


def load_file(path) -> ctypes.CDLL:
    """An emulation library built elsewhere (e.g. from modified sources), typed as the product's C ABI."""
    lib = ctypes.CDLL(str(path))
    from nanovllm.quantization._hip import SYMBOLS
    for name, restype, argtypes in SYMBOLS:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = list(argtypes)
    return lib


def ptr(t):
    return None if t is None else t.data_ptr()


def check(lib, rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: rc={rc}: {lib.tvq_last_error().decode()}")



def symbolize(text: str) -> str:
    """Race reports with each `? (lib.so+0xOFF)` replaced by the function and
    source line, and the outermost caller when inlined (llvm-symbolizer of
    the ROCm toolchain)."""
    import re
    import subprocess
    tool = Path(CLANG).parent / "llvm-symbolizer"
    if not tool.exists():
        return text

    def frame(fn: str, loc: str) -> str:
        fn = fn.replace("(anonymous namespace)::", "")
        depth, cut = 0, len(fn)
        for i, c in enumerate(fn):  # drop the argument list
            if c == "<":
                depth += 1
            elif c == ">":
                depth -= 1
            elif c == "(" and depth == 0:
                cut = i
                break
        return f"{fn[:cut].strip()} {loc.split('/_build/')[-1].split('/', 1)[-1]}"

    def one(m):
        lib = HERE / "_build" / m.group(2)
        out = subprocess.run([str(tool), f"--obj={lib}", m.group(3)], capture_output=True, text=True).stdout
        lines = [ln for ln in out.splitlines() if ln.strip()]
        frames = [frame(lines[i], lines[i + 1]) for i in range(0, len(lines) - 1, 2)]
        if not frames:
            return m.group(0)
        return frames[0] + (f" in {frames[-1]}" if len(frames) > 1 else "")
    return re.sub(r"(\S+ )?\((libtvq_emu\w*\.so)\+(0x[0-9a-f]+)\)", one, text)
