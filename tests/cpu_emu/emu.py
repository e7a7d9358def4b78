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

_LIBS: dict[bool, ctypes.CDLL] = {}
CLANG = "/opt/rocm/llvm/bin/clang++"


def lib_path(asan: bool = False) -> Path:
    return HERE / "_build" / ("libtvq_emu_asan.so" if asan else "libtvq_emu.so")


def ensure_built(asan: bool = False) -> Path:
    """Build the emulated library when it is missing or older than a kernel or emulation source."""
    import fcntl
    path = lib_path(asan)
    srcs = list((ROOT / "tiny-vllm_amd" / "csrc").iterdir()) + [HERE / "emu_runtime.cpp",
                                                               HERE / "hip" / "hip_runtime.h", HERE / "build.py"]
    (HERE / "_build").mkdir(exist_ok=True)
    with open(HERE / "_build" / ".lock", "w") as lk:   # one builder at a time (pytest -n workers)
        fcntl.flock(lk, fcntl.LOCK_EX)
        if not path.is_file() or path.stat().st_mtime < max(p.stat().st_mtime for p in srcs):
            sys.path.insert(0, str(HERE))
            import build as emu_build  # tests/cpu_emu/build.py
            emu_build.build(asan)
    return path


def load(asan: bool = False) -> ctypes.CDLL:
    """The emulated library (built first when missing or stale), typed as the product's C ABI."""
    if asan in _LIBS:
        return _LIBS[asan]
    path = ensure_built(asan)
    lib = ctypes.CDLL(str(path))
    from nanovllm.quantization._hip import SYMBOLS
    for name, restype, argtypes in SYMBOLS:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = list(argtypes)
    _LIBS[asan] = lib
    return lib


def ptr(t):
    return None if t is None else t.data_ptr()


def check(lib, rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: rc={rc}: {lib.tvq_last_error().decode()}")
