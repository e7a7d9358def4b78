"""Build the kernel sources of tiny-vllm_amd/csrc for the CPU emulation
(test infrastructure: hip/hip_runtime.h, emu_runtime.cpp).

The sources are copied unchanged except for these mechanical rewrites, which
host C++ cannot express:
  * kernel<<<grid, block, shmem, stream>>>(args)  ->  ::emu::launch(&kernel, grid, block, shmem, stream, args)
  * inline asm: "s_barrier" -> ::emu::barrier(); a vmcnt(N) wait ->
    ::emu::wait_vm(N); an LDS wait (lgkmcnt) -> ::emu::wave_barrier();
    register pins dropped
  * __attribute__((address_space(N))) and the amdgpu_* kernel attributes dropped
  * extern __shared__ T name[]  ->  T* name = (T*)::emu::dyn_smem(), and a
    static __shared__ T name[..] -> a reference to this workgroup's own
    storage (::emu::lds), so concurrently resident workgroups do not share it
and compiled with the host clang into tests/cpu_emu/_build/libtvq_emu[_asan|_race].so,
which exports the same C ABI as the product library (include/tvq.h). The
_asan build instruments everything for AddressSanitizer. The _race build
compiles the kernel sources with the compiler's ThreadSanitizer
instrumentation (every memory access becomes a call) and links the calls to
racecheck.cpp, which checks each access against the GPU's ordering rules;
no sanitizer runtime is involved.

Usage: python tests/cpu_emu/build.py [--asan | --race]
"""
from __future__ import annotations

import argparse
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CSRC = ROOT / "tiny-vllm_amd" / "csrc"
INCLUDE = ROOT / "include"
BUILD = HERE / "_build"
CLANG = "/opt/rocm/llvm/bin/clang++"


def _match(text: str, i: int, open_c: str, close_c: str) -> int:
    """Index just past the bracket closing the one at text[i]."""
    depth = 0
    j = i
    while j < len(text):
        c = text[j]
        if c == '"':
            j = text.index('"', j + 1)
        elif c == open_c:
            depth += 1
        elif c == close_c:
            depth -= 1
            if depth == 0:
                return j + 1
        j += 1
    raise ValueError("unbalanced")


def _rewrite_launches(src: str) -> str:
    out = []
    pos = 0
    while True:
        i = src.find("<<<", pos)
        if i < 0:
            out.append(src[pos:])
            return "".join(out)
        # kernel expression: identifier chars / :: and balanced template arguments, backwards
        j = i
        while True:
            if j > 0 and src[j - 1] == ">":
                depth = 0
                k = j - 1
                while k >= 0:
                    if src[k] == ">":
                        depth += 1
                    elif src[k] == "<":
                        depth -= 1
                        if depth == 0:
                            break
                    k -= 1
                j = k
                continue
            if j > 0 and (src[j - 1].isalnum() or src[j - 1] in "_:"):
                j -= 1
                continue
            break
        kern = src[j:i]
        cfg_end = src.index(">>>", i)
        cfg = src[i + 3:cfg_end]
        p = cfg_end + 3
        while src[p].isspace():
            p += 1
        assert src[p] == "(", src[i - 40:p + 10]
        q = _match(src, p, "(", ")")
        args = src[p + 1:q - 1]
        out.append(src[pos:j])
        out.append(f"[&] {{ auto* emu_k = &{kern}; ::emu::launch(emu_k, {cfg}, {args}); }}()")
        pos = q


def _rewrite_asm(src: str) -> str:
    out = []
    pos = 0
    pat = re.compile(r"\basm\b\s*(volatile\s*)?\(")
    while True:
        m = pat.search(src, pos)
        if not m:
            out.append(src[pos:])
            return "".join(out)
        start = m.start()
        q = _match(src, m.end() - 1, "(", ")")
        body = src[m.end():q - 1]
        lit = re.match(r'\s*"([^"]*)"', body)
        text = lit.group(1) if lit else ""
        end = q
        while end < len(src) and src[end].isspace():
            end += 1
        if end < len(src) and src[end] == ";":
            end += 1
        out.append(src[pos:start])
        repl = ""
        vm = re.search(r"vmcnt\((\d+|%0)\)", text)
        if vm:
            n = vm.group(1)
            if n == "%0":
                n = re.search(r'"n"\s*\((.*?)\)\s*(?::|$)', body, re.S).group(1)
            repl += f"::emu::wait_vm({n});"
        if "s_barrier" in text:
            repl += "::emu::barrier();"
        elif "lgkmcnt" in text:
            repl += "::emu::wave_barrier();"
        out.append(repl or ";")
        pos = end


def _split_top(text: str) -> list[str]:
    parts, depth, cur = [], 0, ""
    for c in text:
        if c in "[(<":
            depth += 1
        elif c in "])>":
            depth -= 1
        if c == "," and depth == 0:
            parts.append(cur)
            cur = ""
        else:
            cur += c
    parts.append(cur)
    return [p.strip() for p in parts]


def _rewrite_static_shared(src: str) -> str:
    """`__shared__ [attrs] TYPE a[..], b;` -> references to per-workgroup
    storage: `TYPE (&a)[..] = ::emu::lds<TYPE[..]>(key); TYPE (&b) = ...`."""
    out, pos = [], 0
    pat = re.compile(r"(?<!extern )\b__shared__\b")
    while True:
        m = pat.search(src, pos)
        if not m:
            out.append(src[pos:])
            return "".join(out)
        end = src.index(";", m.end())
        body = re.sub(r"__attribute__\(\((?:[^()]|\([^()]*\))*\)\)", " ", src[m.end():end]).strip()
        decls = _split_top(body)
        first = re.match(r"(.*?)\b([A-Za-z_]\w*)\s*((?:\[[^\]]*\]\s*)*)$", decls[0], re.S)
        assert first, decls[0]
        ty = first.group(1).strip()
        items = [(first.group(2), first.group(3).strip())]
        for d in decls[1:]:
            mm = re.match(r"([A-Za-z_]\w*)\s*((?:\[[^\]]*\]\s*)*)$", d, re.S)
            assert mm, d
            items.append((mm.group(1), mm.group(2).strip()))
        key = "([] { static const char emu_tag = 0; return (const void*)&emu_tag; }())"
        repl = " ".join(f"{ty} (&{name}){dims} = ::emu::lds<{ty}{dims}>({key});" for name, dims in items)
        out.append(src[pos:m.start()])
        out.append(repl)
        pos = end + 1


def rewrite(src: str) -> str:
    src = _rewrite_launches(src)
    src = _rewrite_asm(src)
    src = re.sub(r"__attribute__\(\(address_space\(\d\)\)\)", "", src)
    src = re.sub(r"__attribute__\(\(amdgpu_\w+\((?:[^()]|\([^()]*\))*\)\)\)", "", src)
    src = re.sub(r"extern\s+__shared__\s+(?:__attribute__\(\(aligned\(\d+\)\)\)\s+)?(\w+)\s+(\w+)\[\]\s*;",
                 r"\1* \2 = reinterpret_cast<\1*>(::emu::dyn_smem());", src)
    src = _rewrite_static_shared(src)
    return src


def _suffix(asan: bool, race: bool) -> str:
    return "_asan" if asan else "_race" if race else ""


def build(asan: bool = False, jobs: int = 8, csrc: Path = CSRC, include: Path = INCLUDE, name: str = "",
          race: bool = False) -> Path:
    """Compile `csrc` (default: the package's kernel sources) into the
    emulation library; `name` gives another library name (e.g. for sources
    of another revision)."""
    assert not (asan and race)
    stage = BUILD / ((name or "src") + _suffix(asan, race))
    if stage.exists():
        shutil.rmtree(stage)
    (stage / "tiny-vllm_amd" / "csrc").mkdir(parents=True)
    shutil.copytree(include, stage / "include")
    for f in csrc.iterdir():
        if f.suffix in (".hip", ".h"):
            (stage / "tiny-vllm_amd" / "csrc" / (f.stem + (".cpp" if f.suffix == ".hip" else ".h"))).write_text(
                rewrite(f.read_text()))
    flags = ["-std=c++17", "-fPIC", "-g", "-O1" if asan or race else "-O2", "-ffp-contract=off", "-fno-fast-math",
             "-Wno-unused-value", "-Wno-ignored-attributes", "-Wno-unknown-attributes", "-Wno-unused-command-line-argument",
             "-DTVQ_TEST_HOOKS", f"-I{HERE}"]
    if asan:
        flags += ["-fsanitize=address", "-fno-omit-frame-pointer"]
    if race:
        flags += ["-DEMU_RACE"]
    objs = []
    runtime = [HERE / "emu_runtime.cpp"] + ([HERE / "racecheck.cpp"] if race else [])
    srcs = sorted((stage / "tiny-vllm_amd" / "csrc").glob("*.cpp")) + runtime

    def cc(s: Path) -> Path:
        o = stage / (s.stem + ".o")
        extra = ["-fsanitize=thread"] if race and s not in runtime else []
        proc = subprocess.run([CLANG, *flags, *extra, "-c", str(s), "-o", str(o)], capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"emu build failed for {s.name}:\n{proc.stderr[-6000:]}")
        return o

    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(cc, srcs))
    lib = BUILD / (f"libtvq_emu{'_' + name if name else ''}{_suffix(asan, race)}.so")
    san = ["-fsanitize=address", "-shared-libasan"] if asan else []
    link = [CLANG, "-shared", *san, "-o", str(lib), *map(str, objs)]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"emu link failed:\n{proc.stderr[-4000:]}")
    return lib


def asan_runtime() -> str:
    return subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                          text=True, check=True).stdout.strip()



if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asan", action="store_true")
    ap.add_argument("--race", action="store_true")
    ap.add_argument("--csrc", type=Path, default=CSRC, help="kernel source folder (default: the package's)")
    ap.add_argument("--include", type=Path, default=INCLUDE)
    ap.add_argument("--name", default="", help="library name suffix")
    a = ap.parse_args()
    print(build(a.asan, csrc=a.csrc, include=a.include, name=a.name, race=a.race))
    sys.exit(0)
