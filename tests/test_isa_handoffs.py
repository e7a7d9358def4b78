"""CPU checks on the gfx950 assembly of the cross-workgroup handoffs.

Two kinds of kernel pass data between workgroups inside one launch, through
global memory, where the workgroups may sit on different XCDs with separate
L2 caches:
  * the split-K / stream-K DMA GEMMs: each unit stores its accumulator image
    and the last arrival at the tile's counter reads every image back;
  * the attention kernels with o_proj's quantization fused: every workgroup
    stores its output slice, and the last arrival at the row block's counter
    reads the rows back and quantizes them.
Neither uses a release fence (an L2 write-back). Correctness instead rests on
the agent-scope accesses compiling to instructions with the device-scope
coherence bit, sc1: stores written through the XCD's L2, loads that miss past
it. These tests pin that in the compiled code, together with a single atomic
counter update per handoff and no flat (address-space unknown) accesses."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "tiny-vllm_amd" / "csrc"


def _assembly(tmp_path_factory, src: str) -> dict[str, list[str]]:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa_handoff") / (Path(src).stem + ".s")
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(CSRC / src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = out.read_text().split("\n")
    starts = [i for i, l in enumerate(lines) if re.match(r"^_ZN3tvq\w+:", l)]
    starts.append(len(lines))
    return {lines[a].split(":")[0]: [l.strip() for l in lines[a:b] if l.strip() and not l.strip().startswith(";")]
            for a, b in zip(starts, starts[1:])}


def _mem(code: list[str]) -> list[tuple[str, set[str]]]:
    ops = []
    for l in code:
        m = re.match(r"((?:global|flat|buffer)_\w+)\s*(.*)", l)
        if m:
            ops.append((m.group(1), set(m.group(2).replace(",", " ").split())))
    return ops


@pytest.fixture(scope="module")
def attention_asm(tmp_path_factory):
    return _assembly(tmp_path_factory, "attention.hip")


@pytest.fixture(scope="module")
def dma_asm(tmp_path_factory):
    return _assembly(tmp_path_factory, "gemm_dma.hip")


def test_attention_quant_handoff_is_device_coherent(attention_asm):
    quant = {n: c for n, c in attention_asm.items() if re.search(r"attn(32)?_kernelI\w+?Li\d+ELb1E", n)}
    plain = {n: c for n, c in attention_asm.items() if re.search(r"attn(32)?_kernelI\w+?Li\d+ELb0E", n)}
    assert len(quant) == 12 and len(plain) == 12, (len(quant), len(plain))
    for name, code in quant.items():
        ops = _mem(code)
        assert not [o for o, _ in ops if o.startswith("flat_")], name
        out_stores = [mods for o, mods in ops if o == "global_store_dwordx2"]
        readback = [mods for o, mods in ops if o == "global_load_dwordx2"]
        atomics = [o for o, _ in ops if "atomic" in o]
        assert out_stores and all("sc1" in m for m in out_stores), name     # output slices: written through L2
        assert readback and all("sc1" in m for m in readback), name         # rows read back past L2
        assert atomics and set(atomics) == {"global_atomic_add"}, (name, atomics)
        # the counter reset is the only other device-scope store
        resets = [m for o, m in ops if o == "global_store_dword" and "sc1" in m]
        assert len(resets) == len(atomics), name
    for name, code in plain.items():  # the plain variants are untouched: no device-scope traffic, no atomics
        ops = _mem(code)
        assert not [o for o, m in ops if "sc1" in m or "atomic" in o], name


def test_split_k_handoff_is_device_coherent(dma_asm):
    # non-type template arguments after T: kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, kSplit (index 9)
    split = {}
    for name, code in dma_asm.items():
        if "gemm_dma_kernel" not in name:
            continue
        targs = re.findall(r"L[bi](\d+)E", name.split("gemm_dma_kernelI", 1)[1])
        if targs[9] == "1":
            split[name] = code
    assert len(split) >= 10, len(split)
    for name, code in split.items():
        ops = _mem(code)
        assert not [o for o, _ in ops if o.startswith("flat_")], name
        image_stores = [m for o, m in ops if o.startswith("global_store_dword") and "sc1" in m]
        image_loads = [m for o, m in ops if o.startswith("global_load_dword") and not o.startswith("global_load_lds")
                       and "sc1" in m]
        atomics = [o for o, _ in ops if "atomic" in o]
        assert image_stores and image_loads, name
        assert set(atomics) <= {"global_atomic_add", "global_atomic_swap"} and "global_atomic_add" in atomics, \
            (name, atomics)
