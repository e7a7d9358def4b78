"""CPU checks on the gfx950 assembly of the DMA GEMM tiles (hipcc -S).

The kernel's stage waits are explicit (s_waitcnt vmcnt(N) per ring stage); a
wait the compiler adds on its own can silently empty the operand ring. These
tests compile configurations of gemm_dma_kernel.h to assembly and check:

* between a tile's first stage barrier and its first MFMA there is no
  vmcnt(0): the stages prefetched before the barrier stay in flight (the
  scale values parked for the epilogue once forced such a wait here);
* inside the MFMA loop there is no scratch (spill) traffic and no vmcnt wait
  other than the ring's own stage waits, which sit before an s_barrier.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "tiny-vllm_amd" / "csrc" / "gemm_dma_kernel.h"

# (label, template arguments of launch_dma after T: kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, kSplit, ...)
CONFIGS = [
    ("w8a8_64x64_headline", "true, false, 64, 64, 2, 2, 4, 16, 128, false"),
    ("w8a16_64x128w8", "false, false, 64, 128, 2, 4, 4, 16, 128, false"),
    ("w8a8_256x256w4", "true, false, 256, 256, 2, 2, 4, 32, 64, false"),
    ("w8a16_128x256w4", "false, false, 128, 256, 2, 2, 4, 32, 64, false"),
    ("w8a16_16x128_streamk", "false, false, 16, 128, 1, 4, 4, 16, 128, true, false, false, false, false, false, true"),
    ("w8a16_64x256_streamk", "false, false, 64, 256, 2, 4, 3, 16, 128, true, false, false, false, false, false, true"),
    ("w8a16_32x256_streamk", "false, false, 32, 256, 2, 4, 3, 16, 128, true, false, false, false, false, false, true"),
]


def _hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return path if Path(path).exists() else None


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("isa")
    src = d / "cfgs.hip"
    body = [f'#include "{HEADER}"', "namespace tvq {"]
    for i, (_, targs) in enumerate(CONFIGS):
        body.append(f"hipError_t cfg{i}(const void* x, const float* a, const int8_t* q, const float* s, void* y, "
                    f"int M, int N, int K, void* ws, hipStream_t st) {{ return dma::launch_dma<BF16, {targs}>"
                    f"(x, a, q, s, nullptr, y, M, N, K, 8, 1, 1, ws, 1 << 24, st); }}")
    body.append("}")
    src.write_text("\n".join(body) + "\n")
    out = d / "cfgs.s"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    text = out.read_text()
    funcs = {}
    lines = text.split("\n")
    starts = [i for i, l in enumerate(lines) if l.startswith("_ZN3tvq3dma15gemm_dma_kernel") and ": " in l]
    starts.append(len(lines))
    for a, b in zip(starts, starts[1:]):
        funcs[lines[a].split(":")[0]] = [l.strip() for l in lines[a:b]
                                          if l.strip() and not l.strip().startswith(";")]
    return funcs


def _kernel(funcs, targs):
    # mangled template arguments: bools as Lb0E/Lb1E, ints as Li<n>E
    parts = []
    for t in (x.strip() for x in targs.split(",")):
        parts.append("Lb1E" if t == "true" else "Lb0E" if t == "false" else f"Li{t}E")
    key = "INS_4BF16E" + "".join(parts)
    hits = [n for n in funcs if key in n]
    assert len(hits) == 1, (key, list(funcs)[:4])
    return funcs[hits[0]]


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_no_ring_drain_before_first_mfma(assembly, cfg):
    code = _kernel(assembly, cfg[1])
    first = next(i for i, l in enumerate(code) if l.startswith("v_mfma"))
    bar = max(i for i in range(first) if code[i].startswith("s_barrier"))
    waits = [l for l in code[bar:first] if re.match(r"s_waitcnt .*vmcnt\(0\)", l)]
    assert not waits, f"vmcnt(0) between the first stage barrier and the first MFMA: {waits}"


# The 4-wave W8A8 256x256 tile (opt-in) spills ~33 VGPRs outside its MFMA
# loop; the reloads are vector-memory ops waited with vmcnt(0) at tile start.
SPILLING = {"w8a8_256x256w4"}


@pytest.mark.parametrize("cfg", [pytest.param(c, marks=pytest.mark.xfail(strict=True, reason="VGPR spill reloads "
                                                                         "at tile start wait vmcnt(0)"))
                                 if c[0] in SPILLING else c for c in CONFIGS], ids=[c[0] for c in CONFIGS])
def test_every_vmem_wait_up_to_the_loop_end_is_a_barrier_wait(assembly, cfg):
    """From the kernel entry to the last MFMA (the block layout may put a
    tile-start block after the loop body), every vmcnt wait leads to an
    s_barrier within a few instructions: a stage wait, or the scale park
    after a tile's last stage. A wait that does not (the compiler's wait for
    a load consumed between barriers) drains the operand ring there."""
    code = _kernel(assembly, cfg[1])
    last = max(i for i, l in enumerate(code) if l.startswith("v_mfma"))
    for i in range(last):
        l = code[i]
        if l.startswith("s_waitcnt") and "vmcnt" in l:
            ahead = [x for x in code[i + 1:i + 40] if not x.startswith(".")][:16]   # instructions, not labels
            assert any(x.startswith("s_barrier") for x in ahead), f"line {i}: {l} -> {ahead}"


@pytest.mark.parametrize("cfg", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_mfma_loop_has_no_spills_or_extra_vmem_waits(assembly, cfg):
    code = _kernel(assembly, cfg[1])
    idx = [i for i, l in enumerate(code) if l.startswith("v_mfma")]
    span = code[idx[0]:idx[-1]]
    assert not [l for l in span if l.startswith("scratch_")], "scratch traffic inside the MFMA loop"
    # every vmcnt wait in the loop belongs to a stage crossing: an s_barrier follows
    # within the wait_stage branch chain (a few instructions)
    for i, l in enumerate(span):
        if "vmcnt" in l and l.startswith("s_waitcnt"):
            ahead = [x for x in span[i + 1:i + 40] if not x.startswith(".")][:16]
            assert any(x.startswith("s_barrier") for x in ahead), f"vmcnt wait not at a stage crossing: {l}"


@pytest.fixture(scope="module")
def skinny_assembly(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa_skinny") / "skinny.s"
    src = ROOT / "tiny-vllm_amd" / "csrc" / "gemm_skinny.hip"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = out.read_text().split("\n")
    starts = [i for i, l in enumerate(lines) if l.startswith("_ZN3tvq12_GLOBAL__N_113skinny_kernel") and ": " in l]
    starts.append(len(lines))
    return {lines[a].split(":")[0]: [l.strip() for l in lines[a:b] if l.strip() and not l.strip().startswith(";")]
            for a, b in zip(starts, starts[1:])}


def test_skinny_run_issues_all_loads_before_its_mfmas(skinny_assembly):
    """Decode M <= 16 (one 16-token block, one 16-row block, 8 chunks per run):
    the full run's 8 weight + 16 activation loads (W8A16) or 8 + 8 (W8A8) are
    in flight before the first MFMA waits on any of them."""
    checked = 0
    for name, code in skinny_assembly.items():
        m = re.search(r"skinny_kernelINS_\d(BF16|F16)ELb(\d)ELb0ELi1ELi1ELi(\d+)ELi8E", name)
        if not m:
            continue
        w8a8 = m.group(2) == "1"
        first = next(i for i, l in enumerate(code) if l.startswith("v_mfma"))
        loads = sum(1 for l in code[:first] if l.startswith("global_load_dwordx4"))
        assert loads >= (16 if w8a8 else 24), (name, loads)
        checked += 1
    assert checked >= 4


@pytest.fixture(scope="module")
def floor_assembly(tmp_path_factory):
    """gfx950 assembly of gemm_dma.hip, which instantiates the operand-floor
    kernels (kDmaOnly) for every DMA configuration."""
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa_floor") / "dma.s"
    src = ROOT / "tiny-vllm_amd" / "csrc" / "gemm_dma.hip"
    cmd = [hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = out.read_text().split("\n")
    starts = [i for i, l in enumerate(lines) if l.startswith("_ZN3tvq3dma15gemm_dma_kernel") and ": " in l]
    starts.append(len(lines))
    return {lines[a].split(":")[0]: [l.strip() for l in lines[a:b] if l.strip() and not l.strip().startswith(";")]
            for a, b in zip(starts, starts[1:])}


def test_operand_floor_kernels_touch_only_the_operands(floor_assembly):
    """The operand-floor kernels get null scale, bias and output pointers: their
    only vector-memory instructions must be the operand DMA into LDS
    (global_load_lds_*), with no other global, buffer, flat or scratch access."""
    checked = 0
    for name, code in floor_assembly.items():
        # non-type template arguments after T: kW8A8, kRaw, BM, BN, WM, WN, S, MF, KS, kSplit, kNtW, kGlu, kRot,
        # kDmaOnly (index 13), ...
        targs = re.findall(r"L[bi](\d+)E", name.split("gemm_dma_kernelI", 1)[1])
        if targs[13] != "1":
            continue
        vmem = [l.split()[0] for l in code if re.match(r"(global|buffer|flat|scratch)_", l)]
        bad = sorted({op for op in vmem if not op.startswith("global_load_lds_")})
        assert not bad, (name, bad)
        assert vmem, name
        checked += 1
    assert checked >= 13 * 2, checked   # every DmaCfg, unsplit and non-temporal-weight variants


@pytest.mark.parametrize("cfg", [pytest.param(c, marks=pytest.mark.xfail(strict=True, reason="the W8A8 4-wave tile "
                                                                         "spills VGPRs outside its MFMA loop"))
                                 if c[0] in SPILLING else c for c in CONFIGS], ids=[c[0] for c in CONFIGS])
def test_no_scratch_traffic_anywhere(assembly, cfg):
    """No spill code at all (the W8A16 4-wave tile once spilled 2 VGPRs by
    caching 16 scale vectors for its epilogue; it now reads them per use)."""
    code = _kernel(assembly, cfg[1])
    assert not [l for l in code if l.startswith("scratch_")], "scratch traffic"
