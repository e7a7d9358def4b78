"""Benchmark of the MI355X quantized-linear hot path.

Default run (N=1): prints ONE JSON line for BASELINE.json's headline config
(configs[1]): the W8A8 linear (per-token act-quant + int8 GEMM) at the
Qwen3-0.6B QKV shape N=4096, K=1024, M=256. A "step" is one such linear over
one batch of synthetic activations, using the next of a rotating pool of
distinct weight copies (> 512 MB in total, i.e. larger than the 256 MB
Infinity Cache, so weights come from HBM). Steps are captured in a HIP graph
and replayed (the C ABI never allocates or syncs), so the timed region is GPU
work, not Python launch overhead.

Cache discipline: before the timed replay, a 1 GiB device copy (read and
write, outside the timed region) evicts the 256 MB Infinity Cache and the L2s,
and the timed steps use weight copies the warm-up never touched, so every
timed step reads its weights from HBM at any --steps.

Extra keys on the same line:
  roofline      the dominant kernel (the W8A8 GEMM) timed with HIP events on
                its launch stream: algorithmic bytes / average launch time;
                operand_floor_us is the same tiles' operand stream alone
                (tvq_gemm_operand_floor), the floor its data movement sets
  cpu_baseline  the reference's torch path (quantize -> dequantize -> F.linear)
                restated in CPU torch, timed on this host's cores
  targets       the three north-star targets, from the sweep and the E2E leg
  e2e           config 5: random-init Qwen3-0.6B through LLM.generate, bf16 vs
                W8A16 vs W8A8 prefill / decode tok/s and TTFT (run first, in a
                child process, before this process touches the GPU)
  sweep         configs 1-4, one compact entry per (mode, shape, M):
                "cfg mode MxNxK path us frac [floorF us] [aqA us]" (full records:
                bench_sweep.jsonl in the output folder)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu] [--no-e2e]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "tiny-vllm_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

# Native failures must raise, never be served by the torch path.
os.environ["NANOVLLM_NATIVE_STRICT"] = "1"

import torch  # noqa: E402

METRIC = "int8 GEMM TOPS & HBM GB/s (% roofline) at decode/prefill M; decode tok/s"
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, GB/s
PEAK_I8_TOPS = 5000.0       # dense int8 MFMA, TOP/s
PEAK_BF16_TFLOPS = 2500.0   # dense bf16 MFMA, TFLOP/s
POOL_BYTES = 512 << 20      # rotating weight pool must exceed the 256 MB MALL

HEADLINE = dict(name="qkv_0.6b", n=4096, k=1024, m=256)


# ---------------------------------------------------------------- work formulas

def w8a16_bytes(m, n, k):
    return n * k + 4 * n + 2 * m * k + 2 * m * n


def w8a8_gemm_bytes(m, n, k):
    return n * k + 4 * n + m * k + 4 * m + 2 * m * n


def act_quant_bytes(m, k):
    return 3 * m * k + 4 * m


def gemm_ops(m, n, k):
    return 2 * m * n * k


def roofline_for(mode, m, n, k, seconds):
    ops = gemm_ops(m, n, k)
    nbytes = w8a8_gemm_bytes(m, n, k) if mode == "w8a8" else w8a16_bytes(m, n, k)
    peak_ops = PEAK_I8_TOPS if mode == "w8a8" else PEAK_BF16_TFLOPS
    t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
    t_mfma = ops / (peak_ops * 1e12)
    bound = "hbm" if t_hbm >= t_mfma else "mfma"
    gbs = nbytes / seconds / 1e9
    tops = ops / seconds / 1e12
    frac = (t_hbm if bound == "hbm" else t_mfma) / seconds
    return dict(bound=bound, gbs=gbs, tops=tops, frac=frac, bytes=nbytes, ops=ops)


# ---------------------------------------------------------------- inputs

_WCACHE: dict = {}


def _quantized_weights(n, k, seed):
    """W ~ N(0, 0.02) drawn from its own seeded generator (independent of the
    activations, so every mode and M of a shape shares it), quantized per
    output channel: scale = absmax / 127, round-half-even."""
    g = torch.Generator().manual_seed(seed + 1)
    w = torch.randn(n, k, generator=g) * 0.02
    s = (w.abs().amax(dim=1) / 127.0).clamp_min(1e-8)
    q = torch.round(w / s[:, None]).clamp_(-127, 127).to(torch.int8)
    return q, s


def make_inputs(mode, m, n, k, dev, seed=0, pool_bytes=POOL_BYTES, max_copies=256):
    """BASELINE.json's synthetic operands, generated on the host from one seeded
    CPU generator (so the GPU run and the CPU baseline see the same values):
    activations ~N(0,1) in bf16 (W8A8: 1% of the columns x20), weights
    W ~N(0, 0.02) quantized symmetric per output channel (scale = absmax/127,
    round-half-even), then moved to `dev` together with a pool of weight copies
    large enough to defeat the caches."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if mode == "w8a8":
        cols = torch.randperm(k, generator=g)[: max(1, k // 100)]
        x[:, cols] *= 20.0
    x = x.to(torch.bfloat16)
    if dev is not None and torch.device(dev).type != "cpu":
        x = x.to(dev)
        key = (n, k, seed, str(dev))
        if _WCACHE.get("key") != key:   # one shape's weights on the device at a time
            _WCACHE.clear()
            q, s = _quantized_weights(n, k, seed)
            _WCACHE.update(key=key, q=q.to(dev), s=s.to(dev))
        q, s = _WCACHE["q"], _WCACHE["s"]
    else:
        q, s = _quantized_weights(n, k, seed)
    wbytes = n * k + 4 * n
    copies = max(2, min(max_copies, math.ceil(pool_bytes / wbytes)))
    qs = [q] + [q.clone() for _ in range(copies - 1)]
    ss = [s] + [s.clone() for _ in range(copies - 1)]
    return x, qs, ss


# ---------------------------------------------------------------- timing

def _graph(fns):
    """Capture the callables (each launches on the current stream) in a HIP graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fns[: min(len(fns), 4)]:
            f()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for f in fns:
            f()
    torch.cuda.synchronize()
    return g


def time_graph(g, replays):
    """Seconds per replay, HIP events on the current stream (the replay stream)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / replays


class Launcher:
    """Pre-bound C-ABI launches with preallocated outputs (no allocation per call)."""

    def __init__(self, lib, dev):
        self.lib = lib
        self.dev = dev
        from nanovllm.quantization import _hip
        ws = _hip.gemm_workspace(dev)   # split-K workspace, as the Python layer passes it
        self.ws = (ws.data_ptr(), ws.numel())

    def stream(self):
        return torch.cuda.current_stream(self.dev).cuda_stream

    def act_quant(self, x, xq, a_s):
        m, k = x.shape
        return lambda: self._ck(self.lib.tvq_act_quant(x.data_ptr(), 1, m, k, 1e-8, xq.data_ptr(), a_s.data_ptr(),
                                                       self.stream()))

    def w8a8(self, xq, a_s, q, s, y):
        m, k = xq.shape
        n = q.shape[0]
        return lambda: self._ck(self.lib.tvq_w8a8_gemm(xq.data_ptr(), a_s.data_ptr(), q.data_ptr(), s.data_ptr(),
                                                       None, y.data_ptr(), 1, m, n, k, *self.ws, self.stream()))

    def w8a8_linear(self, x, q, s, y, xq, a_s):
        m, k = x.shape
        n = q.shape[0]
        return lambda: self._ck(self.lib.tvq_w8a8_linear(x.data_ptr(), 1, q.data_ptr(), s.data_ptr(), None,
                                                         y.data_ptr(), m, n, k, xq.data_ptr(), a_s.data_ptr(),
                                                         *self.ws, self.stream()))

    def w8a16(self, x, q, s, y):
        m, k = x.shape
        n = q.shape[0]
        return lambda: self._ck(self.lib.tvq_w8a16_gemm(x.data_ptr(), 1, q.data_ptr(), s.data_ptr(), None,
                                                        y.data_ptr(), m, n, k, *self.ws, self.stream()))

    def operand_floor(self, op, x, q):
        m, k = x.shape
        n = q.shape[0]
        return lambda: self._ck(self.lib.tvq_gemm_operand_floor(op, x.data_ptr(), q.data_ptr(), m, n, k,
                                                                self.stream()))

    def _ck(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.tvq_last_error().decode())


def time_kernel(make_fn, copies, min_launches=64, min_seconds=0.02):
    """Average seconds per launch of a graph cycling over `copies` launch closures."""
    fns = [make_fn(i) for i in range(copies)]
    reps = max(1, math.ceil(min_launches / len(fns)))
    fns = fns * reps
    g = _graph(fns)
    time_graph(g, 1)  # warm
    per = time_graph(g, 1)
    replays = max(1, math.ceil(min_seconds / max(per, 1e-9)))
    return time_graph(g, replays) / len(fns)


# ---------------------------------------------------------------- sweep (configs 1-4)

def sweep_cases():
    cases = []
    cases.append(("cfg1", "w8a16", 64, 6144, 1024))                            # W8A16 gate_up 0.6B
    for m in (1, 16, 64, 256, 512):                                            # cfg2 W8A8 QKV sweep
        cases.append(("cfg2", "w8a8", m, 4096, 1024))
    for name, n, k in (("down", 1024, 3072), ("o", 1024, 2048), ("gate_up", 6144, 1024)):  # cfg3 prefill
        for mode in ("w8a8", "w8a16"):
            cases.append((f"cfg3_{name}", mode, 8192, n, k))
    big = (("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096), ("down", 4096, 12288))
    for name, n, k in big:                                                    # cfg4 8B-like
        for m in (1, 64, 512, 4096, 16384):
            for mode in ("w8a16", "w8a8"):
                cases.append((f"cfg4_{name}", mode, m, n, k))
    return cases


def run_sweep(lib, dev, quick=False, tag="", floor=False):
    from nanovllm.quantization import _hip
    L = Launcher(lib, dev)
    out = []
    cases = sweep_cases()
    if quick:
        cases = [c for c in cases if c[0] in ("cfg1", "cfg2") or (c[0].startswith("cfg3") and c[1] == "w8a8")]
    # full records go to a file (the JSON line carries a compact form)
    (ROOT / "gpurun_out").mkdir(exist_ok=True)
    log = open(sweep_file(tag), "w")
    for ci, (cfg, mode, m, n, k) in enumerate(cases):
        if ci % 16 == 0:
            print(f"sweep case {ci}/{len(cases)}", file=sys.stderr, flush=True)
        x, qs, ss = make_inputs(mode, m, n, k, dev)
        copies = len(qs)
        if mode == "w8a8":
            xq, a_s = _hip.act_quant(x)
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            t = time_kernel(lambda i: L.w8a8(xq, a_s, qs[i], ss[i], y), copies)
            xq2 = torch.empty_like(xq)
            a_s2 = torch.empty_like(a_s)
            tq = time_kernel(lambda i: L.act_quant(x, xq2, a_s2), 1)
            path = _hip.select_path(_hip.OP_W8A8, m, n, k)
        else:
            y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
            t = time_kernel(lambda i: L.w8a16(x, qs[i], ss[i], y), copies)
            tq = None
            path = _hip.select_path(_hip.OP_W8A16, m, n, k)
        r = roofline_for(mode, m, n, k, t)
        rec = dict(cfg=cfg, mode=mode, M=m, N=n, K=k, path=path, us=round(t * 1e6, 3), gbs=round(r["gbs"], 1),
                   tops=round(r["tops"], 2), bound=r["bound"], frac=round(r["frac"], 4), weight_copies=copies)
        if floor and path.startswith("dma"):
            # operand-delivery floor of the same tiles (unsplit), same weight copies
            op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
            xa = xq if mode == "w8a8" else x
            try:
                tf = time_kernel(lambda i: L.operand_floor(op, xa, qs[i]), copies)
                rec["floor_us"] = round(tf * 1e6, 3)
            except RuntimeError as exc:
                print(f"operand floor not measured for {cfg} {mode} {m}x{n}x{k}: {exc}", file=sys.stderr)
        if tq is not None:
            rec["act_quant_us"] = round(tq * 1e6, 3)
            rec["act_quant_gbs"] = round(act_quant_bytes(m, k) / tq / 1e9, 1)
        out.append(rec)
        log.write(json.dumps(rec) + "\n")
        log.flush()
        del x, qs, ss, y
        torch.cuda.empty_cache()
    log.close()
    return out


# ---------------------------------------------------------------- CPU baseline

def cpu_baseline(budget_s=12.0):
    """The reference's torch path for the headline step on the host CPU:
    quantize_int8_per_row_dynamic -> w8a8_linear_fallback (dequantize both
    operands to bf16, F.linear), restated in oracle/ (utils.py:28-32,
    cuda.py:455-465)."""
    import oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    m, n, k = HEADLINE["m"], HEADLINE["n"], HEADLINE["k"]
    x, qs, ss = make_inputs("w8a8", m, n, k, "cpu", pool_bytes=0)   # the GPU headline's own operands
    q, s = qs[0], ss[0]

    def step():
        xq, a_s = oracle.quantize_rows_torch(x)
        return oracle.w8a8_torch_path(xq, a_s, q, s, None, torch.bfloat16)

    for _ in range(2):
        step()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    nbytes = w8a8_gemm_bytes(m, n, k) + act_quant_bytes(m, k)
    return dict(value=round(nbytes / med / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                ms_per_step=round(med * 1e3, 3),
                sample=f"{len(times)} steps of the headline W8A8 linear (M={m}, N={n}, K={k}, the GPU run's seeded "
                       f"inputs), "
                       f"median, torch CPU {torch.__version__} with {threads} threads, ~{budget_s:.0f}s budget")


# ---------------------------------------------------------------- profiling one GEMM

def run_profile_case(spec):
    from nanovllm.quantization import _hip
    mode, m, n, k = spec.split(",")
    m, n, k = int(m), int(n), int(k)
    if mode not in ("w8a8", "w8a16"):
        raise SystemExit(f"--profile-case: mode must be w8a8 or w8a16, got {mode}")
    lib = _hip.load_library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = Launcher(lib, dev)
    x, qs, ss = make_inputs(mode, m, n, k, dev)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    if mode == "w8a8":
        xq, a_s = _hip.act_quant(x)
        fns = [L.w8a8(xq, a_s, qs[i % len(qs)], ss[i % len(qs)], y) for i in range(64)]
    else:
        fns = [L.w8a16(x, qs[i % len(qs)], ss[i % len(qs)], y) for i in range(64)]
    g = _graph(fns)
    for _ in range(8):
        g.replay()
    torch.cuda.synchronize()
    op = _hip.OP_W8A8 if mode == "w8a8" else _hip.OP_W8A16
    print(json.dumps(dict(profile_case=spec, path=_hip.select_path(op, m, n, k), launches=8 * 64,
                          weight_copies=len(qs))), flush=True)


# ---------------------------------------------------------------- config 5 (end to end)

def _child(cmd, timeout_s):
    """Run `cmd` as a child process (stdout and stderr to this stderr); returns
    None on success, else a short error string. Never raises."""
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "tiny-vllm_amd"),
                                                       os.environ.get("PYTHONPATH", "")]))
    try:
        proc = subprocess.run(cmd, env=env, stdout=sys.stderr, stderr=sys.stderr, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        return f"timed out after {timeout_s} s"
    except OSError as exc:
        return f"could not start: {exc}"
    if proc.returncode != 0:
        return f"exit code {proc.returncode}"
    return None


def run_e2e(timeout_s=300):
    """Config 5 through the engine (nanovllm.bench_e2e) in a child process:
    256 sequences, inputs and outputs uniform 100-1024, greedy, bf16 vs W8A16
    vs W8A8 on a random-init Qwen3-0.6B. Its report comes back through a JSON
    file. A failed or timed-out leg is recorded as {"error": ...}; it never
    costs the headline."""
    out = ROOT / "gpurun_out" / "bench_e2e.json"
    out.parent.mkdir(exist_ok=True)
    if out.exists():
        out.unlink()
    t0 = time.perf_counter()
    err = _child([sys.executable, "-m", "nanovllm.bench_e2e", "--modes", "bf16,int8,w8a8", "--output", str(out)],
                 timeout_s)
    if err is None and not out.is_file():
        err = "no report written"
    if err is not None:
        return dict(error=f"e2e leg failed: {err}", leg_seconds=round(time.perf_counter() - t0, 1))
    rep = json.loads(out.read_text())
    res = {}
    for r in rep["results"]:
        res[r["mode"]] = dict(prefill_tok_s=round(r["prefill_tokens_per_second"]),
                              decode_tok_s=round(r["decode_tokens_per_second"]),
                              total_tok_s=round(r["throughput_tokens_per_second"]),
                              ttft_s=round(r["ttft_seconds_approx"] or 0.0, 4), wall_s=round(r["wall_time_seconds"], 2),
                              tokens=r["total_tokens"])
    base = res.get("bf16")
    if base:
        for mode, r in res.items():
            if mode != "bf16":
                r["prefill_vs_bf16"] = round(r["prefill_tok_s"] / base["prefill_tok_s"], 3)
                r["decode_vs_bf16"] = round(r["decode_tok_s"] / base["decode_tok_s"], 3)
    res["workload"] = ("random-init Qwen3-0.6B (28 layers), 256 seqs, input/output lengths uniform 100-1024, "
                       "greedy, max_num_batched_tokens 16384, HIP-graph decode")
    res["leg_seconds"] = round(time.perf_counter() - t0, 1)
    return res


def sweep_file(tag):
    return ROOT / "gpurun_out" / (f"bench_sweep_{tag}.jsonl" if tag else "bench_sweep.jsonl")


def run_sweep_child(quick, tag, floor, timeout_s=240):
    """Configs 1-4 in a child process (`bench.py --sweep-only`), so that a
    failure there is recorded instead of losing the headline. Returns
    (records, error): the records the child completed, and None or an error."""
    path = sweep_file(tag)
    path.parent.mkdir(exist_ok=True)
    if path.exists():
        path.unlink()
    cmd = [sys.executable, str(ROOT / "bench.py"), "--sweep-only"] + (["--quick"] if quick else []) \
        + (["--tag", tag] if tag else []) + (["--floor"] if floor else [])
    err = _child(cmd, timeout_s)
    recs = []
    if path.is_file():
        recs = [json.loads(line) for line in path.read_text().splitlines() if line.strip()]
    return recs, (None if err is None else f"sweep leg failed after {len(recs)} cases: {err}")


def targets_from(sweep, e2e):
    """The north-star targets: W8A16 decode >= 0.70 of HBM at M <= 64, W8A8
    prefill >= 0.50 of int8 peak at M = 8192, E2E W8A8 prefill > bf16."""
    t = {}
    if sweep:
        dec = [r for r in sweep if r["mode"] == "w8a16" and r["M"] <= 64]
        if dec:
            t["w8a16_decode_hbm_frac_m_le_64"] = dict(min=min(r["frac"] for r in dec), max=max(r["frac"] for r in dec),
                                                      target=0.70)
        pre = [r for r in sweep if r["mode"] == "w8a8" and r["M"] == 8192]
        if pre:
            t["w8a8_prefill_i8_frac_m8192"] = dict(min=min(r["frac"] for r in pre), max=max(r["frac"] for r in pre),
                                                   target=0.50)
    if e2e and "w8a8" in e2e and "prefill_vs_bf16" in e2e["w8a8"]:
        t["e2e_w8a8_prefill_vs_bf16"] = dict(value=e2e["w8a8"]["prefill_vs_bf16"], target=">1")
    return t


def compact(sweep):
    return [f'{r["cfg"]} {r["mode"]} {r["M"]}x{r["N"]}x{r["K"]} {r["path"]} {r["us"]}us {r["frac"]}'
            + (f' floor{r["floor_us"]}us' if "floor_us" in r else "")
            + (f' aq{r["act_quant_us"]}us' if "act_quant_us" in r else "") for r in sweep]


# ---------------------------------------------------------------- main

KERNEL_SOURCES = ("tiny-vllm_amd/csrc/gemm_dma_kernel.h", "tiny-vllm_amd/csrc/gemm_dma.hip",
                  "tiny-vllm_amd/csrc/tvq_common.h")


def kernel_source_sha():
    """sha256 (first 16 hex digits) over the W8A8 DMA GEMM's sources: a traffic
    record measured on other kernel code does not attach to this one."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--quick", action="store_true", help="only configs 1-2 and W8A8 prefill in the sweep")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 engine leg")
    ap.add_argument("--tag", default="", help="suffix of the sweep record file (bench_sweep_TAG.jsonl in the output "
                                              "folder), for runs under other kernel switches")
    ap.add_argument("--floor", action="store_true",
                    help="also time the DMA tiles' operand stream alone (tvq_gemm_operand_floor) at the headline "
                         "and for every DMA sweep entry")
    ap.add_argument("--e2e-timeout", type=int, default=300, help="seconds allowed to the config-5 leg")
    ap.add_argument("--sweep-timeout", type=int, default=240,
                    help="seconds allowed to the configs 1-4 sweep (the records it completed are kept)")
    ap.add_argument("--sweep-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--profile", action="store_true",
                    help="profiling run for rocprofv3: headline kernels only, plus one 256 MiB copy kernel "
                         "that calibrates the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--profile-case", default=None, metavar="MODE,M,N,K",
                    help="profiling run of one GEMM (mode w8a8 or w8a16) for rocprofv3: 8 graph replays of 64 "
                         "launches over the rotating weight copies; prints nothing but the path")
    args = ap.parse_args()
    if args.profile_case:
        run_profile_case(args.profile_case)
        return
    if args.profile:
        args.no_sweep = args.no_cpu = args.no_e2e = True
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the quantized linear is a per-GPU kernel; sharding is a design note). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.sweep_only:   # child of the sweep leg: records go to the sweep file, nothing to stdout
        from nanovllm.quantization import _hip
        lib = _hip.load_library()
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        run_sweep(lib, dev, quick=args.quick, tag=args.tag, floor=args.floor)
        return

    # The auxiliary legs run first, each in a child process, before this
    # process touches the GPU; a failure in either is recorded in the line.
    e2e = None if args.no_e2e else run_e2e(args.e2e_timeout)
    sweep, sweep_err = (None, None) if args.no_sweep else run_sweep_child(args.quick, args.tag, args.floor,
                                                                          args.sweep_timeout)

    from nanovllm.quantization import _hip
    lib = _hip.load_library()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = Launcher(lib, dev)

    if args.profile:
        # Calibration: a plain device copy of exactly 256 MiB in, 256 MiB out.
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    m, n, k = HEADLINE["m"], HEADLINE["n"], HEADLINE["k"]
    x, qs, ss = make_inputs("w8a8", m, n, k, dev)
    copies = len(qs)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
    xq = torch.empty(m, k, dtype=torch.int8, device=dev)
    a_s = torch.empty(m, dtype=torch.float32, device=dev)

    # Headline: exactly `steps` W8A8 linears, graph-replayed, weights rotating.
    # Warm-up steps use the copies at the end of the pool, timed steps start at
    # copy 0, and a 1 GiB copy between them evicts every cache level.
    g_warm = _graph([L.w8a8_linear(x, qs[copies - 1 - i % copies], ss[copies - 1 - i % copies], y, xq, a_s)
                     for i in range(args.warmup)])
    g_step = _graph([L.w8a8_linear(x, qs[i % copies], ss[i % copies], y, xq, a_s) for i in range(args.steps)])
    flush_src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
    flush_dst = torch.empty_like(flush_src)
    g_warm.replay()
    flush_dst.copy_(flush_src)
    torch.cuda.synchronize()
    del flush_src, flush_dst
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    g_step.replay()
    end.record()
    torch.cuda.synchronize()
    t_step = start.elapsed_time(end) / 1e3 / args.steps
    step_bytes = w8a8_gemm_bytes(m, n, k) + act_quant_bytes(m, k)
    value = step_bytes / t_step / 1e9

    # Dominant kernel (the GEMM) on its own, same stream, HIP events.
    xq0, a_s0 = _hip.act_quant(x)
    t_gemm = time_kernel(lambda i: L.w8a8(xq0, a_s0, qs[i], ss[i], y), copies, min_launches=256)
    r = roofline_for("w8a8", m, n, k, t_gemm)
    kernel = _hip.select_path(_hip.OP_W8A8, m, n, k)
    traffic = None
    tfile = ROOT / "profiles" / "traffic_w8a8_gemm_qkv_m256.json"
    if tfile.is_file():
        rec = json.loads(tfile.read_text())
        # only for the kernel it measured: same path, same kernel source
        if rec.get("kernel") == kernel and rec.get("kernel_source_sha") == kernel_source_sha():
            traffic = rec.get("hbm_bytes_per_launch")
    t_floor = None
    if args.floor:
        # The same tiles' operand stream alone (no MFMA, no output): the floor
        # that the GEMM's data movement sets, over the same rotating copies.
        try:
            t_floor = time_kernel(lambda i: L.operand_floor(_hip.OP_W8A8, xq0, qs[i]), copies, min_launches=256)
        except RuntimeError as exc:
            print(f"operand floor not measured: {exc}", file=sys.stderr)
    roof = dict(bound=r["bound"], achieved=round(r["gbs"], 1), peak=PEAK_HBM_GBS, unit="GB/s",
                frac=round(r["gbs"] / PEAK_HBM_GBS, 4), traffic=traffic,
                kernel=kernel, kernel_us=round(t_gemm * 1e6, 3),
                algorithmic_bytes=r["bytes"], tops=round(r["tops"], 3),
                operand_floor_us=None if t_floor is None else round(t_floor * 1e6, 3),
                floor_over_kernel=None if t_floor is None else round(t_floor / t_gemm, 4))
    del x, qs, ss
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline()
        except Exception as exc:  # reported baseline only: never costs the headline
            cpu = dict(error=f"cpu baseline failed: {type(exc).__name__}: {exc}")

    print(json.dumps(build_line(args, value, t_step, m, n, k, copies, roof, cpu, sweep, sweep_err, e2e)), flush=True)


def build_line(args, value, t_step, m, n, k, copies, roof, cpu, sweep, sweep_err, e2e):
    """The one JSON line (the driver's contract) from the measured pieces."""
    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations with 1% outlier columns x20; N(0,0.02) weights quantized "
                "per output channel to int8)",
        "config": {
            "workload": "W8A8 linear = per-token act-quant + int8 MFMA GEMM, Qwen3-0.6B qkv_proj "
                        f"N={n} K={k}, M={m} tokens (BASELINE configs[1]); {copies} rotating weight copies "
                        f"({copies * (n * k + 4 * n) / 2**20:.0f} MiB > MALL), HIP-graph replay",
            "M": m, "N": n, "K": k, "out_dtype": "bf16",
        },
        "roofline": roof,
        "cpu_baseline": cpu,
        "targets": targets_from(sweep, e2e),
        "e2e": e2e,
        "sweep": None if sweep is None else compact(sweep),
        "sweep_error": sweep_err,
    }


if __name__ == "__main__":
    main()
