"""End-to-end generation benchmark: bf16 vs W8A16 ("int8") vs W8A8 on one GPU
(workload of the reference's bench.py:8-30 and bench_quant.py, here on a
randomly initialised Qwen3-0.6B-shaped model because no checkpoint is
available offline).

Workload (seeded with Python's `random`, as the reference bench): `num_seqs`
prompts of uniform-random token ids in [0, 10000], prompt length uniform in
[100, max_input_len], max_tokens uniform in [100, max_output_len],
ignore_eos, greedy decoding (temperature 0). Every mode sees the same
prompts and the same random weights (quantized per channel for int8/w8a8).

Reported per mode, as the reference's generate_with_stats: prefill and decode
tokens/s, TTFT (approximate), wall time, and total throughput = generated
tokens / wall time (reference bench.py:27-29).

    python -m nanovllm.bench_e2e [--modes bf16,int8,w8a8] [--num-seqs 256] ...
"""
from __future__ import annotations

import argparse
import gc
import json
import random
import sys
import time

import torch

from nanovllm import LLM, SamplingParams
from nanovllm.models.qwen3 import Qwen3Config


def make_workload(num_seqs: int, max_input_len: int, max_output_len: int, seed: int):
    # lengths uniform in [100, max], the reference benchmark's workload (the
    # lower bound shrinks with a smaller max, for short runs)
    rng = random.Random(seed)
    lo_in, lo_out = min(100, max_input_len), min(100, max_output_len)
    prompts = [[rng.randint(0, 10000) for _ in range(rng.randint(lo_in, max_input_len))] for _ in range(num_seqs)]
    params = [SamplingParams(temperature=0.0, ignore_eos=True, max_tokens=rng.randint(lo_out, max_output_len))
              for _ in range(num_seqs)]
    return prompts, params


def run_mode(mode: str, prompts, params, args) -> dict:
    quant = None if mode == "bf16" else mode
    t0 = time.perf_counter()
    llm = LLM(Qwen3Config(), quantization=quant, max_model_len=args.max_model_len,
              max_num_seqs=args.max_num_seqs, max_num_batched_tokens=args.max_num_batched_tokens,
              enforce_eager=args.enforce_eager, seed=args.seed)
    init_s = time.perf_counter() - t0
    llm.generate([[1, 2, 3, 4]], SamplingParams(temperature=0.0, max_tokens=4), use_tqdm=False)  # warm-up
    last = [time.perf_counter()]

    def progress(ev):
        now = time.perf_counter()
        if now - last[0] > 20:
            print(f"  [{mode}] t={ev['elapsed_seconds']:.0f}s", file=sys.stderr, flush=True)
            last[0] = now

    torch.cuda.synchronize()
    t = time.perf_counter()
    outs, st = llm.generate_with_stats(prompts, params, stats_hook=progress)
    wall = time.perf_counter() - t
    total = sum(len(o["token_ids"]) for o in outs)
    res = {"mode": mode, "init_seconds": round(init_s, 2), "total_tokens": total,
           "throughput_tokens_per_second": total / wall, **st}
    res["first_tokens"] = [o["token_ids"][:8] for o in outs[:2]]
    del llm
    gc.collect()
    torch.cuda.empty_cache()
    return res


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--modes", default="bf16,int8,w8a8")
    ap.add_argument("--num-seqs", type=int, default=256)
    ap.add_argument("--max-input-len", type=int, default=1024)
    ap.add_argument("--max-output-len", type=int, default=1024)
    ap.add_argument("--max-model-len", type=int, default=2048)
    ap.add_argument("--max-num-seqs", type=int, default=512)
    ap.add_argument("--max-num-batched-tokens", type=int, default=16384)
    ap.add_argument("--enforce-eager", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--output", default=None, help="write the JSON report here")
    args = ap.parse_args(argv)
    prompts, params = make_workload(args.num_seqs, args.max_input_len, args.max_output_len, args.seed)
    results = []
    for mode in args.modes.split(","):
        r = run_mode(mode, prompts, params, args)
        results.append(r)
        print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}), flush=True)
    base = next((r for r in results if r["mode"] == "bf16"), None)
    if base:
        for r in results:
            if r is not base:
                print(f"{r['mode']}/bf16: prefill x{r['prefill_tokens_per_second'] / base['prefill_tokens_per_second']:.3f}"
                      f"  decode x{r['decode_tokens_per_second'] / base['decode_tokens_per_second']:.3f}"
                      f"  total x{r['throughput_tokens_per_second'] / base['throughput_tokens_per_second']:.3f}")
    if args.output:
        with open(args.output, "w") as f:
            json.dump({"workload": vars(args), "results": results}, f, indent=1)


if __name__ == "__main__":
    main()
