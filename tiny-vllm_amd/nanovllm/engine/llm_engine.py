"""Engine loop (reference: nanovllm/engine/llm_engine.py).

`LLMEngine(model, **kwargs)` takes the same keyword arguments as the
reference's Config; `generate` / `generate_with_stats` return the same
outputs ({"text", "token_ids"} per prompt, in submission order) and the same
statistics, computed the same way (reference llm_engine.py:86-163): each
step is timed on the host around schedule + model step + postprocess; a step
that prefilled `n` prompt tokens adds `n` to the prefill totals, a decode
step over `b` sequences adds `b` decode tokens; TTFT is approximated by the
elapsed time before the first decode step.

Prompts may be token-id lists or, when the model directory holds a
tokenizer, strings.
"""
from __future__ import annotations

import os
from collections.abc import Callable
from dataclasses import fields
from time import perf_counter

from nanovllm.config import Config
from nanovllm.engine.model_runner import ModelRunner
from nanovllm.engine.scheduler import Scheduler
from nanovllm.engine.sequence import Sequence
from nanovllm.sampling_params import SamplingParams


def _load_tokenizer(model):
    if not isinstance(model, str) or not os.path.exists(os.path.join(model, "tokenizer_config.json")):
        return None
    from transformers import AutoTokenizer
    return AutoTokenizer.from_pretrained(model, use_fast=True)


class LLMEngine:
    def __init__(self, model, device: str = "cuda", **kwargs):
        names = {f.name for f in fields(Config)}
        config = Config(model, **{k: v for k, v in kwargs.items() if k in names})
        self.config = config
        self.tokenizer = _load_tokenizer(model)
        if self.tokenizer is not None and config.eos == -1:
            config.eos = self.tokenizer.eos_token_id
        self.model_runner = ModelRunner(config, device)
        self.scheduler = Scheduler(config.max_num_seqs, config.max_num_batched_tokens,
                                   self.model_runner.num_slots, config.eos)

    def exit(self) -> None:
        self.model_runner = None

    def add_request(self, prompt: str | list[int], sampling_params: SamplingParams) -> None:
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("string prompts need a tokenizer in the model directory; pass token ids")
            prompt = self.tokenizer.encode(prompt)
        if len(prompt) + sampling_params.max_tokens > self.config.max_model_len:
            raise ValueError(f"prompt ({len(prompt)}) + max_tokens ({sampling_params.max_tokens}) exceeds "
                             f"max_model_len ({self.config.max_model_len})")
        if len(prompt) > self.config.max_num_batched_tokens:
            raise ValueError("prompt longer than max_num_batched_tokens")
        self.scheduler.add(Sequence(prompt, sampling_params))

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        token_ids = self.model_runner.run(seqs, is_prefill)
        # no prefix caching here: a prefill step computes every prompt token
        num_tokens = sum(len(s) for s in seqs) if is_prefill else -len(seqs)
        self.scheduler.postprocess(seqs, token_ids)
        outputs = [(s.seq_id, s.completion_token_ids) for s in seqs if s.is_finished]
        return outputs, num_tokens

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def _run_generation(self, prompts, sampling_params, use_tqdm: bool,
                        stats_hook: Callable[[dict], None] | None = None):
        if not isinstance(sampling_params, list):
            sampling_params = [sampling_params] * len(prompts)
        for prompt, sp in zip(prompts, sampling_params):
            self.add_request(prompt, sp)
        pbar = None
        if use_tqdm:
            from tqdm.auto import tqdm
            pbar = tqdm(total=len(prompts), desc="Generating", dynamic_ncols=True)
        outputs: dict[int, list[int]] = {}
        pf_tok = dc_tok = pf_steps = dc_steps = 0
        pf_time = dc_time = 0.0
        pf_rate = dc_rate = 0.0
        ttft = None
        start = perf_counter()
        while not self.is_finished():
            t = perf_counter()
            out, n = self.step()
            dt = perf_counter() - t
            elapsed = perf_counter() - start
            if n > 0:
                pf_tok, pf_time, pf_steps, pf_rate = pf_tok + n, pf_time + dt, pf_steps + 1, n / dt
            else:
                dc_tok, dc_time, dc_steps, dc_rate = dc_tok - n, dc_time + dt, dc_steps + 1, -n / dt
                if ttft is None:
                    ttft = elapsed - dt
            if stats_hook is not None:
                stats_hook({"num_tokens": int(n), "step_time_seconds": dt, "elapsed_seconds": elapsed,
                            "is_prefill": n > 0})
            if pbar is not None:
                pbar.set_postfix({"Prefill": f"{int(pf_rate)}tok/s", "Decode": f"{int(dc_rate)}tok/s"})
            for seq_id, ids in out:
                outputs[seq_id] = ids
                if pbar is not None:
                    pbar.update(1)
        if pbar is not None:
            pbar.close()
        results = []
        for seq_id in sorted(outputs):
            ids = outputs[seq_id]
            text = self.tokenizer.decode(ids) if self.tokenizer is not None else ""
            results.append({"text": text, "token_ids": ids})
        stats = {
            "wall_time_seconds": perf_counter() - start,
            "prefill_tokens": int(pf_tok),
            "prefill_time_seconds": pf_time,
            "prefill_steps": int(pf_steps),
            "prefill_tokens_per_second": pf_tok / pf_time if pf_time > 0 else 0.0,
            "decode_tokens": int(dc_tok),
            "decode_time_seconds": dc_time,
            "decode_steps": int(dc_steps),
            "decode_tokens_per_second": dc_tok / dc_time if dc_time > 0 else 0.0,
            "ttft_seconds_approx": ttft,
        }
        return results, stats

    def generate(self, prompts, sampling_params, use_tqdm: bool = True) -> list[dict]:
        return self._run_generation(prompts, sampling_params, use_tqdm)[0]

    def generate_with_stats(self, prompts, sampling_params, use_tqdm: bool = False, stats_hook=None):
        return self._run_generation(prompts, sampling_params, use_tqdm, stats_hook)
