"""Runs one engine step on the GPU (reference: nanovllm/engine/model_runner.py).

Owns the model, the KV cache and the sampler:
  * the model is built on cuda:0 in bf16. Weights come from `config.model`'s
    safetensors (or `quantized_model_path` for an "int8" / "w8a8" artifact)
    when present; otherwise every parameter is drawn at random
    (projections ~N(0, 0.02), norms 1) from a seeded generator in a fixed
    order, so a bf16 and a quantized engine built with the same seed hold the
    same weights up to quantization (the quantized layers store
    quantize_int8_per_channel of the bf16 draw);
  * KV cache: one tensor [2, layers, slots, kv_heads, max_model_len, head_dim]
    whose per-layer views go to each Attention; one slot per running sequence;
  * sampling: argmax where temperature == 0, otherwise the reference's
    exponential-race sampler (softmax(logits / T) / Exp(1), argmax);
  * decode steps replay HIP graphs captured per batch-size bucket
    (1, 2, 4, 8, 16, 32, ... up to min(slots, 512); reference
    model_runner.py:214-230, 297-335) unless `enforce_eager`. The running
    batch is padded to its bucket with slot -1 / length 0 rows, which the
    decode-attention kernel leaves inert.
"""
from __future__ import annotations

import itertools
import os
from glob import glob

import numpy as np
import torch
from torch import nn

from nanovllm.config import Config
from nanovllm.engine.sequence import Sequence
from nanovllm.layers.linear import LinearBase
from nanovllm.models.qwen3 import Attention, Qwen3ForCausalLM, RMSNorm
from nanovllm.quantization import _hip
from nanovllm.quantization.utils import quantize_int8_per_channel
from nanovllm.utils.context import step_context
from nanovllm.utils.loader import load_model


def sample(logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
    """Greedy rows (T == 0) take argmax; the rest follow reference sampler.py:10-15."""
    greedy = logits.argmax(dim=-1)
    if bool((temperatures > 0).any()):
        t = torch.where(temperatures > 0, temperatures, torch.ones_like(temperatures))
        probs = torch.softmax(logits.float() / t[:, None], dim=-1)
        drawn = probs.div_(torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)).argmax(dim=-1)
        return torch.where(temperatures > 0, drawn, greedy)
    return greedy


@torch.no_grad()
def random_init_(model: nn.Module, seed: int, std: float = 0.02, device: str = "cuda") -> None:
    """Seeded random weights in module order; quantized linears store the
    per-channel int8 quantization of the same bf16 draw."""
    gen = torch.Generator(device=device).manual_seed(seed)
    for mod in model.modules():
        if isinstance(mod, LinearBase):
            n, k = (mod.weight if mod.quant_method is None else mod.qweight).shape
            w = torch.empty(n, k, device=device, dtype=torch.bfloat16).normal_(0.0, std, generator=gen)
            if mod.quant_method is None:
                mod.weight.copy_(w)
            else:
                q, s = quantize_int8_per_channel(w)
                mod.qweight.copy_(q)
                getattr(mod, "scales", getattr(mod, "w_scales", None)).copy_(s)
            if mod.bias is not None:
                mod.bias.zero_()
        elif isinstance(mod, RMSNorm):
            mod.weight.fill_(1.0)
        elif isinstance(mod, nn.Embedding):
            mod.weight.normal_(0.0, std, generator=gen)
        elif isinstance(mod, nn.Linear) and mod.weight is not getattr(model, "model").embed_tokens.weight:
            mod.weight.normal_(0.0, std, generator=gen)


class ModelRunner:
    def __init__(self, config: Config, device: str = "cuda"):
        # device="cpu" exists for host-only tests of the engine logic; the
        # quantized layers then take the reference's torch path.
        if device == "cuda":
            if not torch.cuda.is_available():
                raise RuntimeError("the engine needs a GPU (cuda:0)")
            torch.cuda.set_device(0)
        self.config = config
        self.device = device
        hf = config.hf_config
        default_dtype = torch.get_default_dtype()
        torch.set_default_dtype(torch.bfloat16)
        with torch.device(device):
            self.model = Qwen3ForCausalLM(hf, config.quantization)
        torch.set_default_dtype(default_dtype)
        has_weights = isinstance(config.model, str) and glob(os.path.join(config.model, "*.safetensors"))
        if config.quantization and config.quantized_model_path:
            load_model(self.model, config.quantized_model_path, config.quantization)
        elif has_weights and not config.quantization:
            load_model(self.model, config.model)
        else:
            random_init_(self.model, config.seed, device=device)
        self.model.eval()
        if device == "cuda":
            # the split-K GEMM workspace and the attention kernels' counters
            # must exist before any graph capture
            from nanovllm.quantization import _hip
            _hip.gemm_workspace(torch.device("cuda", 0))
            _hip.attn_counters(torch.device("cuda", 0))
            self._warmup_model()
        self._allocate_kv_cache()
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        if device == "cuda" and not config.enforce_eager:
            self.capture_graphs()

    @torch.no_grad()
    def _warmup_model(self) -> None:
        """One cache-free prefill of the largest batch the scheduler can form
        (max_num_batched_tokens tokens in sequences of max_model_len), so the
        KV cache is sized after the peak activation memory is known and after
        the lazily built per-layer buffers (the regrouped gate_up weights of
        the fused W8A8 MLP) exist. Mirrors warmup_model + the peak accounting
        of the reference (model_runner.py:114-133)."""
        cfg = self.config
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        seq_len = min(cfg.max_model_len, cfg.max_num_batched_tokens)
        num = max(1, min(cfg.max_num_batched_tokens // seq_len, cfg.max_num_seqs))
        total = num * seq_len
        with step_context(True, cu_seqlens_q=torch.arange(0, total + 1, seq_len), max_seqlen_q=seq_len,
                          attn_blocks=_hip.prefill_blocks([(i * seq_len, seq_len) for i in range(num)]).cuda()):
            ids = torch.zeros(total, dtype=torch.int64, device="cuda")
            pos = torch.arange(seq_len, device="cuda").repeat(num)
            hidden = self.model(ids, pos)
            self.model.compute_logits(hidden[seq_len - 1::seq_len])
            torch.cuda.synchronize()
        self.warmup_peak_bytes = torch.cuda.max_memory_allocated()
        torch.cuda.empty_cache()

    def _allocate_kv_cache(self) -> None:
        cfg, hf = self.config, self.config.hf_config
        attns = [m for m in self.model.modules() if isinstance(m, Attention)]
        per_slot = 2 * len(attns) * attns[0].num_kv_heads * cfg.max_model_len * hf.head_dim * 2
        if self.device == "cuda":
            # the reference's accounting (model_runner.py:114-133): the share
            # of total memory left after the warmup's peak, minus what other
            # allocations outside torch already hold
            free, total = torch.cuda.mem_get_info()
            used = total - free
            current = torch.cuda.memory_stats()["allocated_bytes.all.current"]
            peak = max(self.warmup_peak_bytes, current)
            budget = int(total * cfg.gpu_memory_utilization - used - peak + current)
        else:
            budget = 1 << 30
        self.num_slots = min(cfg.max_num_seqs, budget // per_slot)
        if self.num_slots < 1:
            raise RuntimeError(f"not enough GPU memory for one KV slot of {cfg.max_model_len} tokens")
        # Zero-filled once: masked positions still enter p @ V with weight 0,
        # so the cache must never hold non-finite values.
        self.kv_cache = torch.zeros(2, len(attns), self.num_slots, attns[0].num_kv_heads, cfg.max_model_len,
                                    hf.head_dim, dtype=torch.bfloat16, device=self.device)
        for i, a in enumerate(attns):
            a.k_cache, a.v_cache = self.kv_cache[0, i], self.kv_cache[1, i]

    @torch.no_grad()
    def capture_graphs(self) -> None:
        hf = self.config.hf_config
        max_bs = min(self.num_slots, 512)
        self.graph_bs = [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 16))
        if self.graph_bs[-1] < max_bs:
            self.graph_bs.append(max_bs)
        dev = self.device
        gv = dict(input_ids=torch.zeros(max_bs, dtype=torch.int64, device=dev),
                  positions=torch.zeros(max_bs, dtype=torch.int64, device=dev),
                  slot_mapping=torch.full((max_bs,), -1, dtype=torch.int32, device=dev),
                  context_lens=torch.zeros(max_bs, dtype=torch.int32, device=dev),
                  outputs=torch.zeros(max_bs, hf.hidden_size, dtype=torch.bfloat16, device=dev))
        pool = None
        for bs in reversed(self.graph_bs):
            graph = torch.cuda.CUDAGraph()
            with step_context(False, slot_mapping=gv["slot_mapping"][:bs], context_lens=gv["context_lens"][:bs]):
                gv["outputs"][:bs] = self.model(gv["input_ids"][:bs], gv["positions"][:bs])  # warm-up
                with torch.cuda.graph(graph, pool):
                    gv["outputs"][:bs] = self.model(gv["input_ids"][:bs], gv["positions"][:bs])
            if pool is None:
                pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
        self.graph_vars = gv

    def _replay_decode(self, seqs: list[Sequence]) -> torch.Tensor:
        n = len(seqs)
        bs = next(b for b in self.graph_bs if b >= n)
        gv = self.graph_vars
        pad = bs - n
        ids = [s.last_token for s in seqs] + [0] * pad
        pos = [len(s) - 1 for s in seqs] + [0] * pad
        slots = [s.slot for s in seqs] + [-1] * pad
        lens = [len(s) for s in seqs] + [0] * pad
        gv["input_ids"][:bs].copy_(torch.tensor(ids, dtype=torch.int64, pin_memory=True), non_blocking=True)
        gv["positions"][:bs].copy_(torch.tensor(pos, dtype=torch.int64, pin_memory=True), non_blocking=True)
        gv["slot_mapping"][:bs].copy_(torch.tensor(slots, dtype=torch.int32, pin_memory=True), non_blocking=True)
        gv["context_lens"][:bs].copy_(torch.tensor(lens, dtype=torch.int32, pin_memory=True), non_blocking=True)
        self.graphs[bs].replay()
        return gv["outputs"][:n]

    def _to_gpu(self, values, dtype) -> torch.Tensor:
        if self.device == "cpu":
            return torch.tensor(values, dtype=dtype)
        return torch.tensor(values, dtype=dtype, pin_memory=True).cuda(non_blocking=True)

    @torch.no_grad()
    def run(self, seqs: list[Sequence], is_prefill: bool) -> list[int]:
        if is_prefill:
            hidden = self._prefill(seqs)
        elif self.graphs and len(seqs) <= self.graph_bs[-1]:
            with step_context(False):
                hidden = self._replay_decode(seqs)
        else:
            slots = [s.slot for s in seqs]
            lens = [len(s) for s in seqs]
            with step_context(False, max_seqlen_k=max(lens), slot_mapping=self._to_gpu(slots, torch.int32),
                              context_lens=self._to_gpu(lens, torch.int32), kv_lo=min(slots), kv_hi=max(slots) + 1):
                hidden = self.model(self._to_gpu([s.last_token for s in seqs], torch.int64),
                                    self._to_gpu([n - 1 for n in lens], torch.int64))
        logits = self.model.compute_logits(hidden)
        temps = self._to_gpu([s.temperature for s in seqs], torch.float32)
        return sample(logits, temps).tolist()

    def _prefill(self, seqs: list[Sequence]) -> torch.Tensor:
        """Forward of the packed prompts; returns each sequence's last hidden row.

        Per-token inputs are built with array ops: only the token ids cross
        from Python (one fromiter); positions and per-token slots expand from
        the per-sequence lengths on the device. The list loops they replace
        cost ~5 ms of host time per 16k tokens, during which the GPU had
        nothing queued."""
        lens = [len(s) for s in seqs]
        cu = [0, *itertools.accumulate(lens)]
        total = cu[-1]
        ids = torch.from_numpy(np.fromiter(itertools.chain.from_iterable(s.token_ids for s in seqs),
                                           dtype=np.int64, count=total))
        lens_t = self._to_gpu(lens, torch.int64)
        starts = self._to_gpu(cu[:-1], torch.int64)
        pos = torch.arange(total, device=lens_t.device) - torch.repeat_interleave(starts, lens_t, output_size=total)
        meta = dict(cu_seqlens_q=torch.tensor(cu), max_seqlen_q=max(lens))
        if self.device == "cuda":
            slots = self._to_gpu([s.slot for s in seqs], torch.int64)
            blocks = _hip.prefill_blocks([(cu[i], n) for i, n in enumerate(lens)])
            meta.update(slot_mapping=slots, attn_blocks=blocks.pin_memory().cuda(non_blocking=True),
                        token_slots=torch.repeat_interleave(slots, lens_t, output_size=total))
            ids = ids.pin_memory().cuda(non_blocking=True)
        else:
            meta.update(slot_mapping=torch.tensor([s.slot for s in seqs]))
        with step_context(True, **meta):
            hidden = self.model(ids, pos)
        return hidden[self._to_gpu(cu[1:], torch.int64) - 1]
