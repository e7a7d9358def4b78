"""Per-step forward context (reference: nanovllm/utils/context.py).

The quantized path reads only `is_prefill`, to label its one-shot path log;
the remaining fields carry the attention metadata of a model step.
"""
from dataclasses import dataclass

import torch


@dataclass
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    kv_lo: int = 0   # decode: KV-cache slot range of the running batch
    kv_hi: int = 0
    # prefill on the GPU: the attention kernel's 64-query block table and,
    # per packed token, its cache slot (for the KV-cache store)
    attn_blocks: torch.Tensor | None = None
    token_slots: torch.Tensor | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0, slot_mapping=None,
                context_lens=None, block_tables=None, kv_lo=0, kv_hi=0, attn_blocks=None, token_slots=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping,
                       context_lens, block_tables, kv_lo, kv_hi, attn_blocks, token_slots)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
