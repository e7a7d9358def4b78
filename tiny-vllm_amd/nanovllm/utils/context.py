"""Metadata of the model step in flight.

Layers deep inside the model (attention, the quantized-linear path log) need
to know what kind of step is running and where its tokens live in the KV
cache, without threading that through every forward signature. The engine
opens a `step_context(...)` around each forward; layers read it with
`get_context()` (the one name the reference's quantized path imports,
nanovllm/quantization/cuda.py:9, 65-66). Outside any step the context is an
idle decode step with no metadata.

A step is either a prefill (packed prompts) or a decode (one new token per
running sequence); each kind carries only its own fields.
"""
from __future__ import annotations

from collections.abc import Iterator
from contextlib import contextmanager
from dataclasses import dataclass, fields

import torch


@dataclass(frozen=True)
class StepContext:
    is_prefill: bool = False
    # --- prefill: packed prompt batch
    cu_seqlens_q: torch.Tensor | None = None   # host int tensor [B+1], token offsets
    max_seqlen_q: int = 0
    attn_blocks: torch.Tensor | None = None    # device int32 [nblocks, 3], attention block table
    token_slots: torch.Tensor | None = None    # device int64 [T], KV slot of each packed token
    # --- both kinds: KV slot of each sequence
    slot_mapping: torch.Tensor | None = None
    # --- decode: one query token per sequence
    context_lens: torch.Tensor | None = None   # int32 [B], tokens incl. the new one
    max_seqlen_k: int = 0
    kv_lo: int = 0                             # slot range [kv_lo, kv_hi) of the batch (host path)
    kv_hi: int = 0


_PREFILL_ONLY = {"cu_seqlens_q", "max_seqlen_q", "attn_blocks", "token_slots"}
_DECODE_ONLY = {"context_lens", "max_seqlen_k", "kv_lo", "kv_hi"}
_FIELDS = {f.name for f in fields(StepContext)} - {"is_prefill"}

_IDLE = StepContext()
_stack: list[StepContext] = [_IDLE]


def get_context() -> StepContext:
    """The innermost open step (the idle context when none is open)."""
    return _stack[-1]


def make_context(is_prefill: bool, **metadata) -> StepContext:
    """Validated StepContext: unknown names and fields of the other step kind
    are rejected, so a prefill can never carry stale decode metadata."""
    unknown = set(metadata) - _FIELDS
    if unknown:
        raise TypeError(f"unknown step metadata: {sorted(unknown)}")
    wrong = set(metadata) & (_DECODE_ONLY if is_prefill else _PREFILL_ONLY)
    if wrong:
        kind = "prefill" if is_prefill else "decode"
        raise TypeError(f"{sorted(wrong)} do not belong to a {kind} step")
    return StepContext(is_prefill=is_prefill, **metadata)


@contextmanager
def step_context(is_prefill: bool, **metadata) -> Iterator[StepContext]:
    """Open a step for the duration of the block; nested steps restore the
    outer one on exit, exceptions included."""
    ctx = make_context(is_prefill, **metadata)
    _stack.append(ctx)
    try:
        yield ctx
    finally:
        _stack.pop()
