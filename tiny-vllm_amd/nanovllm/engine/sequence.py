"""One generation request as the engine tracks it.

The prompt and the generated tokens are kept apart (the prompt never
changes; generation only appends), and the sampling parameters stay in
their SamplingParams object. While the request runs it owns one KV-cache
slot (`slot`, -1 otherwise). Requests get increasing ids in creation order,
which the engine uses to return outputs in submission order.

The attribute names the engine, scheduler and statistics read
(`token_ids`, `completion_token_ids`, `num_completion_tokens`, `last_token`,
`len(seq)`) follow the reference's Sequence (nanovllm/engine/sequence.py) so
the scheduling policy and token accounting read the same.
"""
from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from enum import Enum

from nanovllm.sampling_params import SamplingParams

_next_id = itertools.count()


class SequenceStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


@dataclass(eq=False)
class Sequence:
    prompt: list[int]
    params: SamplingParams = field(default_factory=SamplingParams)
    output: list[int] = field(default_factory=list)
    status: SequenceStatus = SequenceStatus.WAITING
    slot: int = -1
    seq_id: int = field(default_factory=lambda: next(_next_id))

    def __post_init__(self) -> None:
        self.prompt = list(self.prompt)
        if not self.prompt:
            raise ValueError("empty prompt")

    def __len__(self) -> int:
        return len(self.prompt) + len(self.output)

    # sampling parameters, read per step by the runner and scheduler
    temperature = property(lambda self: self.params.temperature)
    max_tokens = property(lambda self: self.params.max_tokens)
    ignore_eos = property(lambda self: self.params.ignore_eos)

    @property
    def token_ids(self) -> list[int]:
        return self.prompt + self.output

    @property
    def last_token(self) -> int:
        return self.output[-1] if self.output else self.prompt[-1]

    @property
    def num_prompt_tokens(self) -> int:
        return len(self.prompt)

    @property
    def num_completion_tokens(self) -> int:
        return len(self.output)

    @property
    def completion_token_ids(self) -> list[int]:
        return list(self.output)

    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    def append_token(self, token_id: int) -> None:
        self.output.append(token_id)
