"""Per-request sampling parameters (reference: nanovllm/sampling_params.py:1-12).

Same fields and defaults as the reference. One deliberate difference:
`temperature == 0` selects greedy (argmax) decoding, which the reference
rejects (its assertion temperature > 1e-10); the end-to-end quantization
benchmark compares bf16 / W8A16 / W8A8 under greedy decoding. Negative
temperatures still raise.
"""
from dataclasses import dataclass


@dataclass
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0 (0 = greedy), got {self.temperature}")
        if self.max_tokens < 1:
            raise ValueError(f"max_tokens must be >= 1, got {self.max_tokens}")
