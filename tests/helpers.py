"""Shared input generators and converters for the parity tests."""
from __future__ import annotations

import numpy as np
import torch

import oracle


def bits16(t: torch.Tensor) -> np.ndarray:
    """Raw 16-bit words of a bf16/fp16 tensor as uint16 numpy (CPU copy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().float().numpy()


def make_activations(m: int, k: int, seed: int, dtype=torch.bfloat16, outlier_frac: float = 0.01,
                     outlier_scale: float = 20.0) -> torch.Tensor:
    """X ~ N(0,1) with a seeded 1% of columns scaled x20 (the W8A8 config's outliers)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    n_out = int(round(outlier_frac * k))
    if n_out:
        cols = torch.randperm(k, generator=g)[:n_out]
        x[:, cols] *= outlier_scale
    return x.to(dtype)


def make_weights(n: int, k: int, seed: int, std: float = 0.02) -> tuple[torch.Tensor, torch.Tensor]:
    """W ~ N(0, std) in bf16, quantized per output channel by the oracle (utils.py:21-25)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * std).to(torch.bfloat16)
    q, s = oracle.quantize_rows(f32(w))
    return torch.from_numpy(q), torch.from_numpy(s)


def ragged_prefill_rows(total: int, n_seqs: int, lo: int, hi: int, seed: int) -> list[int]:
    """Sequence lengths uniform in [lo, hi], packed and padded up to `total` rows."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n_seqs)
    while lens.sum() > total:
        lens = rng.integers(lo, hi + 1, size=n_seqs)
    return [int(v) for v in lens]
