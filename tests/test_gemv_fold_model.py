"""CPU model of the GEMV's cross-lane reduction (gemm_gemv.hip, fold_sum).

The kernel sums NV per-lane values over a wave's 64 lanes by halving: at
lane offsets 32, 16, ... a lane keeps the half of its values its lane bit
selects and adds the partner's copy of that half; the remaining offsets then
sum within each group. Emulated here with exact integers over 64 lanes, the
property that matters is checked for every NV the kernel uses (1..16) and
for 64: every lane of group j = lane / (64 / NV) ends with the sum over all
64 lanes of value j, and lane j of the final gather reads it.
"""
from __future__ import annotations

import numpy as np
import pytest


def fold_sum(c):
    """c: [64 lanes, NV] -> per-lane result, restating the kernel's steps."""
    c = c.copy()
    lanes = np.arange(64)
    nv = c.shape[1]
    off = 32
    n = nv
    while n > 1:
        hi = (lanes & off) != 0
        half = n // 2
        send = np.where(hi[:, None], c[:, :half], c[:, half:n])
        keep = np.where(hi[:, None], c[:, half:n], c[:, :half])
        c[:, :half] = keep + send[lanes ^ off]
        n, off = half, off // 2
    v = c[:, 0].copy()
    while off >= 1:
        v = v + v[lanes ^ off]
        off //= 2
    return v


@pytest.mark.parametrize("nv", [1, 2, 4, 8, 16, 64])
def test_every_group_holds_its_total(nv):
    rng = np.random.default_rng(nv)
    c = rng.integers(-2**20, 2**20, size=(64, nv)).astype(np.int64)
    v = fold_sum(c)
    group = 64 // nv
    totals = c.sum(axis=0)
    for lane in range(64):
        assert v[lane] == totals[lane // group], (nv, lane)
    # the gather: lane j < nv reads lane (j % nv) * group
    for j in range(nv):
        assert v[(j % nv) * group] == totals[j]
