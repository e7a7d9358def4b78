"""CPU model of the DMA GEMM tiles' two index mappings (gemm_dma_kernel.h).

The kernel writes each stage into LDS with one mapping (set_sources / issue:
8 rows x 128 bytes per 1 KB DMA block, 16-byte chunks XOR-swizzled by row) and
reads MFMA fragments back with another (woff / xoff / load_frags / chunk_off).
Both are restated here from the kernel's formulas, and for every tile
configuration of the dispatch table this checks what neither formula shows on
its own:
* the DMA covers every (operand, row, 16-byte chunk) of a stage exactly once;
* every lane's fragment read returns exactly the operand bytes its MFMA lane
  needs: output channel / token row r of the fragment and the k range the
  lane group owns in that sub-step, with the weight and activation lanes of
  one MFMA agreeing on k;
* each 16-lane phase of a fragment read touches 16 different 16-byte bank
  groups of a 256-byte window (the conflict-free claim of the swizzle).
"""
from __future__ import annotations

import pytest

# (w8a8, BM, BN, WM, WN, MF, KS) -- the configurations of gemm_dma.hip's table
CONFIGS = [
    (True, 256, 256, 2, 4, 32, 128),
    (True, 256, 128, 4, 2, 32, 128),
    (True, 64, 64, 2, 2, 16, 128),
    (True, 64, 128, 2, 4, 16, 128),
    (True, 32, 64, 2, 2, 16, 128),
    (False, 128, 256, 2, 4, 32, 128),
    (False, 64, 128, 2, 2, 32, 128),
    (False, 64, 64, 2, 2, 32, 128),
    (False, 32, 64, 2, 2, 16, 128),
    (False, 64, 128, 2, 4, 16, 128),
    (True, 256, 256, 2, 2, 32, 64),     # 4-wave prefill tiles (TVQ_PREFILL_W4=1)
    (False, 128, 256, 2, 2, 32, 64),
    (False, 16, 128, 1, 4, 16, 128),    # W8A16 M <= 16 under stream-K (TVQ_STREAMK=1)
    (False, 64, 256, 2, 4, 16, 128),    # W8A16 32 < M <= 64 under stream-K
    (False, 32, 256, 2, 4, 16, 128),    # W8A16 16 < M <= 32 under stream-K
]


def swz(rb: int, row: int) -> int:
    return (row >> 1) & 7 if rb == 128 else (row >> 2) & 3


def chunk_off(rb: int, row: int, c: int) -> int:
    kr, kc = 1024 // rb, rb // 16
    return (row // kr) * 1024 + 16 * ((row % kr) * kc + (c ^ swz(rb, row)))


def stage_map(w8a8, bm, bn, ks):
    """LDS byte offset (16-byte granule) -> (operand, row, byte offset in the
    row's stage slice), from the DMA source formulas."""
    e = 1 if w8a8 else 2
    xrow = ks * e
    xrb = min(xrow, 128)
    xhalves = xrow // xrb
    wblk = bn * ks // 1024
    xblk = bm * xrow // 1024
    wch, xch = ks // 16, xrb // 16
    m = {}
    for b in range(wblk + xblk):
        for lane in range(64):
            if b < wblk:
                row = (1024 // ks) * b + lane // wch
                src = ("W", row, 16 * ((lane % wch) ^ swz(ks, row)))
            else:
                xb = b - wblk
                row = (1024 // xrb) * (xb // xhalves) + lane // xch
                src = ("X", row, xrb * (xb % xhalves) + 16 * ((lane % xch) ^ swz(xrb, row)))
            m[b * 1024 + 16 * lane] = src
    return m, wblk, xhalves


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"{'i8' if c[0] else 'f16x'}_{c[1]}x{c[2]}_w{c[3]}x{c[4]}_mf{c[5]}")
def test_dma_layout_and_fragment_reads_agree(cfg):
    w8a8, bm, bn, wm_n, wn_n, mf, ks = cfg
    e = 1 if w8a8 else 2
    lds, wblk, xhalves = stage_map(w8a8, bm, bn, ks)
    # the DMA is a bijection onto the stage's operand chunks
    want = {("W", r, 16 * c) for r in range(bn) for c in range(ks // 16)}
    want |= {("X", r, 16 * c) for r in range(bm) for c in range(ks * e // 16)}
    assert sorted(lds.values()) == sorted(want)

    tm, tn = bm // wm_n, bn // wn_n
    fm, fn = tm // mf, tn // mf
    ksub = ks // (32 if mf == 32 else 64)
    kstep = ks // ksub                      # k per sub-step
    wch = ks // 16
    wfrag, xfrag = mf * ks, mf * ks * e
    for wm in range(wm_n):
        for wn in range(wn_n):
            for ksi in range(ksub):
                reads = {}   # per fragment read instruction: list of 64 addresses
                for lane in range(64):
                    r, g = lane % mf, lane // mf
                    c = ksi * (wch // ksub) + g
                    woff = chunk_off(ks, r, c)
                    k0 = ksi * kstep + 16 * g            # this lane's 16 k values
                    for i in range(fn):
                        addr = wn * fn * wfrag + i * wfrag + woff
                        assert lds[addr] == ("W", (wn * fn + i) * mf + r, k0)
                        reads.setdefault(("W", i), []).append(addr)
                    for j in range(fm):
                        xbase = wblk * 1024 + wm * fm * xfrag + j * xfrag
                        row = (wm * fm + j) * mf + r
                        if w8a8:
                            addr = xbase + woff
                            assert lds[addr] == ("X", row, k0)
                            reads.setdefault(("X", j, 0), []).append(addr)
                        else:
                            for hb in range(2):
                                k = k0 + 8 * hb          # the 8 k values of half hb
                                xoff = ((r >> 3) * 1024 * xhalves + (k >> 6) * 1024
                                        + 16 * ((r & 7) * 8 + (((k & 63) >> 3) ^ swz(128, r))))
                                assert lds[xbase + xoff] == ("X", row, 2 * k)
                                reads.setdefault(("X", j, hb), []).append(xbase + xoff)
                for key, addrs in reads.items():
                    for phase in range(4):
                        groups = [(a % 256) // 16 for a in addrs[16 * phase:16 * phase + 16]]
                        assert len(set(groups)) == 16, (cfg, key, phase, groups)
