"""CPU model of the stream-K work split of the DMA GEMM (gemm_dma_kernel.h).

The kernel and its launcher use closed forms for the work split: the range
length and grid (choose_streamk), a workgroup's segments (seg_coords), the
contributors of a tile (sk_w0, sk_parts) and the image each contributor writes
(own) and the last arrival reads (img_index). This test restates those
closed forms and checks them against a brute-force walk of the
same partition, over every decode shape the dispatcher can send to stream-K
and a sweep of small cases:

  * every (tile, k-stage) is computed by exactly one workgroup;
  * a tile's contributors, found by brute force, are exactly w0 .. w0+parts-1,
    in k order;
  * the image a contributor writes (own) is the image the last arrival reads
    for it (img_index), and no two contributions share an image;
  * images stay within the 2 * grid the launcher reserves in the workspace;
  * a tile with one contributor is a whole tile (it needs no fixup).
"""
from __future__ import annotations

import itertools

import pytest

KSPLIT_CNT_BYTES = 64 * 1024
KSPLIT_MAX_TILES = KSPLIT_CNT_BYTES // 4
MIN_STAGES = 8


def choose_streamk(tiles, nk, cus, tile_bytes, ws_bytes, min_stages=MIN_STAGES):
    """gemm_dma_kernel.h choose_streamk: (range length, grid) or (0, 0)."""
    if cus <= 0 or tiles <= 0 or nk <= 0 or tiles > KSPLIT_MAX_TILES:
        return 0, 0
    total = tiles * nk
    g = max(1, min(cus, total // min_stages))
    length = -(-total // g)
    g = -(-total // length)
    if KSPLIT_CNT_BYTES + 2 * g * tile_bytes > ws_bytes:
        return 0, 0
    return length, g


def kernel_segments(w, length, tiles, nk):
    """The segments workgroup w walks (seg_coords and the loop advance), with
    the image it writes for each (own = 2w + sk)."""
    pos = w * length
    end = min(tiles * nk, pos + length)
    sk = 0
    out = []
    while pos < end:
        tl = pos // nk
        kb = pos - tl * nk
        kn = min(nk - kb, end - pos)
        out.append((tl, kb, kn, 2 * w + sk))
        pos += kn
        sk = 1
    return out


def kernel_contributors(tl, length, nk):
    """sk_w0, sk_parts and img_index(s) of the fixup."""
    w0 = tl * nk // length
    parts = ((tl + 1) * nk - 1) // length - w0 + 1
    imgs = []
    for s in range(parts):
        w = w0 + s
        imgs.append(2 * w + (0 if w * length >= tl * nk else 1))
    return w0, parts, imgs


def check_partition(tiles, nk, length, grid):
    covered = {}
    by_tile = {}
    images = set()
    for w in range(grid):
        segs = kernel_segments(w, length, tiles, nk)
        assert segs, f"workgroup {w} has an empty range"
        assert {img for *_, img in segs} <= {2 * w, 2 * w + 1}, "a workgroup owns images 2w and 2w+1 only"
        for tl, kb, kn, img in segs:
            for k in range(kb, kb + kn):
                assert (tl, k) not in covered, f"stage {(tl, k)} computed twice"
                covered[(tl, k)] = w
            by_tile.setdefault(tl, []).append((kb, w, kn, img))
    assert len(covered) == tiles * nk, "some stage is never computed"
    for tl, contrib in by_tile.items():
        contrib.sort()
        w0, parts, imgs = kernel_contributors(tl, length, nk)
        assert [w for _, w, _, _ in contrib] == list(range(w0, w0 + parts)), (tl, contrib, w0, parts)
        assert sum(kn for _, _, kn, _ in contrib) == nk
        if parts == 1:
            assert contrib[0][0] == 0 and contrib[0][2] == nk, "single contributor must own the whole tile"
            continue
        # the image each contributor writes is the one the last arrival reads for it
        assert [img for *_, img in contrib] == imgs, (tl, contrib, imgs)
        for img in imgs:
            assert 0 <= img < 2 * grid
            assert img not in images, f"image {img} written twice"
            images.add(img)


# (M, N, K) decode shapes x the tiles the dispatcher uses for them with stream-K
DECODE_SHAPES = [(64, 24576, 4096), (64, 6144, 4096), (64, 4096, 4096), (64, 4096, 12288), (48, 6144, 4096),
                 (64, 6144, 1024), (64, 4096, 1024), (64, 3072, 1024), (64, 1024, 3072), (64, 1024, 2048),
                 (32, 24576, 4096), (24, 4096, 4096), (17, 1000, 2048), (33, 136, 2048), (20, 4096, 12288),
                 (16, 24576, 4096), (8, 4096, 12288), (3, 6144, 4096), (13, 1000, 2048)]
WS_BYTES = (32 << 20) + (64 << 10)   # tvq_gemm_workspace_bytes()


def streamk_tile(w8a8, m):
    """gemm_dma.hip choose() under TVQ_STREAMK=1."""
    if w8a8:
        return (64, 128) if m > 32 else (32, 64)
    return (64, 256) if m > 32 else (32, 256) if m > 16 else (16, 128)


@pytest.mark.parametrize("w8a8", [False, True])
@pytest.mark.parametrize("min_stages", [1, 2, 4, 8])
@pytest.mark.parametrize("shape", DECODE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_streamk_partition_decode_shapes(shape, min_stages, w8a8):
    m, n, k = shape
    bm, bn = streamk_tile(w8a8, m)
    tiles = -(-m // bm) * -(-n // bn)
    nk = k // 128
    length, grid = choose_streamk(tiles, nk, 256, bm * bn * 4, WS_BYTES, min_stages)
    assert length > 0, "the default workspace holds two images per workgroup"
    assert grid <= 256
    assert length >= min_stages or grid == 1
    check_partition(tiles, nk, length, grid)


@pytest.mark.parametrize("tiles,nk,cus", list(itertools.product([1, 2, 3, 5, 7, 12, 40, 97], [1, 2, 3, 8, 9, 17, 32, 96],
                                                                [1, 4, 7, 64, 256])))
def test_streamk_partition_sweep(tiles, nk, cus):
    length, grid = choose_streamk(tiles, nk, cus, 64 * 128 * 4, 1 << 40)
    assert length > 0
    check_partition(tiles, nk, length, grid)


def test_streamk_workspace_limit():
    """Without room for two images per workgroup the launch does not use
    stream-K; the default workspace is exactly full with the 64x256 W8A16
    tiles of the 8B gate_up at M = 64 (96 tiles x 32 stages on 256 CUs)."""
    tiles, nk, tb = 96, 32, 64 * 256 * 4
    length, grid = choose_streamk(tiles, nk, 256, tb, WS_BYTES)
    assert length == 12 and grid == 256
    assert KSPLIT_CNT_BYTES + 2 * grid * tb <= WS_BYTES
    assert choose_streamk(tiles, nk, 256, tb, WS_BYTES - 1) == (0, 0)
    assert choose_streamk(tiles, nk, 256, tb, 0) == (0, 0)
