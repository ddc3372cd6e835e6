"""A CPU model of the balanced partition's straddling ranges as the kernels
walk them (csrc/decode_common.h work_range and segment_slot, the segment loop
of the partial kernels, the combine kernel's slot ranges), checked over
random batches: every tile of every sequence is covered by exactly one
segment, a worker's walk never runs past the batch, each segment's worker
lies in the range the combine computes for its sequence, and that range is
exactly the set of workers that wrote a segment of it (so the combine never
reads a slot no worker wrote). The GPU tests check the kernels' results;
this pins the arithmetic they share, including the charge of
kSegCostTiles positions per sequence start."""

import numpy as np
import pytest


def cdiv(a, b):
    return -(-a // b)


def walk(seqlens, workers, seg_cost):
    """Segments (worker, b, t_start, t_end) of the straddling form, or None
    when the batch takes the snapped form."""
    tiles = [cdiv(n, 64) if n > 0 else 0 for n in seqlens]
    total = sum(tiles)
    if total == 0:
        return None
    c = cdiv(total, workers)
    if sum(cdiv(t, c) for t in tiles) <= workers:
        return None
    line = [t + seg_cost if t > 0 else 0 for t in tiles]
    vtotal = sum(line)
    vc = cdiv(vtotal, workers)
    segments = []
    for w in range(workers):
        vlo = w * vc
        if vlo >= vtotal:
            continue
        voff, b = 0, 0
        while not vlo < voff + line[b]:  # the sequence holding position vlo
            voff += line[b]
            b += 1
        first = voff + seg_cost  # position of b's tile 0
        t_start = max(vlo - first, 0)
        remaining = min(vlo + vc, vtotal) - first - t_start
        while remaining > 0:  # the kernels' segment loop
            assert b < len(tiles), "walk ran past the batch"
            if tiles[b] == 0:
                b += 1
                continue
            t_end = min(tiles[b], t_start + remaining)
            assert t_end > t_start
            segments.append((w, b, t_start, t_end))
            remaining -= t_end - t_start + seg_cost
            b += 1
            t_start = 0
    return tiles, vc, line, segments


def combine_range(line, b, vc, seg_cost, nt):
    first = sum(line[:b]) + seg_cost
    return first // vc, (first + nt - 1) // vc


@pytest.mark.parametrize("seg_cost", [0, 1, 2, 3, 5])
def test_straddling_walk_covers_every_tile_once(seg_cost):
    rng = np.random.default_rng(seg_cost)
    checked = 0
    for _ in range(3000):
        batch = int(rng.integers(1, 70))
        pick = rng.integers(0, 8, size=batch)
        lens = [int(x) for x in np.where(pick < 2, 0, np.where(pick < 4, rng.integers(1, 130, size=batch),
                                                                rng.integers(0, 40000, size=batch)))]
        workers = int(rng.integers(1, 300))
        res = walk(lens, workers, seg_cost)
        if res is None:
            continue
        checked += 1
        tiles, vc, line, segments = res
        covered = [[] for _ in tiles]
        for w, b, t0, t1 in segments:
            covered[b].append((w, t0, t1))
        for b, nt in enumerate(tiles):
            got = sorted(t for _, t0, t1 in covered[b] for t in range(t0, t1))
            assert got == list(range(nt)), (lens, workers, b)
            if nt:
                g1, g2 = combine_range(line, b, vc, seg_cost, nt)
                assert [w for w, _, _ in covered[b]] == list(range(g1, g2 + 1)), (lens, workers, b)
    assert checked > 500


def test_host_restatement_agrees_with_the_walk():
    """triton_mla.kernel.balanced_pieces (the bench CSV's split count) is the
    largest number of workers of one sequence in the same walk."""
    from triton_mla.kernel import SEGMENT_START_TILES, balanced_pieces

    rng = np.random.default_rng(7)
    for _ in range(500):
        lens = [int(x) for x in rng.integers(0, 30000, size=int(rng.integers(1, 64)))]
        workers = int(rng.integers(1, 300))
        res = walk(lens, workers, SEGMENT_START_TILES)
        if res is None:
            continue
        tiles, _, _, segments = res
        per_seq = [len({w for w, b2, _, _ in segments if b2 == b}) for b in range(len(tiles))]
        assert balanced_pieces(lens, workers) == max(per_seq)
