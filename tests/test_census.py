"""The work census behind the roofline's algorithmic bytes, recomputed by brute
force.

The oracle's trace (orc_fps_trace) reports, per iteration, the candidate
points and candidate 16-point leaves of the reference's rule: every bucket of
every cell inside the cube of the new sample (src/yuezu_fps.cpp:560-597), all
its points updated (:495-513), its points held in ceil(count / 16) blocks of
MORTON_BLOCK_SIZE (:277-283); iteration 0 is the first full pass (:418-438).
A bucket reached from several cube cells (grids whose block counts are not
powers of two share buckets, :592) is updated once per cell, so it is counted
once per cell.

Here the same counts come from NumPy alone: cells by the float32 cell rule,
buckets from the closed-form Morton tables modulo the bucket count, the cube
half-widths ceil(sqrtf(D) / block_size) in float32, and the clipped cube
enumerated cell by cell.  A double-counted cell, a dropped shared bucket, a
floor instead of a ceil in the leaf count or a missing first pass changes
them."""

import numpy as np
import pytest

from test_oracle import numpy_cells

LEAF = 16  # MORTON_BLOCK_SIZE, src/yuezu_fps.h:19


def morton_tables(blocks):
    """x, y, z tables of the reference's bit interleave (src/yuezu_fps.cpp:52-97):
    min(bits) rounds of x, y, z, then x, y, z where an axis still has bits."""
    bits = [max(1, int(np.ceil(np.log2(b)))) if b > 1 else 1 for b in blocks]
    pos = [[], [], []]
    nxt = 0
    for i in range(max(bits)):
        for a in range(3):
            if i < bits[a]:
                pos[a].append(nxt)
                nxt += 1
    tabs = []
    for a in range(3):
        v = np.arange(1 << bits[a], dtype=np.uint64)
        code = np.zeros_like(v)
        for k, p in enumerate(pos[a]):
            code |= ((v >> np.uint64(k)) & np.uint64(1)) << np.uint64(p)
        tabs.append(code)
    return tabs


def numpy_census(points, rng, idx, max_dist):
    blocks = [int(b) for b in rng[6:9]]
    T = blocks[0] * blocks[1] * blocks[2]
    xl, yl, zl = morton_tables(blocks)
    cells = numpy_cells(points, rng).astype(np.int64)
    bucket = ((xl[cells[:, 0]] | yl[cells[:, 1]] | zl[cells[:, 2]]) % np.uint64(T)).astype(np.int64)
    pop = np.bincount(bucket, minlength=T).astype(np.int64)
    leaves = (pop + LEAF - 1) // LEAF
    bs = [np.float32(np.float32(rng[2 * a + 1]) - np.float32(rng[2 * a])) / np.float32(blocks[a])
          for a in range(3)]
    cand_pts = np.zeros(len(idx), np.int64)
    cand_lv = np.zeros(len(idx), np.int64)
    cand_pts[0] = len(points)
    cand_lv[0] = leaves.sum()
    for it in range(1, len(idx)):
        q = points[idx[it]]
        r = np.sqrt(np.float32(max_dist[it]))
        qc = cells[idx[it]]
        ranges = []
        for a in range(3):
            h = int(np.ceil(np.float32(r / bs[a])))
            ranges.append(np.arange(max(0, qc[a] - h), min(blocks[a] - 1, qc[a] + h) + 1))
        gz, gy, gx = np.meshgrid(ranges[2], ranges[1], ranges[0], indexing="ij")
        b = ((xl[gx.ravel()] | yl[gy.ravel()] | zl[gz.ravel()]) % np.uint64(T)).astype(np.int64)
        cand_pts[it] = pop[b].sum()
        cand_lv[it] = leaves[b].sum()
        assert np.array_equal(cells[idx[it]], numpy_cells(q[None, :], rng)[0])
    return cand_pts, cand_lv


def cloud(seed, n):
    rs = np.random.RandomState(seed)
    p = np.concatenate([rs.randn(n // 2, 3) * 0.4, rs.uniform(-1, 1, (n - n // 2, 3))])
    p[: n // 100] = p[n // 100: 2 * (n // 100)]  # exact duplicates
    return p.astype(np.float32)


@pytest.mark.parametrize("blocks", [(32, 32, 32), (16, 8, 4), (10, 12, 6), (7, 1, 3)])
def test_census_trace_equals_numpy_brute_force(oracle, blocks):
    pts = cloud(31, 6000)
    rng = (-1.5, 1.5, -1.5, 1.5, -1.5, 1.5, *blocks)
    idx, md, cp, cl = oracle.fps_trace(pts, 700, rng, leaves=True)
    assert np.array_equal(idx, oracle.fps(pts, 700, rng))
    want_pts, want_lv = numpy_census(pts, rng, idx, md)
    assert np.array_equal(cp.astype(np.int64), want_pts)
    assert np.array_equal(cl.astype(np.int64), want_lv)
    # the census totals of the roofline are these sums
    _, c = oracle.fps(pts, 700, rng, census=True)
    assert c.first_pass_points == want_pts[0] and c.first_pass_leaves == want_lv[0]
    assert c.cand_points == want_pts[1:].sum() and c.cand_leaves == want_lv[1:].sum()
    assert c.iterations == len(idx) - 1


def test_shared_buckets_are_counted_once_per_cell(oracle):
    """On a 3 x 3 x 1 grid (9 buckets; x and y take 2 bits, z 1, so x's table
    is 0, 1, 8 and y's is 0, 2, 16) cells (1, 0) and (2, 1) have codes 1 and 10,
    both bucket 1 modulo 9.  Row 0 is in cell (0, 0), rows 1 and 2 in bucket 1,
    row 3 in cell (2, 2) and row 4 in cell (0, 2).  From row 0 the farthest is
    row 3 (D = 8), whose cube (half-width ceil(sqrtf(8) / 1) = 3) covers all
    nine cells: bucket 1 is reached twice, so iteration 1 counts 5 + 2 points
    and 4 + 1 leaves."""
    rng = (0.0, 3.0, 0.0, 3.0, 0.0, 1.0, 3, 3, 1)
    xl, yl, zl = morton_tables((3, 3, 1))
    assert list(xl[:3]) == [0, 1, 8] and list(yl[:3]) == [0, 2, 16] and list(zl[:1]) == [0]
    assert int(xl[1] | yl[0]) % 9 == int(xl[2] | yl[1]) % 9 == 1
    pts = np.array([[0.5, 0.5, 0.5], [1.5, 0.5, 0.5], [2.5, 1.5, 0.5], [2.5, 2.5, 0.5],
                    [0.5, 2.5, 0.5]], np.float32)
    idx, md, cp, cl = oracle.fps_trace(pts, 3, rng, leaves=True)
    want_pts, want_lv = numpy_census(pts, rng, idx, md)
    assert np.array_equal(cp.astype(np.int64), want_pts)
    assert np.array_equal(cl.astype(np.int64), want_lv)
    assert idx[1] == 3 and md[1] == np.float32(8.0)
    assert want_pts[1] == 5 + 2 and want_lv[1] == 4 + 1


def test_committed_census_prefix_matches_brute_force(oracle):
    """The first 256 iterations of the 1M-point uniform cube: per-iteration
    algorithmic bytes 16 * points + 8 * leaves, against the prefix sums in
    tests/golden/census.npz that bench.py's roofline divides by."""
    import os
    from conftest import GOLDEN
    from ns_fps_amd.workloads import make_workload
    w = make_workload("uniform_cube")
    P = w["clouds"][0]
    z = np.load(os.path.join(GOLDEN, "census.npz"), allow_pickle=False)
    k = 257
    idx, md, cp, cl = oracle.fps_trace(P, k, w["range"], leaves=True)
    want_pts, want_lv = numpy_census(P, w["range"], idx, md)
    per = 16 * want_pts + 8 * want_lv
    cum = np.concatenate([[0], np.cumsum(per)])
    assert np.array_equal(cum, z["uniform_cube__cum4096"][:k + 1].astype(np.int64))
