"""The grouping step after sampling: gather of the sampled points and the ball
query (PointNet++'s query_ball_point on the FPS distance).  The reference has
no such step, so there are no reference vectors: the oracle's literal scan is
pinned by an independent NumPy brute force (hits = np.nonzero(d2 < r2) in
input order, with the documented padding), and the HIP path is checked
against the oracle on the GPU.
"""

import numpy as np
import pytest

from conftest import GOLDEN


@pytest.fixture(scope="module")
def lib():
    from ns_fps_amd.capi import Lib
    L = Lib()
    if L.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    return L


def numpy_ball_query(points, centers, radius, nsample):
    """Independent statement: float32 ((dx*dx + dy*dy) + dz*dz) < r*r; the first
    nsample hits in index order; pad with the first hit, or zeros."""
    p = np.asarray(points, np.float32)
    r2 = np.float32(radius) * np.float32(radius)
    out = np.zeros((len(centers), nsample), np.int32)
    for j, c in enumerate(np.asarray(centers, np.float32)):
        d = p - c
        d2 = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
        hits = np.flatnonzero(d2 < r2)[:nsample]
        if len(hits):
            out[j, :] = hits[0]
            out[j, :len(hits)] = hits
    return out


def cases():
    out = []
    for seed, n, m, radius, nsample in [(0, 500, 40, 0.3, 16), (1, 3000, 200, 0.1, 32),
                                        (2, 2000, 64, 0.05, 8), (3, 1000, 50, 2.0, 64),
                                        (4, 700, 30, 0.0, 4), (5, 900, 25, 0.25, 1),
                                        (6, 129, 70, 0.4, 100)]:
        rs = np.random.RandomState(seed)
        pts = rs.uniform(-1, 1, (n, 3)).astype(np.float32)
        pts[10:20] = pts[0]  # duplicates: distance 0 hits
        cen = np.concatenate([pts[rs.randint(0, n, m // 2)],
                              rs.uniform(-1.5, 1.5, (m - m // 2, 3)).astype(np.float32)])
        out.append((f"s{seed}_n{n}_m{m}_r{radius}_k{nsample}", pts, cen, radius, nsample))
    return out


CASES = cases()


@pytest.mark.parametrize("name,pts,cen,radius,nsample", CASES, ids=[c[0] for c in CASES])
def test_oracle_ball_query_matches_numpy(oracle, name, pts, cen, radius, nsample):
    from oracle import ball_query
    got = ball_query(oracle, pts, cen, radius, nsample)
    assert np.array_equal(got, numpy_ball_query(pts, cen, radius, nsample))


def test_oracle_ball_query_hand_case(oracle):
    from oracle import ball_query
    pts = np.array([[0, 0, 0], [1, 0, 0], [0.5, 0, 0], [3, 0, 0], [0.1, 0, 0]], np.float32)
    cen = np.array([[0, 0, 0], [3, 0, 0], [10, 0, 0]], np.float32)
    got = ball_query(oracle, pts, cen, 0.6, 3)
    # center 0: rows 0, 2, 4 (1 is at distance 1; strict <); center 1: only row 3,
    # padded with it; center 2: nothing -> zeros
    assert got.tolist() == [[0, 2, 4], [3, 3, 3], [0, 0, 0]]
    # strict: a point exactly at the radius is outside
    assert ball_query(oracle, pts, cen[:1], 1.0, 5).tolist() == [[0, 2, 4, 0, 0]]


def test_oracle_gather_matches_numpy(oracle):
    from oracle import gather_points
    pts = np.random.RandomState(9).randn(100, 3).astype(np.float32)
    idx = np.array([5, 0, 99, 5], np.int32)
    assert np.array_equal(gather_points(oracle, pts, idx), pts[idx])
    with pytest.raises(ValueError):
        gather_points(oracle, pts, np.array([100], np.int32))


def test_module_validates_grouping_arguments_on_the_host(yf):
    pts = np.zeros((10, 3), np.float32)
    with pytest.raises(ValueError):
        yf.ball_query(pts, pts[:2], 0.5, 0)       # nsample >= 1
    with pytest.raises(ValueError):
        yf.ball_query(pts, pts[:2], -0.5, 4)      # radius >= 0
    with pytest.raises(ValueError):
        yf.ball_query(pts, pts[:2], float("nan"), 4)
    with pytest.raises(ValueError):
        yf.gather_points(pts, np.array([3, 10], np.int32))  # index outside the cloud
    with pytest.raises(ValueError):
        yf.gather_points(pts, np.array([-1], np.int32))
    with pytest.raises(ValueError):
        yf.ball_query(np.zeros((4, 2), np.float32), pts[:2], 0.5, 4)  # shape


@pytest.mark.gpu
@pytest.mark.parametrize("name,pts,cen,radius,nsample", CASES, ids=[c[0] for c in CASES])
def test_gpu_ball_query_matches_oracle(yf, oracle, name, pts, cen, radius, nsample):
    from oracle import ball_query
    got = yf.ball_query(pts, cen, radius, nsample)
    assert got.dtype == np.int32 and got.shape == (len(cen), nsample)
    assert np.array_equal(got, ball_query(oracle, pts, cen, radius, nsample))


def grid_cases():
    """Clouds above the scan-only size (8,192 points): the grid path, with its
    overflow to the ordered scan, non-finite points, far and degenerate
    clouds."""
    out = []
    rs = np.random.RandomState(21)
    u = rs.uniform(-1, 1, (40000, 3)).astype(np.float32)
    cu = np.concatenate([u[rs.randint(0, len(u), 1800)],
                         rs.uniform(-1.3, 1.3, (400, 3))]).astype(np.float32)
    out.append(("uniform_r0.05_k32", u, cu, 0.05, 32))
    out.append(("uniform_r0.2_k64", u, cu, 0.2, 64))       # some rows over 1,024 hits
    out.append(("uniform_r0.6_k16", u, cu[:300], 0.6, 16))  # every row over 1,024 hits
    out.append(("uniform_r0.01_k8", u, cu, 0.01, 8))        # mostly 0-2 hits
    c = rs.uniform(-5, 5, (40, 3))
    cl = (c[rs.randint(0, 40, 30000)] + rs.randn(30000, 3) * 0.05).astype(np.float32)
    out.append(("clusters_r0.1_k32", cl, cl[rs.randint(0, len(cl), 500)], 0.1, 32))
    bad = u[:20000].copy()
    bad[::97, 1] = np.nan
    bad[5::101, 0] = np.inf
    out.append(("nonfinite_r0.1_k16", bad, cu[:400], 0.1, 16))
    far = np.array([[1e4, 0, 0], [0, -1e4, 0], [1.001, 0, 0], [np.nan, 0, 0]], np.float32)
    out.append(("far_centers", u, far, 0.3, 8))
    same = np.tile(np.array([[0.25, -0.5, 2.0]], np.float32), (9000, 1))
    out.append(("identical_points", same, same[:5], 1e-3, 12))
    flat = u[:30000].copy()
    flat[:, 2] = 0.5  # one cell thick
    out.append(("plane_r0.08_k24", flat, flat[rs.randint(0, 30000, 300)], 0.08, 24))
    return out


GRID = grid_cases()


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["grid", "scan", "auto"])
@pytest.mark.parametrize("name,pts,cen,radius,nsample", GRID, ids=[c[0] for c in GRID])
def test_gpu_grid_ball_query_matches_oracle(yf, oracle, monkeypatch, path, name, pts, cen, radius,
                                            nsample):
    from oracle import ball_query
    if path != "auto":
        monkeypatch.setenv("NSFPS_BALL_QUERY", path)
    got = yf.ball_query(pts, cen, radius, nsample)
    assert np.array_equal(got, ball_query(oracle, pts, cen, radius, nsample))


@pytest.mark.parametrize("name,pts,cen,radius,nsample", GRID[:1] + GRID[5:8],
                         ids=[c[0] for c in GRID[:1] + GRID[5:8]])
def test_oracle_matches_numpy_on_grid_cases(oracle, name, pts, cen, radius, nsample):
    from oracle import ball_query
    k = min(len(cen), 60)
    assert np.array_equal(ball_query(oracle, pts, cen[:k], radius, nsample),
                          numpy_ball_query(pts, cen[:k], radius, nsample))


@pytest.mark.gpu
def test_gpu_sample_and_group_on_kitti_cut(yf, oracle):
    """FPS of the reference's KITTI cut (its samples), then gather and ball
    query around them: the set-abstraction front end, all on the HIP path."""
    import os
    from oracle import ball_query
    z = np.load(os.path.join(GOLDEN, "kitti.npz"), allow_pickle=False)
    pts = z["k16_xyz"]
    r = z["k16_ex_1024__range"].tolist()
    idx = yf.fps(pts, 1024, yf.make_range(*r[:6], *(int(b) for b in r[6:])))
    assert np.array_equal(idx, z["k16_ex_1024__expected"])
    cen = yf.gather_points(pts, idx)
    assert np.array_equal(cen, pts[idx])
    got = yf.ball_query(pts, cen, 1.5, 32)
    assert np.array_equal(got, ball_query(oracle, pts, cen, 1.5, 32))
    assert np.all(got[:, 0] <= idx)  # the first hit is never after the center itself


@pytest.mark.gpu
def test_gpu_grouping_device_entry_points(lib):
    from ns_fps_amd.capi import Hip
    hip = Hip()
    rs = np.random.RandomState(11)
    pts = rs.uniform(-1, 1, (5000, 3)).astype(np.float32)
    idx = rs.randint(0, 5000, 300).astype(np.int32)
    bufs = []
    try:
        d_p = hip.upload(pts); bufs.append(d_p)
        d_i = hip.upload(idx); bufs.append(d_i)
        d_c = hip.malloc(300 * 12); bufs.append(d_c)
        d_o = hip.malloc(300 * 24 * 4); bufs.append(d_o)
        lib.gather_points_device(d_p, 5000, d_i, 300, d_c)
        cen = hip.download(d_c, 900, np.float32).reshape(300, 3)
        assert np.array_equal(cen, pts[idx])
        lib.ball_query_device(d_p, 5000, d_c, 300, 0.2, 24, d_o)
        got = hip.download(d_o, 300 * 24, np.int32).reshape(300, 24)
        assert np.array_equal(got, lib.ball_query(pts, cen, 0.2, 24))
        assert np.array_equal(got, numpy_ball_query(pts, cen, 0.2, 24))
        # an index outside the cloud is reported (its row zeroed), not read
        bad = idx.copy()
        bad[7] = 5000
        d_b = hip.upload(bad); bufs.append(d_b)
        with pytest.raises(Exception, match="outside"):
            lib.gather_points_device(d_p, 5000, d_b, 300, d_c)
    finally:
        for b in bufs:
            hip.free(b)


@pytest.mark.gpu
def test_gpu_grid_ball_query_at_full_size(yf, oracle):
    """The uniform cube's 1,048,576 points (the FPS workload) around 512 of its
    own points and 64 outside them: the grid path at its real size."""
    from ns_fps_amd.workloads import make_workload
    from oracle import ball_query
    P = make_workload("uniform_cube")["clouds"][0]
    rs = np.random.RandomState(33)
    cen = np.concatenate([P[rs.randint(0, len(P), 512)],
                          rs.uniform(-1.2, 1.2, (64, 3)).astype(np.float32)])
    for radius, k in [(0.05, 32), (0.02, 8)]:
        got = yf.ball_query(P, cen, radius, k)
        assert np.array_equal(got, ball_query(oracle, P, cen, radius, k)), (radius, k)
