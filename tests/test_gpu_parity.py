"""GPU parity: the HIP path against the reference's golden vectors (small
cases in full, the five workloads by SHA-256 of the int32 output) and against
the CPU oracle on seeded clouds, through the Python module and through the C
ABI.  Bit-exact for every index and the output length (integer/index work:
no tolerance)."""

import os

import numpy as np
import pytest

from conftest import GOLDEN_CASES, GOLDEN_CONFIGS, sha256_f32, sha256_i32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from ns_fps_amd.capi import Lib
    L = Lib()
    if L.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    return L


def run_module(yf, case):
    if case.range is None:
        return yf.fps_with_bbox(case.points, case.n_samples, *case.blocks)
    return yf.fps(case.points, case.n_samples, yf.make_range(*case.range))


@pytest.mark.parametrize("case", GOLDEN_CASES, ids=lambda c: c.name)
def test_golden_case_module(yf, lib, case):
    got = run_module(yf, case)
    assert got.dtype == np.int32
    assert np.array_equal(got, case.expected), case.name


@pytest.mark.parametrize("case", GOLDEN_CASES, ids=lambda c: c.name)
def test_golden_case_capi(lib, case):
    if case.range is None:
        got = lib.fps_bbox(case.points, case.n_samples, case.blocks)
    else:
        got = lib.fps(case.points, case.n_samples, case.range)
    assert np.array_equal(got, case.expected)


def run_workload(yf, lib, wname):
    from ns_fps_amd.workloads import make_workload
    w = make_workload(wname)
    g = GOLDEN_CONFIGS[wname]
    assert sha256_f32(np.concatenate(w["clouds"])) == g["input_sha256"]
    if len(w["clouds"]) == 1:
        outs = [yf.fps(w["clouds"][0], w["n_samples"], yf.make_range(*w["range"]))]
    else:
        idx, lens = yf.fps_batched(np.stack(w["clouds"]), w["n_samples"], None, *w["blocks"])
        outs = [idx[b, :lens[b]] for b in range(len(lens))]
    return w, g, outs


@pytest.mark.parametrize("wname", ["quickstart", "uniform_cube", "uniform_cube_30", "lidar_scan",
                                   "batched_shapes"])
def test_workload_matches_reference_hash(yf, lib, wname):
    w, g, outs = run_workload(yf, lib, wname)
    assert [len(o) for o in outs] == g["lengths"]
    assert list(outs[0][:16]) == g["head"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("mixed", ["0", "1"])
@pytest.mark.parametrize("wname", ["quickstart", "uniform_cube", "lidar_scan", "batched_shapes",
                                   "clustered"])
def test_workload_hash_in_both_leaf_layouts(yf, lib, wname, mixed, monkeypatch):
    """Leaves of one bucket each (padded or dense) and mixed leaves (runs of 64
    slots of the logical order, several buckets each, every point's own cell
    tested) give the reference's samples on every workload whose buckets
    have one cell."""
    if wname not in GOLDEN_CONFIGS:
        pytest.skip(f"golden hash of {wname} not generated")
    monkeypatch.setenv("NSFPS_MIXED", mixed)
    w, g, outs = run_workload(yf, lib, wname)
    assert yf.last_stats()["mixed"] == int(mixed)
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("hot", ["64", "128"])
@pytest.mark.parametrize("wname", ["quickstart", "uniform_cube", "uniform_cube_30", "lidar_scan",
                                   "batched_shapes", "clustered"])
def test_workload_hash_with_either_hot_set(yf, lib, wname, hot, monkeypatch):
    """The run kernel takes hot sets of 64 or 128 copies (128 where the points
    fill many buckets; NSFPS_HOT forces either, and grids whose cells share
    buckets always take 64).  Both give the reference's samples."""
    monkeypatch.setenv("NSFPS_HOT", hot)
    w, g, outs = run_workload(yf, lib, wname)
    want = 64 if wname == "uniform_cube_30" else int(hot)
    assert yf.last_stats()["hot_set"] == want
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("dense", ["0", "1"])
@pytest.mark.parametrize("wname", ["uniform_cube", "clustered"])
def test_workload_hash_with_either_walk(yf, lib, wname, dense, monkeypatch):
    """128-copy hot sets walk at most 12 coarse rows a sample on dense clouds
    (more than 64 points a filled bucket) and 16 elsewhere; NSFPS_DENSE_WALK
    forces either.  Both give the reference's samples."""
    monkeypatch.setenv("NSFPS_DENSE_WALK", dense)
    w, g, outs = run_workload(yf, lib, wname)
    assert yf.last_stats()["hot_set"] == 128
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("lb", ["0", "1"])
@pytest.mark.parametrize("wname", ["uniform_cube", "clustered", "lidar_scan"])
def test_workload_hash_with_either_update_bound(yf, lib, wname, lb, monkeypatch):
    """The update pass bounds each pick by each leaf's box for small clouds
    and for dense ones (the clustered cloud), not for the uniform cube;
    NSFPS_LEAF_BOUND forces either way.  Both give the reference's samples."""
    monkeypatch.setenv("NSFPS_LEAF_BOUND", lb)
    w, g, outs = run_workload(yf, lib, wname)
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("streams", ["1", "2", "3"])
def test_batched_hash_with_one_to_three_streams(yf, lib, streams, monkeypatch):
    """Calls of many clouds sample them in groups on their own streams (one
    group's update and gather passes beside another's run kernel; two groups
    by default); NSFPS_STREAMS sets the number.  All give the reference's
    samples."""
    monkeypatch.setenv("NSFPS_STREAMS", streams)
    w, g, outs = run_workload(yf, lib, "batched_shapes")
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("whole", ["0", "1"])
@pytest.mark.parametrize("wname", ["quickstart", "lidar_scan", "batched_shapes"])
def test_workload_hash_with_either_large_cube_form(yf, lib, wname, whole, monkeypatch):
    """Clouds in few buckets (the quickstart's 8) take the run kernel that
    applies a large-cube sample whose cube holds the list's cell box with no
    cell test per entry; NSFPS_WHOLE forces that kernel or the general one.
    Both give the reference's samples."""
    monkeypatch.setenv("NSFPS_WHOLE", whole)
    w, g, outs = run_workload(yf, lib, wname)
    assert yf.last_stats()["hot_set"] == 64
    assert [len(o) for o in outs] == g["lengths"]
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


@pytest.mark.parametrize("wname,hot", [("quickstart", 64), ("lidar_scan", 64), ("batched_shapes", 64),
                                       ("uniform_cube", 128), ("clustered", 128),
                                       ("uniform_cube_30", 64)])
def test_hot_set_size_follows_the_filled_buckets(yf, lib, wname, hot):
    """128-copy hot sets where the points fill at least 6,912 buckets (the
    uniform cube 32,768, the clustered cloud 14,321), 64 otherwise (the
    quickstart 8, the LiDAR scan 1,266, each batched cloud about 2,530) and
    wherever cells share buckets."""
    run_workload(yf, lib, wname)
    assert yf.last_stats()["hot_set"] == hot


@pytest.mark.parametrize("wname", ["quickstart", "batched_shapes"])
def test_workload_hash_with_either_logical_sort(yf, lib, wname, monkeypatch):
    """Clouds of at most 16,384 points are sorted by bucket in one workgroup
    each, in LDS; NSFPS_GLOBAL_SORT=1 takes the radix sort over all clouds
    instead.  Both give the reference's samples."""
    for env in ("1", None):
        if env:
            monkeypatch.setenv("NSFPS_GLOBAL_SORT", env)
        else:
            monkeypatch.delenv("NSFPS_GLOBAL_SORT", raising=False)
        w, g, outs = run_workload(yf, lib, wname)
        assert [len(o) for o in outs] == g["lengths"], env
        assert [sha256_i32(o) for o in outs] == g["output_sha256"], env


def test_clustered_workload_matches_reference_hash(yf, lib):
    if "clustered" not in GOLDEN_CONFIGS:
        pytest.skip("golden hash for the 8,388,608-point workload not generated")
    w, g, outs = run_workload(yf, lib, "clustered")
    assert len(outs[0]) == g["lengths"][0]
    assert list(outs[0][:16]) == g["head"]
    assert sha256_i32(outs[0]) == g["output_sha256"][0]


@pytest.mark.parametrize("seed,n,m,blocks,scale", [
    (100, 20000, 3000, (16, 16, 16), 1.0),
    (101, 50000, 6000, (32, 32, 32), 1.0),
    (102, 30000, 4000, (32, 16, 8), 3.0),
    (103, 40000, 5000, (10, 12, 6), 1.0),     # non-power-of-two: general bucket path
    (104, 25000, 25000 - 1, (8, 8, 8), 1.0),  # every point but one
])
def test_random_clouds_match_oracle(yf, oracle, seed, n, m, blocks, scale):
    rs = np.random.RandomState(seed)
    pts = (rs.randn(n, 3) * scale).astype(np.float32)
    pts[: n // 50] = pts[n // 50: 2 * (n // 50)]   # exact duplicates
    rng = (-3.0 * scale, 3.0 * scale, -3.0 * scale, 3.0 * scale, -3.0 * scale, 3.0 * scale, *blocks)
    got = yf.fps(pts, m, yf.make_range(*rng))
    assert np.array_equal(got, oracle.fps(pts, m, rng))


def test_batched_matches_per_cloud_calls(yf, oracle):
    rs = np.random.RandomState(7)
    clouds = rs.randn(6, 3000, 3).astype(np.float32)
    clouds[2] *= 50
    clouds[3, 100:200] = clouds[3, :100]
    idx, lens = yf.fps_batched(clouds, 500)
    for b in range(6):
        assert np.array_equal(idx[b, :lens[b]], oracle.fps(clouds[b], 500, None, (16, 16, 16)))
        assert np.all(idx[b, lens[b]:] == -1)
    rngs = [yf.make_range(-4, 4, -4, 4, -4, 4, 8, 8, 8)] * 6
    clouds2 = np.clip(clouds, -3.9, 3.9)
    idx2, lens2 = yf.fps_batched(clouds2, 300, rngs)
    for b in range(6):
        want = oracle.fps(clouds2[b], 300, (-4, 4, -4, 4, -4, 4, 8, 8, 8))
        assert np.array_equal(idx2[b, :lens2[b]], want)


def test_batched_mixed_grids_and_many_clouds(yf, oracle):
    """Clouds sorted together with the cloud index above the bucket: grids of
    different bucket counts in one call (tables shared only between equal
    grids), and a call of 100 clouds."""
    rs = np.random.RandomState(9)
    clouds = rs.randn(5, 2000, 3).astype(np.float32)
    clouds[1, 500:700] = clouds[1, :200]  # duplicates
    blocks = [(8, 8, 8), (16, 16, 16), (4, 8, 16), (16, 16, 16), (32, 2, 8)]
    rngs = [yf.make_range(-5, 5, -5, 5, -5, 5, *b) for b in blocks]
    idx, lens = yf.fps_batched(clouds, 400, rngs)
    for b in range(5):
        want = oracle.fps(clouds[b], 400, (-5, 5, -5, 5, -5, 5, *blocks[b]))
        assert np.array_equal(idx[b, :lens[b]], want), b
    many = rs.rand(100, 600, 3).astype(np.float32)
    idx, lens = yf.fps_batched(many, 64)
    for b in range(0, 100, 9):
        assert np.array_equal(idx[b, :lens[b]], oracle.fps(many[b], 64, None, (16, 16, 16))), b


def test_batched_clouds_above_one_workgroup(yf, oracle):
    """Clouds of more than 16,384 points in one batched call.  Without ranges
    (16^3 blocks) their bucket populations are counted by several workgroups
    per cloud, each adding its nonzero bins, and the clouds are sorted
    together by the radix sort over (cloud, bucket) keys; with a 32^3 range
    (32,768 buckets) each cloud is built on its own."""
    rs = np.random.RandomState(12)
    clouds = rs.randn(3, 40000, 3).astype(np.float32)
    clouds[1] *= 20
    clouds[2, 5000:9000] = clouds[2, :4000]  # duplicates
    idx, lens = yf.fps_batched(clouds, 1500)
    for b in range(3):
        assert np.array_equal(idx[b, :lens[b]], oracle.fps(clouds[b], 1500, None, (16, 16, 16))), b
    rng = (-80.0, 80.0, -80.0, 80.0, -80.0, 80.0, 32, 32, 32)
    idx, lens = yf.fps_batched(clouds, 1500, [yf.make_range(*rng)] * 3)
    for b in range(3):
        assert np.array_equal(idx[b, :lens[b]], oracle.fps(clouds[b], 1500, rng)), b


def test_device_pointer_entry_point(lib):
    from ns_fps_amd.capi import Hip
    hip = Hip()
    case = {c.name: c for c in GOLDEN_CASES}["testpy_10k_1k"]
    d_xyz = hip.upload(case.points)
    d_out = hip.malloc(case.n_samples * 4)
    try:
        n = lib.fps_device(d_xyz, len(case.points), case.n_samples, case.range, d_out)
        got = hip.download(d_out, n, np.int32)
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
    assert np.array_equal(got, case.expected)


TREE = {"NSFPS_ENGINE": "tree"}


@pytest.mark.parametrize("env", [
    {}, {"NSFPS_NO_PADDED": "1"}, {"NSFPS_MIXED": "0"}, {"NSFPS_MIXED": "1"},
    {"NSFPS_GLOBAL_SORT": "1"}, {"NSFPS_HOT": "64"}, {"NSFPS_HOT": "128"},
    {"NSFPS_LEAF_BOUND": "0"}, {"NSFPS_LEAF_BOUND": "1"}, {"NSFPS_HOT": "128", "NSFPS_DENSE_WALK": "1"},
    {"NSFPS_WHOLE": "0"}, {"NSFPS_WHOLE": "1"}, {"NSFPS_WHOLE": "1", "NSFPS_PROFILE": "1"},
    {"NSFPS_HOT": "128", "NSFPS_PROFILE": "1"}, {**TREE, "NSFPS_WIDE_ITERS": "0"}, {**TREE, "NSFPS_WIDE_ITERS": "1"},
    {**TREE, "NSFPS_WIDE_ITERS": "37"}, {**TREE, "NSFPS_WIDE_ITERS": "100000"},
    {**TREE, "NSFPS_NO_PADDED": "1"}, {**TREE, "NSFPS_PROFILE": "1"},
    {**TREE, "NSFPS_LATE_THREADS": "1024"},
], ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()) or "runs")
def test_schedule_and_layout_do_not_change_results(yf, env, monkeypatch):
    """The engine (speculative runs, or grid-wide steps + single-workgroup
    tree loop), where the grid-wide phase hands over, the padded, table or
    mixed-leaf layout and the profiling build are result-invariant."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for name in ["testpy_10k_1k", "lattice_ties_16", "granularity_64x64x64", "boundary_aligned"]:
        case = {c.name: c for c in GOLDEN_CASES}[name]
        assert np.array_equal(run_module(yf, case), case.expected), name


def test_repeated_and_resized_calls(yf):
    """The cached device workspace is reused and regrown between calls."""
    by = {c.name: c for c in GOLDEN_CASES}
    seq = ["trace_100_20", "quickstart_full", "testpy_100_10", "granularity_32x32x32",
           "trace_100_20"]
    for name in seq:
        case = by[name]
        assert np.array_equal(run_module(yf, case), case.expected), name


def test_non_finite_points_are_rejected(yf):
    pts = np.random.RandomState(0).randn(1000, 3).astype(np.float32)
    pts[17, 1] = np.nan
    with pytest.raises(ValueError, match="finite"):
        yf.fps(pts, 100, yf.make_range(-4, 4, -4, 4, -4, 4, 8, 8, 8))
    pts[17, 1] = np.inf
    with pytest.raises(ValueError, match="finite"):
        yf.fps(pts, 100, yf.make_range(-4, 4, -4, 4, -4, 4, 8, 8, 8))


def test_full_size_properties(yf):
    """Size-independent properties of a full-size run: distinct indices in
    range, the first sample is row 0, and sampling is deterministic."""
    from ns_fps_amd.workloads import make_workload
    w = make_workload("uniform_cube")
    r = yf.make_range(*w["range"])
    a = yf.fps(w["clouds"][0], w["n_samples"], r)
    b = yf.fps(w["clouds"][0], w["n_samples"], r)
    assert np.array_equal(a, b)
    assert a[0] == 0 and len(np.unique(a)) == len(a) == w["n_samples"]
    assert a.min() >= 0 and a.max() < len(w["clouds"][0])


def test_engine_choice(yf, monkeypatch):
    """Speculative runs on every grid (cells sharing buckets included), the
    tree loop when asked for."""
    by = {c.name: c for c in GOLDEN_CASES}
    run_module(yf, by["granularity_32x32x32"])
    st = yf.last_stats()
    assert st["engine"] == "runs" and st["rounds"] >= 1
    run_module(yf, by["general_10x10x10"])
    assert yf.last_stats()["engine"] == "runs"
    monkeypatch.setenv("NSFPS_ENGINE", "tree")
    for name in ["granularity_32x32x32", "general_10x10x10"]:
        assert np.array_equal(run_module(yf, by[name]), by[name].expected)
        assert yf.last_stats()["engine"] == "tree"


# Grids whose cells share buckets (Morton code modulo the block count): up to
# seven cells per bucket (17^3: codes run to 2^15 over 4,913 buckets), a
# single block, one axis of 1,000 blocks beside powers of two, an axis of
# 1,024 blocks, and the 30^3 grid of the general-path benchmark.
SHARED_GRIDS = [(17, 17, 17), (1, 1, 1), (3, 5, 7), (1000, 4, 2), (1024, 3, 8), (30, 30, 30),
                (20, 12, 6), (1, 64, 33)]


@pytest.mark.parametrize("blocks", SHARED_GRIDS, ids=lambda b: "x".join(map(str, b)))
def test_shared_bucket_grids_match_oracle(yf, oracle, blocks, monkeypatch):
    """The runs engine where cells share buckets (every cell of a bucket in a
    sample's cube updates the bucket's points), against the oracle, and the
    tree engine on the same input."""
    rs = np.random.RandomState(sum(blocks))
    pts = rs.uniform(-1.2, 1.2, (60000, 3)).astype(np.float32)  # some outside: clamped
    pts[:500] = pts[500:1000]                                     # duplicates
    rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, *blocks)
    want = oracle.fps(pts, 6000, rng)
    got = yf.fps(pts, 6000, yf.make_range(*rng))
    assert yf.last_stats()["engine"] == "runs"
    assert np.array_equal(got, want)
    monkeypatch.setenv("NSFPS_ENGINE", "tree")
    assert np.array_equal(yf.fps(pts, 6000, yf.make_range(*rng)), want)


@pytest.mark.parametrize("wname", ["quickstart", "lidar_scan"])
def test_workload_on_tree_engine(yf, lib, wname, monkeypatch):
    monkeypatch.setenv("NSFPS_ENGINE", "tree")
    w, g, outs = run_workload(yf, lib, wname)
    assert yf.last_stats()["engine"] == "tree"
    assert [sha256_i32(o) for o in outs] == g["output_sha256"]


def lattice(k, lo=0.0, hi=1.0):
    g = np.linspace(lo, hi, k, dtype=np.float32)
    return np.stack(np.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3).astype(np.float32)


@pytest.mark.parametrize("name,pts,m,rng", [
    # thousands of exactly equal distances: the threshold selection refines
    # down to logical ranks or falls back to the maximum key
    ("lattice40", lattice(40), 3000, (-0.01, 1.01, -0.01, 1.01, -0.01, 1.01, 16, 16, 16)),
    ("lattice32_fine", lattice(32), 5000, (-0.01, 1.01, -0.01, 1.01, -0.01, 1.01, 64, 64, 64)),
    # 2,000 distinct points, each 30 times
    ("dup30", np.repeat(np.random.RandomState(11).rand(2000, 3).astype(np.float32), 30, axis=0),
     2500, (0.0, 1.0, 0.0, 1.0, 0.0, 1.0, 32, 32, 32)),
    # 1024 blocks on one axis: early cubes span the whole axis (half-width 1024)
    ("blocks1024", np.random.RandomState(14).rand(30000, 3).astype(np.float32), 3000,
     (0.0, 1.0, 0.0, 1.0, 0.0, 1.0, 1024, 4, 4)),
    # two far clusters: the threshold window must move far between rounds
    ("two_clusters", np.concatenate([np.random.RandomState(12).randn(30000, 3) * 0.01,
                                     np.random.RandomState(13).randn(30000, 3) * 0.01 + 5.0]
                                    ).astype(np.float32),
     4000, (-1.0, 6.0, -1.0, 6.0, -1.0, 6.0, 32, 32, 32)),
], ids=lambda v: v if isinstance(v, str) else "")
def test_tie_heavy_clouds_match_oracle(yf, oracle, name, pts, m, rng):
    got = yf.fps(pts, m, yf.make_range(*rng))
    assert yf.last_stats()["engine"] == "runs"
    want = oracle.fps(pts, m, rng)
    assert len(got) == len(want)
    assert np.array_equal(got, want), name


@pytest.mark.parametrize("mixed", ["0", "1"])
def test_many_level1_nodes_on_the_runs_engine(yf, oracle, mixed, monkeypatch):
    """1M uniform points on a 128^3 grid: about 825k occupied buckets.  With a
    leaf per bucket (NSFPS_MIXED=0) that is some 12,900 level-1 nodes, above
    what the tree engine's single-workgroup loop holds; with mixed leaves
    (runs of 64 slots over about 50 buckets each) 16,384 leaves whose cell
    boxes span several cells.  The runs engine samples both exactly."""
    monkeypatch.setenv("NSFPS_MIXED", mixed)
    rs = np.random.RandomState(21)
    pts = rs.uniform(-1, 1, (1 << 20, 3)).astype(np.float32)
    rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 128, 128, 128)
    got = yf.fps(pts, 3000, yf.make_range(*rng))
    st = yf.last_stats()
    assert st["engine"] == "runs" and st["mixed"] == int(mixed)
    assert st["n_leaves"] == (16384 if mixed == "1" else st["n_leaves"])
    if mixed == "0":
        assert st["n_leaves"] > 64 * 4096
    assert np.array_equal(got, oracle.fps(pts, 3000, rng))


def test_tree_engine_level1_limit_is_reported(yf, oracle, monkeypatch):
    """The tree engine, asked for, refuses a cloud needing more than 4,096
    level-1 nodes with a message naming the limit, not sampling it wrongly;
    the runs engine (the default) samples the same cloud."""
    rs = np.random.RandomState(22)
    pts = rs.uniform(-1, 1, (1 << 20, 3)).astype(np.float32)
    rng = (-1, 1, -1, 1, -1, 1, 100, 100, 100)
    monkeypatch.setenv("NSFPS_ENGINE", "tree")
    with pytest.raises(RuntimeError, match="level-1 nodes"):
        yf.fps(pts, 100, yf.make_range(*rng))
    # the library stays usable after the refusal
    case = {c.name: c for c in GOLDEN_CASES}["general_10x10x10"]
    assert np.array_equal(run_module(yf, case), case.expected)
    monkeypatch.delenv("NSFPS_ENGINE")
    assert np.array_equal(yf.fps(pts, 1000, yf.make_range(*rng)), oracle.fps(pts, 1000, rng))
    assert yf.last_stats()["engine"] == "runs"


@pytest.mark.parametrize("engine", ["runs", "tree"])
def test_shared_buckets_visited_once(yf, engine, monkeypatch):
    """Grids whose block counts are not powers of two map several cells to one
    bucket; on the tree engine each bucket of a cube must be updated by one
    wave only (two waves on one leaf could pair a new leaf key with an old
    winner), and the runs engine must reach every cell of a bucket.  Repeated
    after a large call so that the workspace holds stale data."""
    from ns_fps_amd.workloads import make_workload
    if engine == "tree":
        monkeypatch.setenv("NSFPS_ENGINE", "tree")
    w = make_workload("lidar_scan")
    yf.fps(w["clouds"][0], w["n_samples"], yf.make_range(*w["range"]))
    cases = [c for c in GOLDEN_CASES if c.name.startswith("general_")]
    assert cases
    for rep in range(3):
        for case in cases:
            assert np.array_equal(run_module(yf, case), case.expected), (case.name, rep)
            assert yf.last_stats()["engine"] == engine


@pytest.mark.parametrize("name", ["manual_includes_all", "quickstart_full", "lattice_ties_16",
                                  "shell_duplicates"])
def test_repeated_calls_are_bit_identical(lib, name):
    """The list and its cell order are built with atomics, so they differ from
    call to call; the samples must not.  Thirty calls of one case, each against
    the reference's golden vector."""
    case = next(c for c in GOLDEN_CASES if c.name == name)
    for i in range(30):
        if case.range is None:
            got = lib.fps_bbox(case.points, case.n_samples, case.blocks)
        else:
            got = lib.fps(case.points, case.n_samples, case.range)
        assert np.array_equal(got, case.expected), (name, i)


def test_host_buffer_calls_across_a_workspace_release(lib):
    """Host-buffer inputs reach the device through a pinned buffer kept per
    device, in 2 MB chunks.  Fresh arrays each call, a 1M-point cloud (six
    chunks) and calls after nsfps_release_workspace has freed the buffer all
    return the reference's samples."""
    from ns_fps_amd.workloads import make_workload
    case = next(c for c in GOLDEN_CASES if c.name == "quickstart_full")
    w = make_workload("uniform_cube")
    P, m = w["clouds"][0], int(w["n_samples"])
    digest = GOLDEN_CONFIGS["uniform_cube"]["output_sha256"][0]
    for step in ("before", "after"):
        for _ in range(2):
            got = lib.fps(case.points.copy(), case.n_samples, case.range)
            assert np.array_equal(got, case.expected), step
        assert sha256_i32(lib.fps(P.copy(), m, w["range"])) == digest, step
        assert np.array_equal(lib.fps(case.points.copy(), case.n_samples, case.range),
                              case.expected), step
        if step == "before":
            lib.release_workspace()


@pytest.mark.parametrize("n, blocks", [
    (700000, (16, 16, 16)),  # one cell per bucket
    (320000, (15, 15, 15)),  # cells sharing buckets
    (200000, (24, 24, 24)),  # cells sharing buckets, at most 262,144 points: leaf-box bound too
])
def test_split_update_pass_on_a_mid_size_cloud(yf, oracle, n, blocks):
    """A cloud of 129 to 256 level-1 nodes: the update pass splits each node's
    leaves over four workgroups (node keys kept as four parts; the call's
    statistics say so); the samples are the oracle's."""
    rs = np.random.RandomState(31)
    pts = rs.uniform(-1, 1, (n, 3)).astype(np.float32)
    rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, *blocks)
    got = yf.fps(pts, 8000, yf.make_range(*rng))
    st = yf.last_stats()
    nl1 = (st["n_leaves"] + 63) // 64
    assert st["engine"] == "runs" and 128 < nl1 <= 256, nl1
    assert st["update_split"] == 4, st["update_split"]
    assert np.array_equal(got, oracle.fps(pts, 8000, rng))


def test_whole_node_update_pass_is_reported(yf):
    """Above 256 level-1 nodes in all, each node takes one workgroup."""
    rs = np.random.RandomState(32)
    pts = rs.uniform(-1, 1, (1 << 20, 3)).astype(np.float32)
    yf.fps(pts, 200, yf.make_range(-1, 1, -1, 1, -1, 1, 32, 32, 32))
    st = yf.last_stats()
    assert (st["n_leaves"] + 63) // 64 > 256 and st["update_split"] == 1
