"""KITTI scan path: the binary reader, the z filter, the bounds range, and FPS
on the reference's own scan against the reference's samples.

Fixtures (tests/golden/make_kitti_golden.py, from the reference library built
from its own sources): the 16,384-point cut of frame 0 with the samples of
the reference's two drivers (eval/src_cpu/compare_cpu_test_kitti.cpp and
semantickitti_example.py), and hashes of the samples on the six full frames.
The six full frames are too large for the repository's history: the build
copies them into tests/golden/kitti_frames/ (git-ignored, shipped with the
working tree; tests/golden/copy_kitti_frames.py), and NSFPS_KITTI_DIR may name
another directory holding 000000.bin .. 000005.bin.
"""

import hashlib
import json
import os
import warnings

import numpy as np
import pytest

from conftest import GOLDEN

Z = np.load(os.path.join(GOLDEN, "kitti.npz"), allow_pickle=False)
FRAMES = json.load(open(os.path.join(GOLDEN, "kitti.json")))
CMP_CASES = sorted(k[:-len("__n")] for k in Z.files if k.endswith("__n") and "_cmp_" in k)


def lowz(k16):
    """The cut with every 997th point's z set to -7.5 (as the fixture script)."""
    low = k16.copy()
    low[::997, 2] = np.float32(-7.5)
    return low


def cloud_of(case):
    k16 = Z["k16_xyz"]
    return lowz(k16) if case.startswith("lowz") else k16


def range_of(case):
    r = Z[case + "__range"].tolist()
    return tuple(r[:6]) + tuple(int(b) for b in r[6:])


def write_scan(path, xyz, stride=4):
    """A scan file: x, y, z (+ an intensity that must be ignored) as float32."""
    rec = np.zeros((len(xyz), stride), np.float32)
    rec[:, :3] = xyz
    if stride == 4:
        rec[:, 3] = np.arange(len(xyz), dtype=np.float32) * np.float32(0.25)
    rec.tofile(path)


# ---------------------------------------------------------------- CPU ----

def test_reader_strides_partial_and_empty(tmp_path):
    from ns_fps_amd import kitti
    rng = np.random.default_rng(7)
    xyz = rng.standard_normal((37, 3)).astype(np.float32)
    for stride in (3, 4):
        p = tmp_path / f"s{stride}.bin"
        write_scan(p, xyz, stride)
        got = kitti.read_bin_pointcloud(str(p), stride)
        assert got.dtype == np.float32 and got.flags.c_contiguous
        assert np.array_equal(got, xyz)
    # a trailing partial record is dropped with a warning (the C++ reader's
    # num_floats / stride)
    p = tmp_path / "partial.bin"
    np.concatenate([np.hstack([xyz, np.zeros((37, 1), np.float32)]).ravel(),
                    np.ones(2, np.float32)]).tofile(p)
    with pytest.warns(UserWarning):
        got = kitti.read_bin_pointcloud(str(p), 4)
    assert np.array_equal(got, xyz)
    e = tmp_path / "empty.bin"
    e.write_bytes(b"")
    with pytest.raises(ValueError):
        kitti.read_bin_pointcloud(str(e))
    with pytest.raises(ValueError):
        kitti.read_bin_pointcloud(str(p), 5)
    with pytest.raises(OSError):
        kitti.read_bin_pointcloud(str(tmp_path / "missing.bin"))
    # load_kitti_point_cloud is the stride-4 read
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        q = tmp_path / "s4b.bin"
        write_scan(q, Z["k16_xyz"], 4)
        assert np.array_equal(kitti.load_kitti_point_cloud(str(q)), Z["k16_xyz"])


def test_keep_z_at_least_hand_case():
    from ns_fps_amd import kitti
    pts = np.array([[0, 0, -5.0], [1, 1, -5.000001], [2, 2, 3.0], [3, 3, np.nan],
                    [4, 4, -100.0], [5, 5, 0.0]], np.float32)
    kept, rows = kitti.keep_z_at_least(pts)
    # z >= -5 keeps -5 itself; NaN fails the comparison, as in C++
    assert rows.tolist() == [0, 2, 5]
    assert np.array_equal(kept, pts[[0, 2, 5]])


def test_bounds_tuple_hand_case_and_golden_ranges():
    from ns_fps_amd import kitti
    pts = np.array([[0.5, -2.0, 1.0], [3.0, 4.0, -1.5]], np.float32)
    f = np.float32
    want = (float(f(0.5) - f(1e-6)), float(f(3.0) + f(1e-6)), float(f(-2.0) - f(1e-6)),
            float(f(4.0) + f(1e-6)), float(f(-1.5) - f(1e-6)), float(f(1.0) + f(1e-6)),
            128, 128, 2)
    assert kitti.bounds_tuple(pts) == want
    assert kitti.bounds_tuple(pts, eps=0.0)[:6] == (0.5, 3.0, -2.0, 4.0, -1.5, 1.0)
    # float32 arithmetic: 3.0 + 1e-6 rounds to 3.0 + 4 ulps, not to the double sum
    assert want[1] == float(np.nextafter(np.nextafter(np.nextafter(np.nextafter(
        f(3.0), f(4)), f(4)), f(4)), f(4))) and want[1] != 3.0 + 1e-6
    for case in CMP_CASES:
        kept, _ = kitti.keep_z_at_least(cloud_of(case))
        assert kitti.bounds_tuple(kept) == range_of(case)
    assert kitti.bounds_tuple(Z["k16_xyz"], eps=0.0) == range_of("k16_ex_1024")


@pytest.mark.parametrize("case", CMP_CASES + ["k16_ex_1024"])
def test_oracle_matches_reference_on_scan(oracle, case):
    """The restatement reproduces the reference's samples on the real scan."""
    pts = cloud_of(case)
    rows = np.flatnonzero(pts[:, 2] >= np.float32(-5.0)) if "_cmp_" in case else \
        np.arange(len(pts))
    got = oracle.fps(np.ascontiguousarray(pts[rows]), int(Z[case + "__n"]), range_of(case))
    assert np.array_equal(rows[got], Z[case + "__expected"])


def test_fixture_cases_cover_filter():
    """lowz drops points; its samples are record numbers of the unfiltered cut."""
    exp = Z["lowz_cmp_1024__expected"]
    assert len(exp) == 1024 and not np.any(exp % 997 == 0)
    assert len(np.flatnonzero(lowz(Z["k16_xyz"])[:, 2] < -5)) == len(range(0, 16384, 997))


# ---------------------------------------------------------------- GPU ----

@pytest.mark.gpu
@pytest.mark.parametrize("case", CMP_CASES)
def test_gpu_scan_file_run(tmp_path, case):
    """compare_cpu_test_kitti.cpp's run (read, z >= -5, bounds -/+ 1e-6,
    128 x 128 x 2) on the HIP path: the reference's record numbers."""
    from ns_fps_amd import kitti
    p = tmp_path / "scan.bin"
    write_scan(p, cloud_of(case), 4)
    got, kept = kitti.fps_kitti_file(str(p), int(Z[case + "__n"]))
    assert kept == len(np.flatnonzero(cloud_of(case)[:, 2] >= -5))
    assert np.array_equal(got, Z[case + "__expected"])


@pytest.mark.gpu
def test_gpu_semantickitti_example_run():
    """semantickitti_example.py's run (exact bounds, 128 x 128 x 2, 1024)."""
    from ns_fps_amd import kitti
    got = kitti.sample_kitti_point_cloud(Z["k16_xyz"], 1024)
    assert got.dtype == np.int32
    assert np.array_equal(got, Z["k16_ex_1024__expected"])


@pytest.mark.gpu
@pytest.mark.parametrize("frame", sorted(FRAMES))
@pytest.mark.parametrize("n", [1024, 16384])
def test_gpu_full_frames(frame, n):
    d = os.environ.get("NSFPS_KITTI_DIR") or os.path.join(GOLDEN, "kitti_frames")
    path = os.path.join(d, frame)
    if not os.path.exists(path):
        pytest.skip("full KITTI frames not present (tests/golden/copy_kitti_frames.py, or set "
                    "NSFPS_KITTI_DIR)")
    rec = FRAMES[frame]
    with open(path, "rb") as fh:
        assert hashlib.sha256(fh.read()).hexdigest() == rec["file_sha256"]
    from ns_fps_amd import kitti
    got, kept = kitti.fps_kitti_file(path, n)
    assert kept == rec["kept"]
    assert len(got) == rec[str(n)]["len"]
    assert got[:8].tolist() == rec[str(n)]["head"]
    assert hashlib.sha256(got.astype(np.int64).tobytes()).hexdigest() == rec[str(n)]["sha256"]
