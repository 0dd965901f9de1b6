"""compute_bbox on the device (src/yuezu_fps.cpp:643-670, reached for
range=None from yuezu_fps/yuezu_fps_pybind.cpp:74-76) and the device-resident
batched call.

The device finds each cloud's bounds with order-preserving integer atomics and
derives the range (block size, inv_bs, clamp bound, cube thresholds) on one
wave per cloud.  Both must give the bits the host gives: nsfps_bbox's bounds
and nsfps_range_derive's fields, compared here word for word on clouds chosen
to stress the -/+ 1e-6 rounding, signed zeros, tiny and huge extents and
block counts that are not powers of two.  The samples of the range-less calls
are pinned by the reference's golden vectors (fps_with_bbox cases, the
batched workload's hashes)."""

import ctypes

import numpy as np
import pytest

from conftest import GOLDEN_CONFIGS, sha256_i32
from test_host_api import Range, RangeInfo

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from ns_fps_amd.capi import Lib
    L = Lib()
    if L.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    return L


@pytest.fixture(scope="module")
def hip():
    from ns_fps_amd.capi import Hip
    return Hip()


def host_bbox_and_info(lib, pts, blocks):
    r = Range()
    assert lib.lib.nsfps_bbox(pts.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(len(pts)),
                              *[ctypes.c_uint32(b) for b in blocks], ctypes.byref(r)) == 0
    info = RangeInfo()
    assert lib.lib.nsfps_range_derive(ctypes.byref(r), ctypes.byref(info), None,
                                      ctypes.c_uint64(0)) == 0
    return r, info


def clouds():
    rs = np.random.RandomState(7)
    yield "normal", rs.randn(5000, 3).astype(np.float32), (16, 16, 16)
    yield "unit_cube_30", rs.uniform(-1, 1, (20000, 3)).astype(np.float32), (30, 30, 30)
    z = rs.uniform(-1, 1, (3000, 3)).astype(np.float32)
    z[:, 0] = np.where(rs.rand(3000) < 0.5, np.float32(0.0), np.float32(-0.0))  # +-0 on x
    z[:, 1] = np.abs(z[:, 1])
    z[0, 1] = np.float32(-0.0)
    yield "signed_zeros", z, (8, 8, 8)
    yield "tiny_extent", (np.float32(1.0) + rs.rand(4000, 3).astype(np.float32)
                          * np.float32(3e-6)).astype(np.float32), (16, 16, 16)
    yield "huge_coords", (rs.randn(4000, 3) * 1e7).astype(np.float32), (64, 64, 8)
    yield "one_block_axis", rs.randn(3000, 3).astype(np.float32), (1, 32, 5)
    yield "far_offset", (rs.rand(6000, 3) * 2 + 500).astype(np.float32), (128, 128, 2)


@pytest.mark.parametrize("name,pts,blocks", list(clouds()), ids=lambda v: v if isinstance(v, str) else "")
def test_device_bbox_equals_host_bbox_and_derivation(lib, hip, name, pts, blocks):
    want_r, want_i = host_bbox_and_info(lib, pts, blocks)
    d = hip.upload(pts)
    try:
        got, info_bytes = lib.bbox_device(d, len(pts), blocks)
    finally:
        hip.free(d)
    want = (want_r.min_x, want_r.max_x, want_r.min_y, want_r.max_y, want_r.min_z, want_r.max_z,
            want_r.x_blocks, want_r.y_blocks, want_r.z_blocks)
    assert np.array(got[:6], np.float32).tobytes() == np.array(want[:6], np.float32).tobytes(), name
    assert got[6:] == want[6:]
    assert info_bytes[:ctypes.sizeof(RangeInfo)] == bytes(want_i), name


def test_range_less_calls_equal_calls_with_the_host_bbox(lib):
    """fps(range=None) and fps_with_bbox use the device's range; with the
    host's nsfps_bbox range passed explicitly the samples are the same."""
    for name, pts, blocks in clouds():
        r, _ = host_bbox_and_info(lib, pts, blocks)
        m = min(len(pts) - 1, 700)
        want = lib.fps(pts, m, (r.min_x, r.max_x, r.min_y, r.max_y, r.min_z, r.max_z, *blocks))
        assert np.array_equal(lib.fps_bbox(pts, m, blocks), want), name


def test_batched_device_matches_reference_hashes(lib, hip):
    """The batched workload (64 clouds, range=None) through the device-resident
    batched call: every cloud's samples equal the reference's."""
    from ns_fps_amd.workloads import make_workload
    w = make_workload("batched_shapes")
    g = GOLDEN_CONFIGS["batched_shapes"]
    P = np.ascontiguousarray(np.stack(w["clouds"]))
    B, n, m = P.shape[0], P.shape[1], int(w["n_samples"])
    d_xyz, d_out = hip.upload(P), hip.malloc(B * m * 4)
    try:
        for _ in range(2):  # the second call replays the first's round schedule
            lens = lib.fps_batched_device(d_xyz, B, n, m, d_out, None, w["blocks"])
            out = hip.download(d_out, B * m, np.int32).reshape(B, m)
            assert lens == g["lengths"]
            assert [sha256_i32(out[b, :lens[b]]) for b in range(B)] == g["output_sha256"]
    finally:
        hip.free(d_xyz)
        hip.free(d_out)


def test_batched_device_with_ranges_and_trivial_guards(lib, hip, oracle):
    """Explicit per-cloud ranges, and the guards (m >= n: every row, m = 0:
    nothing) through the device-resident batched call."""
    rs = np.random.RandomState(31)
    B, n, m = 5, 3000, 400
    P = rs.randn(B, n, 3).astype(np.float32)
    ranges = [(-4.0 - b, 4.0, -4.0, 4.0 + b, -5.0, 5.0, 16, 8, 32) for b in range(B)]
    d_xyz, d_out = hip.upload(P), hip.malloc(B * (n + 5) * 4)  # rows of up to n + 5
    try:
        lens = lib.fps_batched_device(d_xyz, B, n, m, d_out, ranges)
        out = hip.download(d_out, B * m, np.int32).reshape(B, m)
        for b in range(B):
            assert np.array_equal(out[b, :lens[b]], oracle.fps(P[b], m, ranges[b])), b
        lens = lib.fps_batched_device(d_xyz, B, n, n + 5, d_out, ranges)
        assert lens == [n] * B
        out = hip.download(d_out, B * (n + 5), np.int32)
        assert all(np.array_equal(out[b * (n + 5): b * (n + 5) + n], np.arange(n)) for b in range(B))
        assert lib.fps_batched_device(d_xyz, B, n, 0, d_out, ranges) == [0] * B
    finally:
        hip.free(d_xyz)
        hip.free(d_out)


def test_non_finite_points_are_refused_by_range_less_calls(lib, hip):
    pts = np.random.RandomState(3).randn(1000, 3).astype(np.float32)
    pts[17, 2] = np.inf
    from ns_fps_amd.capi import NsfpsError
    with pytest.raises(NsfpsError, match="finite"):
        lib.fps_bbox(pts, 100, (16, 16, 16))
    P = np.stack([pts, pts])
    d_xyz, d_out = hip.upload(P), hip.malloc(2 * 100 * 4)
    try:
        with pytest.raises(NsfpsError, match="finite"):
            lib.fps_batched_device(d_xyz, 2, 1000, 100, d_out)
        # and the next call still gives the reference's samples
        pts[17, 2] = 0.5
        assert len(lib.fps_bbox(pts, 100, (16, 16, 16))) == 100
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
