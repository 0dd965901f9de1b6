"""nsfps_fps_device_noalloc: the allocation-free variant of nsfps_fps_device
(workspace in the library's static device array).  Through the C ABI, its
samples must equal nsfps_fps_device's on the same device buffers, on two
calls in a row (the second with a smaller input, so the array holds the
first call's data), and a cloud beyond the array is refused with a clear
error, after which the entry point still works."""

import numpy as np
import pytest

from conftest import GOLDEN_CASES, GOLDEN_CONFIGS, sha256_i32

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


def both(lib, hip, pts, m, rng):
    d_xyz = hip.upload(np.ascontiguousarray(pts, np.float32))
    d_a, d_b = hip.malloc(max(m, 1) * 4), hip.malloc(max(m, 1) * 4)
    try:
        na = lib.fps_device(d_xyz, len(pts), m, rng, d_a)
        a = hip.download(d_a, na, np.int32)
        nb = lib.fps_device_noalloc(d_xyz, len(pts), m, rng, d_b)
        b = hip.download(d_b, nb, np.int32)
    finally:
        for d in (d_xyz, d_a, d_b):
            hip.free(d)
    return a, b


def test_noalloc_equals_device_entry_point_larger_then_smaller(lib, hip):
    from ns_fps_amd.workloads import make_workload
    w = make_workload("lidar_scan")
    a, b = both(lib, hip, w["clouds"][0], w["n_samples"], w["range"])
    assert np.array_equal(a, b)
    assert sha256_i32(b) == GOLDEN_CONFIGS["lidar_scan"]["output_sha256"][0]
    case = next(c for c in GOLDEN_CASES if c.name == "testpy_10k_1k")
    a, b = both(lib, hip, case.points, case.n_samples, case.range)
    assert np.array_equal(a, b) and np.array_equal(b, case.expected)


@pytest.mark.parametrize("name", ["general_10x10x10", "lattice_ties_16", "boundary_aligned",
                                  "early_stop_duplicates", "identity_m_gt_n"])
def test_noalloc_on_golden_cases(lib, hip, name):
    case = next(c for c in GOLDEN_CASES if c.name == name)
    if case.range is None:
        pytest.skip("the device entry points take an explicit range")
    a, b = both(lib, hip, case.points, case.n_samples, case.range)
    assert np.array_equal(a, b) and np.array_equal(b, case.expected)


def test_noalloc_refuses_a_cloud_beyond_its_array(lib, hip):
    from ns_fps_amd.capi import NsfpsError
    from ns_fps_amd.workloads import make_workload
    assert lib.noalloc_scratch_bytes() == 64 << 20
    w = make_workload("uniform_cube")
    P = w["clouds"][0]
    d_xyz, d_out = hip.upload(P), hip.malloc(1000 * 4)
    try:
        with pytest.raises(NsfpsError, match="more than the 67108864 available") as ei:
            lib.fps_device_noalloc(d_xyz, len(P), 1000, w["range"], d_out)
        assert ei.value.status == 4  # NSFPS_EUNSUPPORTED
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
    case = next(c for c in GOLDEN_CASES if c.name == "testpy_10k_1k")
    a, b = both(lib, hip, case.points, case.n_samples, case.range)
    assert np.array_equal(b, case.expected)
