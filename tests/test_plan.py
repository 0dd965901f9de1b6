"""The plan entry points (nsfps_plan_create / _sample / _destroy): a cloud
built once and sampled many times, the split of the reference GPU driver's
FpsGPU::initialize / FpsGPU::sample (eval/src_gpu/yuezu_fps_gpu.h:90-126).
Every sampling of a plan must give the samples of a fresh call on the same
points and range -- the reference's golden vectors and hashes -- whatever was
sampled from the plan before, and plans must not disturb each other."""

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


def sample(lib, hip, plan, m):
    d_out = hip.malloc(max(m, 1) * 4)
    try:
        n = lib.plan_sample(plan, m, d_out)
        return hip.download(d_out, n, np.int32)
    finally:
        hip.free(d_out)


def test_one_plan_many_sample_counts_on_the_uniform_cube(lib, hip):
    from ns_fps_amd.workloads import make_workload
    w = make_workload("uniform_cube")
    g = GOLDEN_CONFIGS["uniform_cube"]
    P = w["clouds"][0]
    d_xyz = hip.upload(P)
    plan = lib.plan_create(d_xyz, len(P), w["range"], on_device=True)
    try:
        hip.free(d_xyz)  # the plan does not read its input again
        d_xyz = None
        a = sample(lib, hip, plan, 1000)
        full = sample(lib, hip, plan, 65536)
        b = sample(lib, hip, plan, 1000)
        assert sha256_i32(full) == g["output_sha256"][0] and len(full) == 65536
        # fewer samples: the same sequence, cut short
        assert np.array_equal(a, full[:1000]) and np.array_equal(b, full[:1000])
        assert lib.stats()["engine"] == 1
    finally:
        lib.plan_destroy(plan)
        if d_xyz is not None:
            hip.free(d_xyz)


def test_two_plans_alive_at_once(lib, hip):
    """Interleaved samplings of a LiDAR-scan plan (host input) and a
    quick-start plan (device input), each against its golden hash."""
    from ns_fps_amd.workloads import make_workload
    wl, wq = make_workload("lidar_scan"), make_workload("quickstart")
    pl = lib.plan_create(wl["clouds"][0], len(wl["clouds"][0]), wl["range"], on_device=False)
    d_q = hip.upload(wq["clouds"][0])
    pq = lib.plan_create(d_q, len(wq["clouds"][0]), wq["range"], on_device=True)
    try:
        for _ in range(2):
            ql = sample(lib, hip, pq, wq["n_samples"])
            ll = sample(lib, hip, pl, wl["n_samples"])
            assert sha256_i32(ql) == GOLDEN_CONFIGS["quickstart"]["output_sha256"][0]
            assert sha256_i32(ll) == GOLDEN_CONFIGS["lidar_scan"]["output_sha256"][0]
    finally:
        lib.plan_destroy(pl)
        lib.plan_destroy(pq)
        hip.free(d_q)


@pytest.mark.parametrize("name", ["testpy_10k_1k", "general_10x10x10", "lattice_ties_16",
                                  "tie_bucket_order", "early_stop_duplicates"])
def test_plan_on_golden_cases(lib, hip, name):
    """Golden cases through a plan: a grid whose cells share buckets
    (general_10x10x10), ties, and the trivial guards (m >= n, m = 0, m = 1)."""
    case = next(c for c in GOLDEN_CASES if c.name == name)
    if case.range is None:
        pytest.skip("a plan takes an explicit range")
    plan = lib.plan_create(case.points, len(case.points), case.range, on_device=False)
    try:
        for _ in range(2):
            assert np.array_equal(sample(lib, hip, plan, case.n_samples), case.expected)
        assert len(sample(lib, hip, plan, 0)) == 0
        assert list(sample(lib, hip, plan, 1)) == [0]
        n = len(case.points)
        assert list(sample(lib, hip, plan, n + 3)) == list(range(n))
    finally:
        lib.plan_destroy(plan)


def test_plan_rejects_bad_arguments(lib):
    from ns_fps_amd.capi import NsfpsError
    with pytest.raises(NsfpsError, match="max > min"):
        lib.plan_create(np.zeros((10, 3), np.float32), 10, (1, 1, 0, 1, 0, 1, 4, 4, 4))
    with pytest.raises(NsfpsError, match="finite"):
        bad = np.zeros((100, 3), np.float32)
        bad[5, 0] = np.nan
        lib.plan_create(bad, 100, (-1, 1, -1, 1, -1, 1, 4, 4, 4))
    lib.plan_destroy(None)  # ignored
