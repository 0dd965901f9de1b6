"""Error paths of the host library, forced from the host.

NSFPS_INJECT=<kind>:<n> makes the n-th allocation, kernel launch, copy or
wait of a call fail inside the library's HIP wrappers without reaching the
runtime (every kernel that was launched still runs to its end).  Each case
checks the status the C ABI returns (NSFPS_ENOMEM for allocations,
NSFPS_EDEVICE otherwise) and its message, then that the next call, with
nothing injected, returns the reference's samples: a failed call leaves the
cached workspace, the pinned staging buffer and the round schedule usable.
The reference has no such paths (a CPU library whose allocations throw);
its golden vectors pin the calls after the failures."""

import numpy as np
import pytest

from conftest import GOLDEN_CASES, GOLDEN_CONFIGS, sha256_i32

pytestmark = pytest.mark.gpu

NSFPS_EDEVICE, NSFPS_ENOMEM = 2, 3


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


CASE = {c.name: c for c in GOLDEN_CASES}["testpy_10k_1k"]


def golden_call(lib):
    return lib.fps(CASE.points, CASE.n_samples, CASE.range)


def expect_failure(lib, monkeypatch, spec, status, call):
    from ns_fps_amd.capi import NsfpsError
    monkeypatch.setenv("NSFPS_INJECT", spec)
    try:
        with pytest.raises(NsfpsError) as ei:
            call()
    finally:
        monkeypatch.delenv("NSFPS_INJECT")
    assert ei.value.status == status, (spec, str(ei.value))
    assert "injected failure" in str(ei.value), (spec, str(ei.value))


def sweep(lib, monkeypatch, kind, call, check, statuses=(NSFPS_EDEVICE,)):
    """Fails the 1st, 2nd, ... operation of `kind` in `call` until a call
    finishes without reaching the armed operation; after every failure the
    next call must pass `check`.  Returns how many operations failed."""
    from ns_fps_amd.capi import NsfpsError
    n = 1
    while True:
        monkeypatch.setenv("NSFPS_INJECT", f"{kind}:{n}")
        raised, got = None, None
        try:
            got = call()
        except NsfpsError as e:
            raised = e
        finally:
            monkeypatch.delenv("NSFPS_INJECT")
        if raised is None:  # the call has fewer such operations: it ran normally
            check(got)
            return n - 1
        assert raised.status in statuses, (kind, n, str(raised))
        assert "injected failure" in str(raised), (kind, n, str(raised))
        check(call())
        n += 1
        assert n < 1000, "the injection never stops firing"


def golden_check(got):
    assert np.array_equal(got, CASE.expected)


@pytest.mark.parametrize("kind", ["launch", "copy", "sync", "any"])
def test_every_operation_of_a_host_buffer_call_fails_cleanly(lib, monkeypatch, kind):
    golden_check(golden_call(lib))  # workspace, staging buffer and round schedule warm
    failed = sweep(lib, monkeypatch, kind, lambda: golden_call(lib), golden_check,
                   (NSFPS_EDEVICE, NSFPS_ENOMEM) if kind == "any" else (NSFPS_EDEVICE,))
    assert failed >= (8 if kind in ("launch", "any") else 2), (kind, failed)


def test_workspace_allocation_failure(lib, monkeypatch):
    """The device workspace is freed; the next call must allocate it, and that
    allocation fails; the call after it allocates again."""
    lib.release_workspace()
    expect_failure(lib, monkeypatch, "alloc:1", NSFPS_ENOMEM, lambda: golden_call(lib))
    assert np.array_equal(golden_call(lib), CASE.expected)


def test_pinned_staging_failure_falls_back_to_direct_copies(lib, monkeypatch):
    """Without the pinned staging buffer (its allocation fails) the input is
    copied from the caller's array directly: the call still succeeds."""
    lib.release_workspace()
    monkeypatch.setenv("NSFPS_INJECT", "alloc:2")  # 1: the workspace, 2: the staging buffer
    try:
        assert np.array_equal(golden_call(lib), CASE.expected)
    finally:
        monkeypatch.delenv("NSFPS_INJECT")
    assert np.array_equal(golden_call(lib), CASE.expected)


@pytest.mark.parametrize("kind", ["launch", "copy", "sync", "any"])
def test_every_operation_of_a_device_call_fails_cleanly(lib, hip, monkeypatch, kind):
    P = CASE.points
    d_xyz, d_out = hip.upload(P), hip.malloc(CASE.n_samples * 4)
    try:
        def call():
            n = lib.fps_device(d_xyz, len(P), CASE.n_samples, CASE.range, d_out)
            return hip.download(d_out, n, np.int32)
        golden_check(call())
        assert sweep(lib, monkeypatch, kind, call, golden_check) >= 1
    finally:
        hip.free(d_xyz)
        hip.free(d_out)


@pytest.mark.parametrize("kind", ["launch", "copy", "sync"])
def test_every_operation_of_a_batched_call_fails_cleanly(lib, monkeypatch, kind):
    from ns_fps_amd.workloads import make_workload
    w = make_workload("batched_shapes")
    P = np.stack(w["clouds"][:16])
    g = GOLDEN_CONFIGS["batched_shapes"]

    def call():
        return lib.fps_batched(P, w["n_samples"], None, w["blocks"])

    def check(outs):
        assert [sha256_i32(o) for o in outs] == g["output_sha256"][:16]
    assert sweep(lib, monkeypatch, kind, call, check) >= 1


def test_plan_failures(lib, hip, monkeypatch):
    """A plan whose allocation fails is not created; a sampling that fails
    leaves the plan usable."""
    expect_failure(lib, monkeypatch, "alloc:1", NSFPS_ENOMEM,
                   lambda: lib.plan_create(CASE.points, len(CASE.points), CASE.range))
    plan = lib.plan_create(CASE.points, len(CASE.points), CASE.range)
    d_out = hip.malloc(CASE.n_samples * 4)
    try:
        def sample():
            n = lib.plan_sample(plan, CASE.n_samples, d_out)
            return hip.download(d_out, n, np.int32)
        golden_check(sample())
        for kind in ("launch", "copy", "sync"):
            assert sweep(lib, monkeypatch, kind, sample, golden_check) >= 1, kind
    finally:
        lib.plan_destroy(plan)
        hip.free(d_out)


def test_staged_host_copies_fail_cleanly(lib, oracle, monkeypatch):
    """A host input of 4 MB or more is copied into the pinned stage by the
    host pool's threads and sent in one DMA; a result of 256 KB or more comes
    back through the stage and the pool's threads copy it out.  Every copy of
    such a call fails in turn; the call after each failure returns the
    oracle's samples."""
    rs = np.random.RandomState(41)
    pts = rs.uniform(-1, 1, (1 << 20, 3)).astype(np.float32)  # 12 MB in, 256 KB out
    rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 32, 32, 32)
    want = oracle.fps(pts, 65536, rng)

    def check(got):
        assert np.array_equal(got, want)
    check(lib.fps(pts, 65536, rng))
    assert sweep(lib, monkeypatch, "copy", lambda: lib.fps(pts, 65536, rng), check) >= 3


def test_unarmed_or_unknown_injection_changes_nothing(lib, monkeypatch):
    for spec in ["", "nothing:1", "launch:100000"]:
        monkeypatch.setenv("NSFPS_INJECT", spec)
        assert np.array_equal(golden_call(lib), CASE.expected), spec
    monkeypatch.delenv("NSFPS_INJECT")
