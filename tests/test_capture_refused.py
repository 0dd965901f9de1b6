"""Calls on a stream that is being captured into a HIP graph are refused.

Every entry point that takes a caller's stream reads results back between
batches of rounds and waits for the stream, so it cannot be captured; it
returns NSFPS_EUNSUPPORTED with a message saying so before enqueuing
anything.  The capture then ends with nothing recorded, and the same stream
serves the next call, which returns the reference's samples.  No graph is
launched here."""

import numpy as np
import pytest

from conftest import GOLDEN_CASES

pytestmark = pytest.mark.gpu

NSFPS_EUNSUPPORTED = 4
CASE = {c.name: c for c in GOLDEN_CASES}["testpy_10k_1k"]


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


def refused_under_capture(hip, stream, call):
    from ns_fps_amd.capi import NsfpsError
    hip.begin_capture(stream)
    try:
        with pytest.raises(NsfpsError) as ei:
            call()
    finally:
        assert hip.end_capture(stream) == 0  # the capture ends cleanly: nothing was recorded
    assert ei.value.status == NSFPS_EUNSUPPORTED, str(ei.value)
    assert "captured" in str(ei.value)


def test_device_entry_points_refuse_a_capturing_stream(lib, hip):
    P = CASE.points
    n, m = len(P), CASE.n_samples
    st = hip.stream_create()
    d_xyz, d_out = hip.upload(P), hip.malloc(4 * n)
    plan = lib.plan_create(P, n, CASE.range)
    try:
        calls = {
            "fps_device": lambda: lib.fps_device(d_xyz, n, m, CASE.range, d_out, st),
            "fps_device_noalloc": lambda: lib.fps_device_noalloc(d_xyz, n, m, CASE.range, d_out,
                                                                 st),
            "plan_sample": lambda: lib.plan_sample(plan, m, d_out, st),
            "fps_batched_device": lambda: lib.fps_batched_device(d_xyz, 1, n, m, d_out,
                                                                 [CASE.range], stream=st),
            "bbox_device": lambda: lib.bbox_device(d_xyz, n, (16, 16, 16), st),
        }
        for name, call in calls.items():
            refused_under_capture(hip, st, call)
            got = call()  # the same stream, no capture: the call runs
            if name == "bbox_device":
                continue
            k = got if isinstance(got, int) else got[0]
            assert np.array_equal(hip.download(d_out, k, np.int32), CASE.expected), name
    finally:
        lib.plan_destroy(plan)
        hip.free(d_xyz)
        hip.free(d_out)
        hip.stream_destroy(st)
