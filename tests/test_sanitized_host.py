"""The host library's CPU tests under AddressSanitizer and
UndefinedBehaviorSanitizer (python -m ns_fps_amd.sanitize): range derivation
and thresholds, compute_bbox on the worker pool (and in a forked child),
argument checks, error statuses and messages, the module's surface and
guards.  The sanitized library and module are built by
__graft_entry__.build() (python -m ns_fps_amd.build sanitize); every report
is fatal, and the run passes only without one."""

import os

import pytest


def test_host_library_under_asan_and_ubsan():
    from ns_fps_amd import build as b
    from ns_fps_amd import sanitize
    lib = os.path.join(b.SAN_DIR, "ns_fps_amd", "libnsfps.so")
    if not os.path.exists(lib):
        pytest.skip("sanitized build missing: python -m ns_fps_amd.build sanitize")
    rc, out = sanitize.run(build=False)
    found = sanitize.reports()
    assert not found, "\n".join(text[:3000] for _, text in found)
    assert rc == 0, out[-3000:]
    assert " passed" in out and "failed" not in out, out[-2000:]
