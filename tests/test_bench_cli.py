"""bench.py's command-line contract where no GPU is needed: more than one GPU
is refused with a JSON line naming the reason, and a machine without a HIP
device gets a JSON error instead of a CPU fallback."""

import json
import os
import subprocess
import sys

from conftest import ROOT


def run_bench(*args):
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    lines = [l for l in p.stdout.splitlines() if l.startswith("{")]
    return p.returncode, json.loads(lines[-1]) if lines else None


def test_more_than_one_gpu_is_refused():
    rc, line = run_bench("--gpus", "2")
    assert rc == 2
    assert "one GPU" in line["error"]


def test_no_device_is_an_error_not_a_fallback():
    import ctypes
    from ns_fps_amd.capi import LIB_PATH
    lib = ctypes.CDLL(LIB_PATH)
    if lib.nsfps_device_count() > 0:
        import pytest
        pytest.skip("a HIP device is visible")
    rc, line = run_bench("--steps", "1", "--warmup", "0", "--no-cpu-baseline")
    assert rc != 0
    assert "device" in line["error"]


def test_graft_entry_points_exist():
    sys.path.insert(0, ROOT)
    import __graft_entry__ as g
    assert callable(g.build) and callable(g.smoke)
