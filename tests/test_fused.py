"""Fused rounds: one launch carries the run and helper workgroups that apply
its picks while it goes on.  The samples must not depend on it: the same
golden hashes with the default choice, with fused rounds forced
(NSFPS_FUSED=1), with classic rounds (NSFPS_NO_FUSED=1), and when the host
forces every helper to give up waiting (NSFPS_HELP_WAIT_US=0), in which case
the host redoes the rounds' update passes (stats "repairs")."""

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


@pytest.mark.parametrize("wname", ["uniform_cube", "lidar_scan", "quickstart"])
@pytest.mark.parametrize("env", [{}, {"NSFPS_FUSED": "1"}, {"NSFPS_NO_FUSED": "1"},
                                 {"NSFPS_FUSED": "1", "NSFPS_HELP_WAIT_US": "0"}],
                         ids=["default", "fused", "classic", "forced_give_up"])
def test_rounds_give_the_reference_samples(yf, lib, monkeypatch, wname, env):
    from ns_fps_amd.workloads import make_workload
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    w = make_workload(wname)
    got = yf.fps(w["clouds"][0], w["n_samples"], yf.make_range(*w["range"]))
    assert sha256_i32(got) == GOLDEN_CONFIGS[wname]["output_sha256"][0]
    st = yf.last_stats()
    assert st["engine"] == "runs"
    if "NSFPS_HELP_WAIT_US" in env:
        assert st["repairs"] >= 1  # the give-up path ran and was repaired
    else:
        assert st["repairs"] == 0


@pytest.mark.parametrize("name", ["testpy_10k_1k", "lattice_ties_16", "boundary_aligned",
                                  "early_stop_duplicates", "granularity_64x64x64",
                                  "manual_z_too_tight"])
def test_forced_give_up_on_golden_cases(yf, monkeypatch, name):
    monkeypatch.setenv("NSFPS_FUSED", "1")
    monkeypatch.setenv("NSFPS_HELP_WAIT_US", "0")
    case = next(c for c in GOLDEN_CASES if c.name == name)
    got = yf.fps(case.points, case.n_samples, yf.make_range(*case.range))
    assert np.array_equal(got, case.expected)


def test_fused_rounds_repeated_calls(lib, monkeypatch):
    """Thirty calls of one golden case: the helpers' records, histograms and
    the run's publication are rebuilt every call."""
    monkeypatch.setenv("NSFPS_FUSED", "1")
    case = next(c for c in GOLDEN_CASES if c.name == "quickstart_full")
    for i in range(30):
        assert np.array_equal(lib.fps(case.points, case.n_samples, case.range), case.expected), i
