"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on a
CPU-only machine (the C ABI library still loads there and fails loudly on
compute calls)."""

import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import ORACLE_SO, Oracle
    if not os.path.exists(ORACLE_SO):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True,
                       stdout=subprocess.DEVNULL)
    return Oracle()


def _module_override():
    """NSFPS_MODULE names another build of the module (the sanitized one): it
    is imported under the module's own name, so every import of it gets it."""
    path = os.environ.get("NSFPS_MODULE")
    if not path or "yuezu_fps.yuezu_fps_module" in sys.modules:
        return
    import importlib.util
    import yuezu_fps  # noqa: F401  (the package the module belongs to)
    spec = importlib.util.spec_from_file_location("yuezu_fps.yuezu_fps_module", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules["yuezu_fps.yuezu_fps_module"] = mod


_module_override()


@pytest.fixture(scope="session")
def yf():
    import yuezu_fps.yuezu_fps_module as m
    return m


@pytest.fixture(scope="session")
def capi():
    from ns_fps_amd.capi import LIB_PATH
    return ctypes.CDLL(LIB_PATH)


class GoldenCase:
    def __init__(self, name, points, n_samples, rng, blocks, expected):
        self.name = name
        self.points = points
        self.n_samples = n_samples
        self.range = rng          # 9-tuple, or None for compute_bbox
        self.blocks = blocks      # block counts for compute_bbox
        self.expected = expected


def load_golden_cases():
    z = np.load(os.path.join(GOLDEN, "cases.npz"), allow_pickle=False)
    names = sorted({k.split("__")[0] for k in z.files if "__" in k})
    cases = []
    for n in names:
        meta = z[f"{n}__meta"]
        pts = z[f"P{int(z[f'{n}__pid'][0])}"]
        m = int(meta[0])
        if int(meta[1]) == 1:
            rng, blocks = None, tuple(int(b) for b in meta[2:5])
        else:
            r = z[f"{n}__range"]
            rng = tuple(float(v) for v in r[:6]) + tuple(int(v) for v in r[6:9])
            blocks = rng[6:9]
        cases.append(GoldenCase(n, pts, m, rng, blocks, z[f"{n}__expected"]))
    return cases


def load_golden_configs():
    with open(os.path.join(GOLDEN, "configs.json")) as f:
        return json.load(f)


GOLDEN_CASES = load_golden_cases()
GOLDEN_CONFIGS = load_golden_configs()


def sha256_i32(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(np.asarray(a, dtype=np.int32)).tobytes()).hexdigest()


def sha256_f32(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()
