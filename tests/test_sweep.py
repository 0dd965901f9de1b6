"""Seeded sweep of cloud shapes, grids and ranges: the HIP path against the
oracle (GPU), and the oracle against the reference library built from its
own sources (CPU, where oracle/_ref is built).

Shapes: uniform box, Gaussian, tight clusters, a flat plane (one axis
constant), a line, an integer lattice (many equal distances), and clouds
reaching outside the range (clamped into the boundary cells).  Grids mix
powers of two (one cell per bucket) with other block counts (cells sharing
buckets), from 1 to 64 blocks per axis.
"""

import os

import numpy as np
import pytest

from conftest import ROOT

SHAPES = ["box", "gauss", "clusters", "plane", "line", "lattice", "outside"]


def make_case(seed):
    rs = np.random.RandomState(1000 + seed)
    shape = SHAPES[seed % len(SHAPES)]
    n = int(rs.randint(200, 40000))
    if shape == "box":
        p = rs.uniform(-1, 1, (n, 3))
    elif shape == "gauss":
        p = rs.randn(n, 3) * 0.4
    elif shape == "clusters":
        c = rs.uniform(-0.8, 0.8, (int(rs.randint(2, 30)), 3))
        p = c[rs.randint(0, len(c), n)] + rs.randn(n, 3) * 0.02
    elif shape == "plane":
        p = rs.uniform(-1, 1, (n, 3))
        p[:, rs.randint(0, 3)] = 0.25
    elif shape == "line":
        t = rs.uniform(-1, 1, n)
        p = np.stack([t, 0.5 * t, -0.3 * t], 1)
    elif shape == "lattice":
        p = rs.randint(-6, 7, (n, 3)) / 6.0
    else:  # outside: a third of the points beyond the range
        p = rs.uniform(-1.5, 1.5, (n, 3))
    p = np.ascontiguousarray(p, dtype=np.float32)
    choices = [1, 2, 3, 4, 5, 7, 8, 12, 16, 20, 32, 64]
    blocks = tuple(int(rs.choice(choices)) for _ in range(3))
    if seed % 3 == 0:  # a power-of-two grid on every third case at least
        blocks = tuple(int(rs.choice([1, 2, 4, 8, 16, 32, 64])) for _ in range(3))
    m = int(rs.randint(1, n + 1)) if seed % 5 else int(rs.randint(1, min(n, 64) + 1))
    rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, *blocks)
    return shape, p, m, rng


SEEDS = list(range(42))


def _ids(seed):
    shape, p, m, rng = make_case(seed)
    return f"{seed}-{shape}-{len(p)}-{m}-{'x'.join(map(str, rng[6:]))}"


@pytest.mark.parametrize("seed", SEEDS, ids=_ids)
def test_oracle_matches_reference_on_sweep(oracle, seed):
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libyuezu_ref.so")
    if not os.path.exists(ref_so):
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    from oracle import Reference
    shape, p, m, rng = make_case(seed)
    assert np.array_equal(oracle.fps(p, m, rng), Reference(ref_so).fps(p, m, rng))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS, ids=_ids)
def test_gpu_matches_oracle_on_sweep(yf, oracle, seed):
    shape, p, m, rng = make_case(seed)
    got = yf.fps(p, m, yf.make_range(*rng))
    want = oracle.fps(p, m, rng)
    assert got.dtype == np.int32
    assert np.array_equal(got, want), f"first difference at {np.argmax(got[:len(want)] != want[:len(got)])}"


@pytest.mark.gpu
def test_gpu_round_schedule_of_one_cloud_on_others(yf, oracle):
    """A call replays the round batches of the last call of the same shape;
    clouds of one shape but different contents (and so different round
    counts) still give the oracle's samples, in either order."""
    rs = np.random.RandomState(77)
    n, m, rng = 30000, 6000, (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 32, 32, 32)
    c = rs.uniform(-0.9, 0.9, (5, 3))
    clouds = [rs.uniform(-1, 1, (n, 3)), rs.randn(n, 3) * 0.3,
              c[rs.randint(0, 5, n)] + rs.randn(n, 3) * 0.01, rs.uniform(-1, 1, (n, 3))]
    clouds = [np.ascontiguousarray(x, dtype=np.float32) for x in clouds]
    want = [oracle.fps(x, m, rng) for x in clouds]
    for order in ([0, 1, 2, 3], [2, 0, 3, 1, 1, 2]):
        for i in order:
            assert np.array_equal(yf.fps(clouds[i], m, yf.make_range(*rng)), want[i]), (order, i)


# A second sweep over other regimes: clouds a few cells wide inside a range
# many cells wide (every cube then holds every point, as in the README's
# example), shells (many near-equal distances), two far-apart clusters,
# heavy duplication (the run ends at distance 0), skewed densities, points on
# the cell boundaries of a power-of-two grid, and a dense core with far
# outliers; ranges symmetric, asymmetric, or found from the points
# (range=None, the reference's compute_bbox with the case's block counts).
SHAPES2 = ["speck", "shell", "far", "dups", "skewed", "aligned", "outliers"]


def make_case2(seed):
    rs = np.random.RandomState(5000 + seed)
    shape = SHAPES2[seed % len(SHAPES2)]
    n = int(rs.randint(100, 30000))
    if shape == "speck":
        p = rs.randn(n, 3) * float(rs.choice([0.001, 0.01, 0.05]))
    elif shape == "shell":
        v = rs.randn(n, 3)
        p = 0.8 * v / np.linalg.norm(v, axis=1, keepdims=True)
    elif shape == "far":
        p = rs.randn(n, 3) * 0.01 + np.where(rs.rand(n, 1) < 0.5, -0.9, 0.9)
    elif shape == "dups":
        base = rs.uniform(-1, 1, (int(rs.randint(1, 40)), 3))
        p = base[rs.randint(0, len(base), n)]
    elif shape == "skewed":
        p = np.sign(rs.randn(n, 3)) * rs.exponential(0.1, (n, 3))
    elif shape == "aligned":
        k = int(rs.choice([2, 4, 8, 16]))
        p = rs.randint(-k, k + 1, (n, 3)) / k
    else:  # outliers
        p = rs.randn(n, 3) * 0.05
        far = rs.randint(0, n, max(1, n // 1000))
        p[far] = rs.uniform(-1, 1, (len(far), 3))
    p = np.ascontiguousarray(p, dtype=np.float32)
    blocks = tuple(int(rs.choice([1, 2, 3, 4, 6, 8, 10, 16, 24, 32, 64])) for _ in range(3))
    if seed % 2 == 0:
        blocks = tuple(int(rs.choice([1, 2, 4, 8, 16, 32, 64])) for _ in range(3))
    r1, r2 = int(rs.randint(1, n + 1)), int(rs.randint(1, min(n, 2000) + 1))
    m = int(rs.choice([2, r1, r2, r2, n + 5]))
    if seed % 4 == 3:
        rng = None
    elif seed % 4 == 1:
        lo = rs.uniform(-1.3, -0.6, 3)
        hi = rs.uniform(0.6, 1.3, 3)
        rng = (float(lo[0]), float(hi[0]), float(lo[1]), float(hi[1]), float(lo[2]), float(hi[2]),
               *blocks)
    else:
        rng = (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, *blocks)
    return shape, p, m, rng, blocks


SEEDS2 = list(range(42))


def _ids2(seed):
    shape, p, m, rng, blocks = make_case2(seed)
    return f"{seed}-{shape}-{len(p)}-{m}-{'x'.join(map(str, blocks))}{'-bbox' if rng is None else ''}"


@pytest.mark.parametrize("seed", SEEDS2, ids=_ids2)
def test_oracle_matches_reference_on_second_sweep(oracle, seed):
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libyuezu_ref.so")
    if not os.path.exists(ref_so):
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    from oracle import Reference
    shape, p, m, rng, blocks = make_case2(seed)
    want = Reference(ref_so).fps(p, m, rng, blocks=blocks)
    assert np.array_equal(oracle.fps(p, m, rng, blocks=blocks), want)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", SEEDS2, ids=_ids2)
def test_gpu_matches_oracle_on_second_sweep(yf, oracle, seed):
    from ns_fps_amd.capi import Lib
    shape, p, m, rng, blocks = make_case2(seed)
    if rng is None:
        got = Lib().fps_bbox(p, m, blocks)
    else:
        got = yf.fps(p, m, yf.make_range(*rng))
    want = oracle.fps(p, m, rng, blocks=blocks)
    assert got.dtype == np.int32
    assert np.array_equal(got, want), (len(got), len(want), f"first difference at "
                                       f"{np.argmax(got[:len(want)] != want[:len(got)])}")


@pytest.mark.gpu
@pytest.mark.parametrize("sweep,seed", [(1, s) for s in SEEDS] + [(2, s) for s in SEEDS2],
                         ids=lambda v: str(v))
def test_gpu_matches_oracle_with_hot_sets_of_128(yf, oracle, sweep, seed, monkeypatch):
    """Both sweeps with the run kernel's 128-copy hot sets forced (the size
    otherwise taken only where the points fill many buckets; grids whose
    cells share buckets keep 64)."""
    from ns_fps_amd.capi import Lib
    monkeypatch.setenv("NSFPS_HOT", "128")
    if sweep == 1:
        shape, p, m, rng = make_case(seed)
        blocks = rng[6:9]
    else:
        shape, p, m, rng, blocks = make_case2(seed)
    if rng is None:
        got = Lib().fps_bbox(p, m, blocks)
    else:
        got = yf.fps(p, m, yf.make_range(*rng))
    want = oracle.fps(p, m, rng, blocks=blocks)
    assert np.array_equal(got, want), (len(got), len(want), f"first difference at "
                                       f"{np.argmax(got[:len(want)] != want[:len(got)])}")


@pytest.mark.gpu
@pytest.mark.parametrize("sweep,seed", [(1, s) for s in SEEDS] + [(2, s) for s in SEEDS2],
                         ids=lambda v: str(v))
def test_gpu_matches_oracle_with_the_list_box_form(yf, oracle, sweep, seed, monkeypatch):
    """Both sweeps with the run kernel forced to the form that applies a
    large-cube sample holding the list's cell box with no cell test (taken
    otherwise only for clouds in few buckets; grids whose cells share buckets
    and 128-copy hot sets keep the general form)."""
    from ns_fps_amd.capi import Lib
    monkeypatch.setenv("NSFPS_WHOLE", "1")
    if sweep == 1:
        shape, p, m, rng = make_case(seed)
        blocks = rng[6:9]
    else:
        shape, p, m, rng, blocks = make_case2(seed)
    if rng is None:
        got = Lib().fps_bbox(p, m, blocks)
    else:
        got = yf.fps(p, m, yf.make_range(*rng))
    want = oracle.fps(p, m, rng, blocks=blocks)
    assert np.array_equal(got, want), (len(got), len(want), f"first difference at "
                                       f"{np.argmax(got[:len(want)] != want[:len(got)])}")
