"""Host-side checks that need no GPU: the C ABI library loads and exports
every declared entry point, range derivation matches the oracle and the
reference, the Python module mirrors the reference surface
(yuezu_fps/yuezu_fps_pybind.cpp:103-150) and its error behaviour, and compute
calls fail loudly without a device (no CPU fallback)."""

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT


class Range(ctypes.Structure):
    _fields_ = [("min_x", ctypes.c_float), ("max_x", ctypes.c_float),
                ("min_y", ctypes.c_float), ("max_y", ctypes.c_float),
                ("min_z", ctypes.c_float), ("max_z", ctypes.c_float),
                ("x_blocks", ctypes.c_uint32), ("y_blocks", ctypes.c_uint32),
                ("z_blocks", ctypes.c_uint32)]


class RangeInfo(ctypes.Structure):
    _fields_ = [("inv_bs", ctypes.c_float * 3), ("block_size", ctypes.c_float * 3),
                ("bits", ctypes.c_uint32 * 3), ("total_bits", ctypes.c_uint32),
                ("total_blocks", ctypes.c_uint64), ("cube_thr", (ctypes.c_float * 8) * 3)]


def declared_symbols():
    with open(os.path.join(ROOT, "include", "nsfps.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(nsfps_[a-z_]+)\s*\(", text)))


def has_gpu(yf):
    return yf.device_count() > 0


def test_capi_exports_every_declared_symbol(capi):
    syms = declared_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(capi, s), s


def test_capi_range_derive_matches_oracle(capi, oracle):
    for rng in [(-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 32, 32, 32),
                (-80.0, 80.0, -80.0, 80.0, -4.0, 4.0, 32, 32, 8),
                (-5.0, 7.0, 0.0, 1.0, -2.0, 2.0, 10, 3, 1)]:
        r = Range(*rng)
        info = RangeInfo()
        luts = (ctypes.c_uint32 * 4096)()
        assert capi.nsfps_range_derive(ctypes.byref(r), ctypes.byref(info), luts,
                                       ctypes.c_uint64(4096)) == 0
        o = oracle.range(rng)
        assert list(info.bits) == o["bits"]
        assert np.array(list(info.inv_bs), np.float32).tobytes() == o["inv_bs"].tobytes()
        assert np.array(list(info.block_size), np.float32).tobytes() == o["block_size"].tobytes()
        off = 0
        for a in range(3):
            n = 1 << o["bits"][a]
            assert list(luts[off:off + n]) == list(o["luts"][a])
            off += n
        assert info.total_blocks == rng[6] * rng[7] * rng[8]


def numpy_half_width(D, bs, blocks):
    """get_morton_codes_in_range's half-width (src/yuezu_fps.cpp:564-570) in
    NumPy float32: ceil(sqrtf(D) / block_size), clipped to blocks - 1."""
    D = np.asarray(D, np.float32)
    f = np.ceil(np.sqrt(D) / np.float32(bs)).astype(np.float64)
    return np.minimum(f, blocks - 1).astype(np.int64)


@pytest.mark.parametrize("rng", [(-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 32, 32, 32),
                                 (-80.0, 80.0, -80.0, 80.0, -4.0, 4.0, 32, 32, 8),
                                 (-100.0, 100.0, -100.0, 100.0, -100.0, 100.0, 16, 16, 16),
                                 (-600.0, 600.0, -600.0, 600.0, -600.0, 600.0, 64, 64, 64),
                                 (-5.0, 7.0, 0.0, 1.0, -2.0, 2.0, 10, 3, 1),
                                 (0.0, 1e-3, 0.0, 3.0, 0.0, 7.0, 1024, 5, 2)])
def test_cube_thresholds_match_the_reference_half_width(capi, rng):
    """The range's cube thresholds: half-width k + 1 starts exactly at
    cube_thr[k] (the float below gives less), and below the last threshold
    the half-width of any D is the number of thresholds <= D -- checked
    against the reference's arithmetic restated in NumPy float32 on
    thresholds, their neighbours and random distances over 40 binades."""
    info = RangeInfo()
    assert capi.nsfps_range_derive(ctypes.byref(Range(*rng)), ctypes.byref(info), None,
                                   ctypes.c_uint64(0)) == 0
    rs = np.random.RandomState(5)
    for a in range(3):
        b = rng[6 + a]
        bs = np.float32(info.block_size[a])
        thr = np.array(list(info.cube_thr[a]), np.float32)
        for k, t in enumerate(thr):
            if k + 1 > b - 1:
                assert np.isinf(t)
                continue
            assert np.isfinite(t) and numpy_half_width(t, bs, b) >= k + 1
            below = np.nextafter(t, np.float32(0)) if t > 0 else None
            if below is not None:
                assert numpy_half_width(below, bs, b) < k + 1
        D = np.concatenate([thr[np.isfinite(thr)],
                            np.nextafter(thr[np.isfinite(thr)], np.float32(0)),
                            (np.float32(bs) ** 2 * np.float32(10.0) **
                             rs.uniform(-6, 3, 20000)).astype(np.float32),
                            np.array([0.0, 1e-45, 1e-38], np.float32)])
        h = numpy_half_width(D, bs, b)
        count = (D[:, None] >= thr[None, :]).sum(1)
        low = D < thr[-1] if np.isfinite(thr[-1]) else np.ones(len(D), bool)
        assert np.array_equal(count[low], h[low])
        assert np.all(h[~low] >= 8)


def _capi_bbox(capi, pts):
    out = Range()
    assert capi.nsfps_bbox(pts.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(len(pts)), 16, 8, 4,
                           ctypes.byref(out)) == 0
    assert (out.x_blocks, out.y_blocks, out.z_blocks) == (16, 8, 4)
    return np.array([out.min_x, out.max_x, out.min_y, out.max_y, out.min_z, out.max_z], np.float32)


# sizes around the 8-point lane step, the 65,536-point pieces and the
# threaded split (from 262,144 points)
@pytest.mark.parametrize("n", [1, 7, 8, 9, 777, 65536, 65537, 300001, 1 << 20])
def test_capi_bbox_matches_oracle(capi, oracle, n):
    pts = np.random.RandomState(n).randn(n, 3).astype(np.float32) * 5
    got = _capi_bbox(capi, pts)
    assert got.tobytes() == oracle.bbox(pts).tobytes()
    # the exact float32 extremes, widened by 1e-6 in float32
    e = np.float32(1e-6)
    want = np.array([pts[:, 0].min() - e, pts[:, 0].max() + e, pts[:, 1].min() - e,
                     pts[:, 1].max() + e, pts[:, 2].min() - e, pts[:, 2].max() + e], np.float32)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("n", [9, 300001])
def test_capi_bbox_nan_rules_match_the_running_pass(capi, oracle, n):
    """A NaN at point 0 poisons its axis; a later NaN is skipped (the
    reference's running compare-select from point 0)."""
    base = np.random.RandomState(5).randn(n, 3).astype(np.float32)
    for where in (0, n // 2, n - 1):
        pts = base.copy()
        pts[where, 1] = np.nan
        got = _capi_bbox(capi, pts)
        want = oracle.bbox(pts)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
        assert np.isnan(got[2]) == (where == 0)


def test_capi_bbox_in_a_child_forked_after_the_worker_threads_started(capi, oracle):
    """Large bounds run on worker threads that the library starts once and
    keeps.  A process forked after they started (multiprocessing's default on
    Linux) has none of them; its calls must still return, with the same
    bounds."""
    import signal
    import time
    pts = np.random.RandomState(11).randn(1 << 20, 3).astype(np.float32)
    want = _capi_bbox(capi, pts)  # starts the workers in this process
    assert want.tobytes() == oracle.bbox(pts).tobytes()
    pid = os.fork()
    if pid == 0:  # the child: exit status 0 only for the same bounds, twice
        code = 1
        try:
            ok = all(_capi_bbox(capi, pts).tobytes() == want.tobytes() for _ in range(2))
            code = 0 if ok else 1
        finally:
            os._exit(code)
    deadline = time.monotonic() + 60
    while True:
        done, status = os.waitpid(pid, os.WNOHANG)
        if done:
            break
        if time.monotonic() > deadline:
            os.kill(pid, signal.SIGKILL)
            os.waitpid(pid, 0)
            pytest.fail("the forked child's bounds call did not return")
        time.sleep(0.05)
    assert os.WIFEXITED(status) and os.WEXITSTATUS(status) == 0
    # and the parent's workers still serve it
    assert _capi_bbox(capi, pts).tobytes() == want.tobytes()


def test_capi_rejects_bad_arguments(capi):
    capi.nsfps_last_error.restype = ctypes.c_char_p
    pts = np.zeros((10, 3), np.float32)
    out = np.zeros(10, np.int32)
    n = ctypes.c_uint64()
    bad = Range(1.0, 1.0, 0.0, 1.0, 0.0, 1.0, 4, 4, 4)  # max == min
    rc = capi.nsfps_fps(pts.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(10), ctypes.c_uint64(5),
                        ctypes.byref(bad), out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n))
    assert rc == 1 and b"max > min" in capi.nsfps_last_error()
    zero = Range(0.0, 1.0, 0.0, 1.0, 0.0, 1.0, 0, 4, 4)
    rc = capi.nsfps_fps(pts.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(10), ctypes.c_uint64(5),
                        ctypes.byref(zero), out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n))
    assert rc == 1
    rc = capi.nsfps_fps(None, ctypes.c_uint64(10), ctypes.c_uint64(5), None,
                        out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(n))
    assert rc == 1


@pytest.mark.parametrize("blocks", [(1025, 4, 4), (4, 2048, 4), (4, 4, 100000)])
def test_more_than_1024_blocks_per_axis_is_unsupported(capi, yf, blocks):
    """The reference accepts any block count (src/yuezu_fps.cpp:45-50, 136-161);
    this build packs a cell's coordinates 10 bits per axis and refuses larger
    grids with NSFPS_EUNSUPPORTED and a message naming the limit, before any
    device work (so the check runs without a GPU)."""
    capi.nsfps_last_error.restype = ctypes.c_char_p
    pts = np.random.RandomState(1).rand(100, 3).astype(np.float32)
    out = np.zeros(100, np.int32)
    n = ctypes.c_uint64()
    r = Range(0.0, 1.0, 0.0, 1.0, 0.0, 1.0, *blocks)
    rc = capi.nsfps_fps(pts.ctypes.data_as(ctypes.c_void_p), ctypes.c_uint64(100),
                        ctypes.c_uint64(10), ctypes.byref(r), out.ctypes.data_as(ctypes.c_void_p),
                        ctypes.byref(n))
    assert rc == 4  # NSFPS_EUNSUPPORTED
    assert b"above 1024 per axis" in capi.nsfps_last_error()
    # the module maps it to RuntimeError (not the input-error class)
    with pytest.raises(RuntimeError, match="above 1024 per axis") as ei:
        yf.fps(pts, 10, yf.make_range(0, 1, 0, 1, 0, 1, *blocks))
    assert not isinstance(ei.value, ValueError)
    # 1024 is still accepted (the trivial identity path needs no device)
    assert list(yf.fps(pts[:3], 5, yf.make_range(0, 1, 0, 1, 0, 1, 1024, 1, 1))) == [0, 1, 2]


def test_module_surface_mirrors_reference(yf):
    for name in ["SpaceRange", "make_range", "make_uniform_range", "fps", "fps_with_bbox",
                 "DEFAULT_X_BLOCKS", "DEFAULT_Y_BLOCKS", "DEFAULT_Z_BLOCKS",
                 "MORTON_BLOCK_SIZE", "CACHE_BLOCK_SIZE"]:
        assert hasattr(yf, name), name
    assert (yf.DEFAULT_X_BLOCKS, yf.MORTON_BLOCK_SIZE, yf.CACHE_BLOCK_SIZE) == (16, 16, 16)
    r = yf.make_range(-150, 150, -150, 150, -150, 150, 16, 16, 16)   # example.py:115
    assert (r.min_x, r.max_x, r.x_blocks) == (-150.0, 150.0, 16)
    assert r.total_bits() == 12 and r.total_blocks() == 4096
    assert r.block_size_x() == np.float32(300.0 / 16)
    u = yf.make_uniform_range(-1, 1, -2, 2, -3, 3, 8)
    assert (u.x_blocks, u.y_blocks, u.z_blocks) == (8, 8, 8)
    assert (u.x_bits(), u.y_bits(), u.z_bits()) == (3, 3, 3)
    s = yf.SpaceRange()
    s.min_x, s.max_x, s.min_y, s.max_y, s.min_z, s.max_z = -1, 1, -1, 1, -1, 1
    s.x_blocks, s.y_blocks, s.z_blocks = 32, 16, 8
    assert (s.x_bits(), s.y_bits(), s.z_bits(), s.total_bits()) == (5, 4, 3, 12)
    # derived values follow field edits (the reference keeps stale ones)
    s.x_blocks = 64
    assert s.x_bits() == 6 and s.inv_bs_x == np.float32(32.0)


def test_module_trivial_guards_need_no_device(yf):
    pts = np.random.RandomState(0).randn(5, 3).astype(np.float32)
    r = yf.make_range(-4, 4, -4, 4, -4, 4, 4, 4, 4)
    assert list(yf.fps(pts, 5, r)) == [0, 1, 2, 3, 4]           # n >= N: identity
    assert list(yf.fps(pts, 9, r)) == [0, 1, 2, 3, 4]
    assert list(yf.fps(pts, 0, r)) == []
    assert list(yf.fps(pts, 1, r)) == [0]
    assert list(yf.fps(np.zeros((0, 3), np.float32), 4, r)) == []
    assert yf.fps(pts, 5, r).dtype == np.int32
    # keyword spellings: the binding's sample_count and the README's n_samples
    assert list(yf.fps(pts, sample_count=7, range=r)) == [0, 1, 2, 3, 4]
    assert list(yf.fps(pts, n_samples=7, range=r)) == [0, 1, 2, 3, 4]
    assert list(yf.fps_with_bbox(pts, 6)) == [0, 1, 2, 3, 4]


def test_module_error_behaviour(yf):
    pts = np.random.RandomState(0).randn(50, 3).astype(np.float32)
    with pytest.raises(RuntimeError, match="shape"):          # reference: RuntimeError
        yf.fps(np.zeros((10, 2), np.float32), 3)
    with pytest.raises(ValueError):
        yf.fps(np.zeros((10, 2), np.float32), 3)
    with pytest.raises(yf.InputError):
        yf.fps(pts, 10, {"min_x": 0, "max_x": 1})              # incomplete dict
    with pytest.raises(yf.InputError):
        yf.fps(pts, 10, yf.make_range(1, 1, 0, 1, 0, 1, 4, 4, 4))
    with pytest.raises(yf.InputError):
        yf.fps(pts, 10, yf.make_range(0, 1, 0, 1, 0, 1, 0, 4, 4))
    with pytest.raises(yf.InputError):
        yf.fps(pts, 10, 5)


def test_module_converts_strided_and_float64_input(yf):
    """The reference reads a strided view such as pc[:, :3] as if it were
    contiguous (yuezu_fps/yuezu_fps_pybind.cpp:17-33); here it is converted.
    Checked through the trivial identity path so it runs without a device."""
    pc = np.random.RandomState(0).randn(6, 4).astype(np.float32)
    r = yf.make_range(-4, 4, -4, 4, -4, 4, 4, 4, 4)
    assert list(yf.fps(pc[:, :3], 10, r)) == list(range(6))
    assert list(yf.fps(pc[:, :3].astype(np.float64), 10, r)) == list(range(6))


def test_compute_fails_loudly_without_device(yf):
    if has_gpu(yf):
        pytest.skip("a GPU is present")
    pts = np.random.RandomState(0).randn(100, 3).astype(np.float32)
    with pytest.raises(RuntimeError, match="no HIP device"):
        yf.fps(pts, 10, yf.make_range(-4, 4, -4, 4, -4, 4, 8, 8, 8))
    with pytest.raises(RuntimeError, match="no HIP device"):
        yf.fps_batched(np.stack([pts, pts]), 10)


def test_dict_range_uses_default_blocks(yf):
    """A dict range takes the six bounds and optional block counts, default 16
    (yuezu_fps/yuezu_fps_pybind.cpp:48-58); via the identity path."""
    pts = np.random.RandomState(0).randn(4, 3).astype(np.float32)
    d = {"min_x": -4, "max_x": 4, "min_y": -4, "max_y": 4, "min_z": -4, "max_z": 4}
    assert list(yf.fps(pts, 4, d)) == [0, 1, 2, 3]
