"""ctypes wrapper of the CPU checkers -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg.
The product package ns_fps_amd never imports this module.

* ``Oracle``: our C restatement (oracle/nsfps_oracle.c -> liboracle.so).
* ``Reference``: the reference library compiled from its own sources by
  oracle/Makefile into oracle/_ref/ (absent where it was not built).
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libyuezu_ref.so")
REF_ASBUILT_SO = os.path.join(HERE, "_ref", "libyuezu_ref_asbuilt.so")

_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64


class Census(ctypes.Structure):
    _fields_ = [("iterations", ctypes.c_uint64), ("cand_cells", ctypes.c_uint64),
                ("cand_points", ctypes.c_uint64), ("cand_leaves", ctypes.c_uint64),
                ("first_pass_points", ctypes.c_uint64),
                ("first_pass_leaves", ctypes.c_uint64),
                ("audit_violations", ctypes.c_uint64)]

    def as_dict(self):
        return {k: int(getattr(self, k)) for k, _ in self._fields_}

    def alg_bytes(self):
        """16 B per candidate point-iteration (12 B xyz + 4 B min-distance) and
        8 B per candidate 16-point leaf, including the first full pass."""
        pts = self.cand_points + self.first_pass_points
        leaves = self.cand_leaves + self.first_pass_leaves
        return 16 * pts + 8 * leaves


def _ptr(a):
    return a.ctypes.data_as(_vp)


def _pts(points):
    p = np.ascontiguousarray(points, dtype=np.float32)
    if p.ndim != 2 or p.shape[1] != 3:
        raise ValueError("points must be (N, 3)")
    return p


def _range_args(rng, blocks):
    """rng: 9-tuple (bounds6 + blocks3) or None (compute_bbox with blocks)."""
    if rng is None:
        return None, (ctypes.c_uint32 * 3)(*blocks)
    return (ctypes.c_float * 6)(*rng[:6]), (ctypes.c_uint32 * 3)(*rng[6:9])


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        self.lib = ctypes.CDLL(path)

    def range(self, rng):
        b6, b3 = _range_args(rng, None)
        inv = (ctypes.c_float * 3)()
        bs = (ctypes.c_float * 3)()
        bits = (ctypes.c_uint32 * 3)()
        luts = np.zeros(3 * (1 << 21), np.uint32)
        n = self.lib.orc_range(b6, b3, inv, bs, bits, _ptr(luts), ctypes.c_uint32(len(luts)))
        if n < 0:
            raise ValueError("bad range")
        b = list(bits)
        x = luts[:1 << b[0]].copy()
        y = luts[1 << b[0]:(1 << b[0]) + (1 << b[1])].copy()
        z = luts[(1 << b[0]) + (1 << b[1]):n].copy()
        return {"inv_bs": np.array(list(inv), np.float32),
                "block_size": np.array(list(bs), np.float32),
                "bits": b, "luts": (x, y, z)}

    def bbox(self, points):
        p = _pts(points)
        b6 = (ctypes.c_float * 6)()
        self.lib.orc_bbox(_ptr(p), _u64(len(p)), b6)
        return np.array(list(b6), np.float32)

    def cell_code(self, points, rng):
        p = _pts(points)
        b6, b3 = _range_args(rng, None)
        cells = np.zeros((len(p), 3), np.uint32)
        codes = np.zeros(len(p), np.uint32)
        if self.lib.orc_cell_code(_ptr(p), _u64(len(p)), b6, b3, _ptr(cells), _ptr(codes)):
            raise ValueError("bad range")
        return cells, codes

    def layout(self, points, rng):
        p = _pts(points)
        b6, b3 = _range_args(rng, None)
        bucket = np.zeros(len(p), np.uint32)
        order = np.zeros(len(p), np.uint32)
        if self.lib.orc_layout(_ptr(p), _u64(len(p)), b6, b3, _ptr(bucket), _ptr(order)):
            raise ValueError("bad range")
        return bucket, order

    def fps(self, points, n_samples, rng=None, blocks=(16, 16, 16), census=False,
            audit=False):
        p = _pts(points)
        b6, b3 = _range_args(rng, blocks)
        out = np.zeros(max(int(n_samples), 1), np.int32)
        ol = ctypes.c_uint64()
        c = Census()
        rc = self.lib.orc_fps(_ptr(p), _u64(len(p)), _u64(int(n_samples)), b6, b3,
                              _ptr(out), ctypes.byref(ol), ctypes.byref(c),
                              ctypes.c_int(1 if audit else 0))
        if rc:
            raise ValueError(f"orc_fps failed ({rc})")
        res = out[:ol.value].copy()
        return (res, c) if (census or audit) else res

    def fps_trace(self, points, n_samples, rng=None, blocks=(16, 16, 16), leaves=False):
        p = _pts(points)
        b6, b3 = _range_args(rng, blocks)
        m = max(int(n_samples), 1)
        out = np.zeros(m, np.int32)
        md = np.zeros(m, np.float32)
        cp = np.zeros(m, np.uint32)
        cl = np.zeros(m, np.uint32)
        ol = ctypes.c_uint64()
        rc = self.lib.orc_fps_trace(_ptr(p), _u64(len(p)), _u64(int(n_samples)), b6, b3,
                                    _ptr(out), ctypes.byref(ol), _ptr(md), _ptr(cp), _ptr(cl))
        if rc:
            raise ValueError(f"orc_fps_trace failed ({rc})")
        k = ol.value
        if leaves:
            return out[:k].copy(), md[:k].copy(), cp[:k].copy(), cl[:k].copy()
        return out[:k].copy(), md[:k].copy(), cp[:k].copy()

    def fps_naive(self, points, n_samples, tie="index", rng=None, blocks=(16, 16, 16),
                  max_iters=0):
        p = _pts(points)
        b6, b3 = _range_args(rng, blocks)
        out = np.zeros(max(int(n_samples), 1), np.int32)
        ol = ctypes.c_uint64()
        rc = self.lib.orc_fps_naive(_ptr(p), _u64(len(p)), _u64(int(n_samples)), b6, b3,
                                    ctypes.c_int(1 if tie == "logical" else 0),
                                    _ptr(out), ctypes.byref(ol), _u64(int(max_iters)))
        if rc:
            raise ValueError(f"orc_fps_naive failed ({rc})")
        return out[:ol.value].copy()


    def fps_naive_mt(self, points, n_samples, max_iters=0, threads=0):
        """Naive FPS, ties to the lowest index, over `threads` OpenMP threads
        (0: the OpenMP default); the same indices as fps_naive(tie="index")."""
        p = _pts(points)
        out = np.zeros(max(int(n_samples), 1), np.int32)
        ol = ctypes.c_uint64()
        rc = self.lib.orc_fps_naive_mt(_ptr(p), _u64(len(p)), _u64(int(n_samples)), _ptr(out),
                                       ctypes.byref(ol), _u64(int(max_iters)),
                                       ctypes.c_int(int(threads)))
        if rc:
            raise ValueError(f"orc_fps_naive_mt failed ({rc})")
        return out[:ol.value].copy()

    def max_threads(self):
        return int(self.lib.orc_max_threads())


def gather_points(orc, points, idx):
    """orc_gather_points: (M, 3) float32; ValueError for an index outside [0, N)."""
    p = _pts(points)
    ix = np.ascontiguousarray(idx, dtype=np.int32).ravel()
    out = np.zeros((len(ix), 3), np.float32)
    if orc.lib.orc_gather_points(_ptr(p), _u64(len(p)), _ptr(ix), _u64(len(ix)), _ptr(out)):
        raise ValueError("index outside the cloud")
    return out


def ball_query(orc, points, centers, radius, nsample):
    """orc_ball_query with r2 = radius * radius in float32: (M, nsample) int32."""
    p, c = _pts(points), _pts(centers)
    r = np.float32(radius)
    out = np.zeros((len(c), int(nsample)), np.int32)
    orc.lib.orc_ball_query(_ptr(p), _u64(len(p)), _ptr(c), _u64(len(c)),
                           ctypes.c_float(float(r * r)), ctypes.c_uint32(int(nsample)), _ptr(out))
    return out


class Reference:
    """The reference library built from its own sources (oracle/_ref)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run make -C oracle ref)")
        self.path = path
        self.lib = ctypes.CDLL(path)

    def fps(self, points, n_samples, rng=None, blocks=(16, 16, 16)):
        p = _pts(points)
        out = np.zeros(max(int(n_samples), 1), np.int64)
        ol = ctypes.c_uint64()
        if rng is None:
            b3 = (ctypes.c_uint32 * 3)(*blocks)
            self.lib.ref_fps_bbox(_ptr(p), _u64(len(p)), _u64(int(n_samples)), b3,
                                  _ptr(out), ctypes.byref(ol))
        else:
            b6, b3 = _range_args(rng, None)
            self.lib.ref_fps(_ptr(p), _u64(len(p)), _u64(int(n_samples)), b6, b3,
                             _ptr(out), ctypes.byref(ol))
        return out[:ol.value].astype(np.int32)

    def range(self, rng):
        b6, b3 = _range_args(rng, None)
        inv = (ctypes.c_float * 3)()
        bs = (ctypes.c_float * 3)()
        bits = (ctypes.c_uint32 * 3)()
        luts = np.zeros(3 * (1 << 21), np.uint32)
        n = self.lib.ref_range(b6, b3, inv, bs, bits, _ptr(luts), ctypes.c_uint32(len(luts)))
        b = list(bits)
        x = luts[:1 << b[0]].copy()
        y = luts[1 << b[0]:(1 << b[0]) + (1 << b[1])].copy()
        z = luts[(1 << b[0]) + (1 << b[1]):n].copy()
        return {"inv_bs": np.array(list(inv), np.float32),
                "block_size": np.array(list(bs), np.float32),
                "bits": b, "luts": (x, y, z)}

    def cell_code(self, points, rng):
        p = _pts(points)
        b6, b3 = _range_args(rng, None)
        cells = np.zeros((len(p), 3), np.uint32)
        codes = np.zeros(len(p), np.uint32)
        self.lib.ref_cell_code(_ptr(p), _u64(len(p)), b6, b3, _ptr(cells), _ptr(codes))
        return cells, codes

    def bbox(self, points):
        p = _pts(points)
        b6 = (ctypes.c_float * 6)()
        self.lib.ref_bbox(_ptr(p), _u64(len(p)), b6)
        return np.array(list(b6), np.float32)
