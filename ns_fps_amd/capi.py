"""ctypes binding of the C ABI in include/nsfps.h (libnsfps.so).

Mirrors the header one to one; the pybind11 module yuezu_fps_module is the
drop-in Python surface, this binding exists for callers that need the raw
entry points (device-resident input, statistics, loop profile).  A minimal
HIP helper (hipMalloc / hipMemcpy / hipFree from libamdhip64) provides device
buffers for nsfps_fps_device without any other framework.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# NSFPS_LIB names another build of the library (the sanitized one, say)
LIB_PATH = os.environ.get("NSFPS_LIB") or os.path.join(HERE, "libnsfps.so")

NSFPS_OK, NSFPS_EINVAL, NSFPS_EDEVICE, NSFPS_ENOMEM, NSFPS_EUNSUPPORTED = range(5)


class Range(ctypes.Structure):
    _fields_ = [("min_x", ctypes.c_float), ("max_x", ctypes.c_float),
                ("min_y", ctypes.c_float), ("max_y", ctypes.c_float),
                ("min_z", ctypes.c_float), ("max_z", ctypes.c_float),
                ("x_blocks", ctypes.c_uint32), ("y_blocks", ctypes.c_uint32),
                ("z_blocks", ctypes.c_uint32)]

    @classmethod
    def of(cls, rng):
        if isinstance(rng, cls):  # already converted (a caller's loop converts once)
            return rng
        return cls(*[float(v) for v in rng[:6]], *[int(v) for v in rng[6:9]])


class Stats(ctypes.Structure):
    _fields_ = [("build_ms", ctypes.c_double), ("sample_ms", ctypes.c_double),
                ("wide_ms", ctypes.c_double), ("late_ms", ctypes.c_double),
                ("device_ms", ctypes.c_double),
                ("e2e_ms", ctypes.c_double), ("n_points", ctypes.c_uint64),
                ("n_clouds", ctypes.c_uint64), ("n_leaves", ctypes.c_uint64),
                ("wide_iters", ctypes.c_uint64), ("samples", ctypes.c_uint64),
                ("padded", ctypes.c_uint32), ("lds_bytes", ctypes.c_uint32),
                ("rounds", ctypes.c_uint64), ("engine", ctypes.c_uint32),
                ("update_split", ctypes.c_uint32),
                ("mixed", ctypes.c_uint32), ("hot_set", ctypes.c_uint32)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class NsfpsError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"nsfps status {status}: {msg}")
        self.status = status


_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64


class Lib:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (python -m ns_fps_amd.build)")
        self.lib = ctypes.CDLL(path)
        self.lib.nsfps_last_error.restype = ctypes.c_char_p
        self.lib.nsfps_version.restype = ctypes.c_char_p

    def _check(self, rc):
        if rc != NSFPS_OK:
            raise NsfpsError(rc, self.lib.nsfps_last_error().decode())

    def device_count(self):
        return self.lib.nsfps_device_count()

    def init_device(self):
        """nsfps_init_device: the current device's one-time set-up, ahead of
        its first call."""
        self._check(self.lib.nsfps_init_device())

    def fps(self, points, n_samples, rng=None):
        p = np.ascontiguousarray(points, dtype=np.float32)
        out = np.zeros(max(int(n_samples), 1), np.int32)
        n = _u64()
        r = ctypes.byref(Range.of(rng)) if rng is not None else None
        self._check(self.lib.nsfps_fps(p.ctypes.data_as(_vp), _u64(len(p)), _u64(int(n_samples)),
                                       r, out.ctypes.data_as(_vp), ctypes.byref(n)))
        return out[:n.value].copy()

    def release_workspace(self):
        """Frees the cached device workspace and the pinned input stage."""
        self.lib.nsfps_release_workspace.restype = None
        self.lib.nsfps_release_workspace()

    def fps_bbox(self, points, n_samples, blocks=(16, 16, 16)):
        p = np.ascontiguousarray(points, dtype=np.float32)
        out = np.zeros(max(int(n_samples), 1), np.int32)
        n = _u64()
        self._check(self.lib.nsfps_fps_bbox(p.ctypes.data_as(_vp), _u64(len(p)),
                                            _u64(int(n_samples)), *[ctypes.c_uint32(b) for b in blocks],
                                            out.ctypes.data_as(_vp), ctypes.byref(n)))
        return out[:n.value].copy()

    def fps_batched(self, clouds, n_samples, ranges=None, blocks=(16, 16, 16)):
        P = np.ascontiguousarray(clouds, dtype=np.float32)
        B, n = P.shape[0], P.shape[1]
        out = np.zeros((B, max(int(n_samples), 1)), np.int32)
        lens = np.zeros(B, np.uint64)
        rs = None
        if ranges is not None:
            arr = (Range * B)(*[Range.of(r) for r in ranges])
            rs = arr
        b3 = (ctypes.c_uint32 * 3)(*blocks)
        self._check(self.lib.nsfps_fps_batched(P.ctypes.data_as(_vp), _u64(B), _u64(n),
                                               _u64(int(n_samples)), rs, b3,
                                               out.ctypes.data_as(_vp), lens.ctypes.data_as(_vp)))
        return [out[b, :int(lens[b])].copy() for b in range(B)]

    def fps_batched_device(self, d_xyz, batch, n, n_samples, d_out, ranges=None,
                           blocks=(16, 16, 16), stream=None):
        """nsfps_fps_batched_device: batch clouds of n points at d_xyz (device),
        samples into d_out (device, batch x n_samples int32).  Returns the
        per-cloud sample counts."""
        lens = np.zeros(batch, np.uint64)
        rs = None
        if ranges is not None:
            rs = (Range * batch)(*[Range.of(r) for r in ranges])
        b3 = (ctypes.c_uint32 * 3)(*blocks)
        self._check(self.lib.nsfps_fps_batched_device(_vp(d_xyz), _u64(batch), _u64(n),
                                                      _u64(int(n_samples)), rs, b3, _vp(d_out),
                                                      lens.ctypes.data_as(_vp), _vp(stream)))
        return [int(v) for v in lens]

    def bbox_device(self, d_xyz, n, blocks=(16, 16, 16), stream=None):
        """nsfps_bbox_device: compute_bbox of device-resident points, found on
        the device.  Returns (range tuple, nsfps_range_info bytes)."""
        r = Range()
        info = (ctypes.c_char * 256)()
        self._check(self.lib.nsfps_bbox_device(_vp(d_xyz), _u64(n),
                                               *[ctypes.c_uint32(b) for b in blocks],
                                               ctypes.byref(r), info, _vp(stream)))
        return ((r.min_x, r.max_x, r.min_y, r.max_y, r.min_z, r.max_z,
                 r.x_blocks, r.y_blocks, r.z_blocks), bytes(info))

    def fps_device(self, d_xyz, n, n_samples, rng, d_out, stream=None):
        n_out = _u64()
        self._check(self.lib.nsfps_fps_device(_vp(d_xyz), _u64(n), _u64(int(n_samples)),
                                              ctypes.byref(Range.of(rng)), _vp(d_out),
                                              ctypes.byref(n_out), _vp(stream)))
        return n_out.value

    def fps_device_noalloc(self, d_xyz, n, n_samples, rng, d_out, stream=None):
        """nsfps_fps_device_noalloc: nsfps_fps_device with its workspace in the
        library's static device array (no device allocation)."""
        n_out = _u64()
        self._check(self.lib.nsfps_fps_device_noalloc(_vp(d_xyz), _u64(n), _u64(int(n_samples)),
                                                      ctypes.byref(Range.of(rng)), _vp(d_out),
                                                      ctypes.byref(n_out), _vp(stream)))
        return n_out.value

    def noalloc_scratch_bytes(self):
        self.lib.nsfps_noalloc_scratch_bytes.restype = ctypes.c_uint64
        return int(self.lib.nsfps_noalloc_scratch_bytes())

    def plan_create(self, xyz, n, rng, on_device=False):
        """nsfps_plan_create: xyz is a device pointer (int) when on_device,
        else a host (N, 3) float32 array.  Returns the plan handle."""
        plan = _vp()
        if on_device:
            ptr = _vp(xyz)
        else:
            arr = np.ascontiguousarray(xyz, dtype=np.float32)
            n = len(arr)
            ptr = arr.ctypes.data_as(_vp)
        self._check(self.lib.nsfps_plan_create(ptr, _u64(n), ctypes.byref(Range.of(rng)),
                                               ctypes.c_int(1 if on_device else 0),
                                               ctypes.byref(plan)))
        return plan.value

    def plan_sample(self, plan, n_samples, d_out, stream=None):
        n_out = _u64()
        self._check(self.lib.nsfps_plan_sample(_vp(plan), _u64(int(n_samples)), _vp(d_out),
                                               ctypes.byref(n_out), _vp(stream)))
        return n_out.value

    def plan_destroy(self, plan):
        self.lib.nsfps_plan_destroy.restype = None
        self.lib.nsfps_plan_destroy(_vp(plan))

    def gather_points(self, points, idx):
        p = np.ascontiguousarray(points, dtype=np.float32)
        ix = np.ascontiguousarray(idx, dtype=np.int32).ravel()
        out = np.zeros((len(ix), 3), np.float32)
        self._check(self.lib.nsfps_gather_points(p.ctypes.data_as(_vp), _u64(len(p)),
                                                 ix.ctypes.data_as(_vp), _u64(len(ix)),
                                                 out.ctypes.data_as(_vp)))
        return out

    def ball_query(self, points, centers, radius, nsample):
        p = np.ascontiguousarray(points, dtype=np.float32)
        c = np.ascontiguousarray(centers, dtype=np.float32)
        out = np.zeros((len(c), int(nsample)), np.int32)
        self._check(self.lib.nsfps_ball_query(p.ctypes.data_as(_vp), _u64(len(p)),
                                              c.ctypes.data_as(_vp), _u64(len(c)),
                                              ctypes.c_float(radius), ctypes.c_uint32(int(nsample)),
                                              out.ctypes.data_as(_vp)))
        return out

    def gather_points_device(self, d_xyz, n, d_idx, m, d_out, stream=None):
        self._check(self.lib.nsfps_gather_points_device(_vp(d_xyz), _u64(n), _vp(d_idx), _u64(m),
                                                        _vp(d_out), _vp(stream)))

    def ball_query_device(self, d_xyz, n, d_centers, m, radius, nsample, d_out, stream=None):
        self._check(self.lib.nsfps_ball_query_device(_vp(d_xyz), _u64(n), _vp(d_centers), _u64(m),
                                                     ctypes.c_float(radius),
                                                     ctypes.c_uint32(int(nsample)), _vp(d_out),
                                                     _vp(stream)))

    def stats(self):
        return self.stats_raw().as_dict()

    def stats_raw(self):
        """The last call's statistics as the C struct (as_dict() converts)."""
        s = Stats()
        self._check(self.lib.nsfps_get_stats(ctypes.byref(s)))
        return s

    def loop_profile(self):
        w = (ctypes.c_uint64 * 64)()
        self._check(self.lib.nsfps_get_loop_profile(w, ctypes.c_uint32(64)))
        return list(w)


class Hip:
    """Just enough of the HIP runtime for device buffers."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so")

    def _ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def malloc(self, nbytes):
        p = _vp()
        self._ck(self.rt.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)), "hipMalloc")
        return p.value

    def free(self, p):
        self._ck(self.rt.hipFree(_vp(p)), "hipFree")

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        d = self.malloc(a.nbytes)
        self._ck(self.rt.hipMemcpy(_vp(d), a.ctypes.data_as(_vp), ctypes.c_size_t(a.nbytes), self.H2D),
                 "hipMemcpy")
        return d

    def download(self, d, count, dtype):
        out = np.zeros(count, dtype)
        if count:
            self._ck(self.rt.hipMemcpy(out.ctypes.data_as(_vp), _vp(d), ctypes.c_size_t(out.nbytes),
                                       self.D2H), "hipMemcpy")
        return out

    def memcpy_d2d(self, dst, src, nbytes):
        self._ck(self.rt.hipMemcpy(_vp(dst), _vp(src), ctypes.c_size_t(nbytes), self.D2D),
                 "hipMemcpy")

    def synchronize(self):
        self._ck(self.rt.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream_create(self):
        s = _vp()
        self._ck(self.rt.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_destroy(self, s):
        self._ck(self.rt.hipStreamDestroy(_vp(s)), "hipStreamDestroy")

    def begin_capture(self, s, mode=2):
        """hipStreamBeginCapture (mode 2: hipStreamCaptureModeRelaxed)."""
        self._ck(self.rt.hipStreamBeginCapture(_vp(s), ctypes.c_int(mode)), "hipStreamBeginCapture")

    def end_capture(self, s):
        """hipStreamEndCapture; the graph is destroyed at once (nothing here
        launches one).  Returns the status of the end."""
        g = _vp()
        rc = self.rt.hipStreamEndCapture(_vp(s), ctypes.byref(g))
        if g.value:
            self.rt.hipGraphDestroy(g)
        return rc
