"""KITTI / SemanticKITTI point-cloud files and the FPS runs the reference
makes on them, over the HIP path of ``yuezu_fps_module``.

The reference's real-data workload is a Velodyne scan stored as float32
records of ``stride`` floats per point (x, y, z, intensity for KITTI; a few
files hold x, y, z only).  Two drivers use it:

* semantickitti_example.py:6-37 -- ``load_kitti_point_cloud`` keeps x, y, z
  of every record, and ``sample_kitti_point_cloud`` samples with a range
  spanning the exact bounds and 128 x 128 x 2 blocks;
* eval/src_cpu/compare_cpu_test_kitti.cpp:69-130, 195-240 -- reads the file
  (stride 4 or 3), drops points with z < -5, and samples with the bounds
  widened by 1e-6 in float32 and 128 x 128 x 2 blocks.  Its samples are the
  file's record numbers (Point3D.original_index survives the filter).

Both are mirrored here; every sample comes from the GPU path (no CPU
fallback).
"""

import os
import warnings

import numpy as np

import yuezu_fps.yuezu_fps_module as yf

KITTI_BLOCKS = (128, 128, 2)
KITTI_Z_MIN = -5.0
KITTI_EPS = 1e-6


def read_bin_pointcloud(path, stride=4):
    """x, y, z (float32, N x 3, C order) of a binary point file with
    ``stride`` float32 values per point (eval/src_cpu/compare_cpu_test_kitti.cpp:69-130).

    A file whose size is not a whole number of points is read up to its last
    whole point, with a warning, as the reference does; an empty file raises
    ValueError and a missing one OSError."""
    if stride not in (3, 4):
        raise ValueError("stride must be 3 or 4")
    size = os.path.getsize(path)
    if size == 0:
        raise ValueError(f"empty point file: {path}")
    nf = size // 4
    if nf % stride:
        warnings.warn(f"{path}: {nf} floats is not a multiple of stride {stride}; "
                      "the trailing partial point is ignored")
    n = nf // stride
    raw = np.fromfile(path, dtype=np.float32, count=n * stride)
    return np.ascontiguousarray(raw.reshape(n, stride)[:, :3])


def load_kitti_point_cloud(bin_path):
    """semantickitti_example.py:6-13: x, y, z of a stride-4 KITTI scan."""
    return read_bin_pointcloud(bin_path, 4)


def keep_z_at_least(points, z_min=KITTI_Z_MIN):
    """Points with z >= z_min, in file order, and their record numbers
    (eval/src_cpu/compare_cpu_test_kitti.cpp:202-215)."""
    pts = np.ascontiguousarray(points, dtype=np.float32).reshape(-1, 3)
    rows = np.flatnonzero(pts[:, 2] >= np.float32(z_min))
    return np.ascontiguousarray(pts[rows]), rows


def bounds_tuple(points, blocks=KITTI_BLOCKS, eps=KITTI_EPS):
    """(min_x, max_x, min_y, max_y, min_z, max_z, x_blocks, y_blocks, z_blocks):
    the exact float32 bounds, each widened by ``eps`` in float32 arithmetic
    (eval/src_cpu/compare_cpu_test_kitti.cpp:226-240; eps = 0 gives
    semantickitti_example.py:20-31)."""
    pts = np.asarray(points, dtype=np.float32).reshape(-1, 3)
    if len(pts) == 0:
        raise ValueError("no points to bound")
    lo = pts.min(axis=0) - np.float32(eps)
    hi = pts.max(axis=0) + np.float32(eps)
    return (float(lo[0]), float(hi[0]), float(lo[1]), float(hi[1]), float(lo[2]), float(hi[2]),
            *(int(b) for b in blocks))


def bounds_range(points, blocks=KITTI_BLOCKS, eps=KITTI_EPS):
    """``SpaceRange`` of :func:`bounds_tuple`."""
    return yf.make_range(*bounds_tuple(points, blocks, eps))


def sample_kitti_point_cloud(points, n_samples=1024):
    """semantickitti_example.py:15-37: FPS over the exact bounds with
    128 x 128 x 2 blocks; int32 positions in ``points``."""
    return yf.fps(points, n_samples, bounds_range(points, eps=0.0))


def fps_kitti_file(path, n_samples, stride=4, z_min=KITTI_Z_MIN, blocks=KITTI_BLOCKS,
                   eps=KITTI_EPS):
    """The sampling run of eval/src_cpu/compare_cpu_test_kitti.cpp: read,
    keep z >= z_min, range over the bounds widened by eps, FPS.  Returns the
    samples as the file's record numbers (int64) and the number of points
    kept."""
    pts, rows = keep_z_at_least(read_bin_pointcloud(path, stride), z_min)
    if len(pts) == 0:
        raise ValueError(f"no points with z >= {z_min} in {path}")
    idx = yf.fps(pts, n_samples, bounds_range(pts, blocks, eps))
    return rows[idx], len(pts)
