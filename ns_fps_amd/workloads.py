"""Seeded synthetic point clouds for the FPS workloads: the five benchmark
configurations and the uniform cube on a 30^3 grid (the general bucket path).

Every generator uses the legacy ``numpy.random.RandomState`` stream (frozen by
NEP 19, so the same seed gives the same cloud on every machine), draws in
float64 and casts to float32 at the end.  Each workload is a dict::

    {"name", "clouds": [float32 (N, 3) C-contiguous], "n_samples",
     "range": (min_x, max_x, min_y, max_y, min_z, max_z, xb, yb, zb) or None,
     "blocks": (xb, yb, zb)}

``range=None`` means the reference's ``compute_bbox`` path
(yuezu_fps/yuezu_fps_pybind.cpp:74-76): exact fp32 bounds +/- 1e-6 with the
given block counts.
"""

import numpy as np

__all__ = ["WORKLOADS", "make_workload", "quickstart", "uniform_cube", "uniform_cube_30",
           "lidar_scan", "batched_shapes", "clustered"]


def quickstart(n=10000, n_samples=1000):
    """10,000 points ~ N(0,1), seed 42, [-100,100]^3 with 16^3 blocks
    (README.md:59-71; test.py:94)."""
    rs = np.random.RandomState(42)
    pts = rs.randn(n, 3).astype(np.float32)
    return {"name": "quickstart", "clouds": [np.ascontiguousarray(pts)],
            "n_samples": n_samples,
            "range": (-100.0, 100.0, -100.0, 100.0, -100.0, 100.0, 16, 16, 16),
            "blocks": (16, 16, 16)}


def uniform_cube(n=1048576, n_samples=65536):
    """1,048,576 points uniform in [-1,1]^3, seed 2, 32^3 blocks."""
    rs = np.random.RandomState(2)
    pts = rs.uniform(-1.0, 1.0, (n, 3)).astype(np.float32)
    return {"name": "uniform_cube", "clouds": [np.ascontiguousarray(pts)],
            "n_samples": n_samples,
            "range": (-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 32, 32, 32),
            "blocks": (32, 32, 32)}


def uniform_cube_30(n=1048576, n_samples=65536):
    """The uniform cube's points (seed 2) on a 30^3 grid: block counts that are
    not powers of two, so Morton codes (src/yuezu_fps.cpp:136-161) taken modulo
    the block count share buckets (src/yuezu_fps.cpp:413, 592) and the sampling
    takes the general bucket path."""
    w = uniform_cube(n, n_samples)
    w.update(name="uniform_cube_30", range=(-1.0, 1.0, -1.0, 1.0, -1.0, 1.0, 30, 30, 30),
             blocks=(30, 30, 30))
    return w


def _box_surface(rs, centre_xy, sides, ground_z, count):
    """Points on the five visible faces of an axis-aligned box resting on the
    ground (the bottom face is hidden), faces chosen with probability
    proportional to their area."""
    sx, sy, sz = sides
    # faces: +x, -x, +y, -y, top
    areas = np.array([sy * sz, sy * sz, sx * sz, sx * sz, sx * sy])
    face = rs.choice(5, size=count, p=areas / areas.sum())
    u = rs.uniform(0.0, 1.0, count)
    v = rs.uniform(0.0, 1.0, count)
    x = np.empty(count)
    y = np.empty(count)
    z = np.empty(count)
    x0, y0 = centre_xy[0] - sx / 2, centre_xy[1] - sy / 2
    for f in range(5):
        m = face == f
        if f in (0, 1):
            x[m] = x0 + (sx if f == 0 else 0.0)
            y[m] = y0 + u[m] * sy
            z[m] = ground_z + v[m] * sz
        elif f in (2, 3):
            x[m] = x0 + u[m] * sx
            y[m] = y0 + (sy if f == 2 else 0.0)
            z[m] = ground_z + v[m] * sz
        else:
            x[m] = x0 + u[m] * sx
            y[m] = y0 + v[m] * sy
            z[m] = ground_z + sz
    return np.stack([x, y, z], axis=1)


def lidar_scan(n_beams=64, per_beam=1500, n_boxes=40, per_box=600, n_samples=16384):
    """Synthetic rotating-LiDAR scan, seed 3: 64 beams (elevation U[-25,+3] deg,
    sorted) x 1,500 returns with azimuth U[0,360) deg and range
    clip(lognormal(ln 15, 0.6), 2, 80) m; a downward ray that reaches the ground
    plane z = -1.7 m first lands there with z jitter N(0, 0.03).  Plus 40 boxes
    (sides U[1,5] m, centres U[-60,60]^2 m, on the ground) with 600 surface
    points each.  Rows shuffled.  Range x,y in [-80,80], z in [-4,4] with
    32x32x8 blocks; points outside it are clamped into boundary cells."""
    rs = np.random.RandomState(3)
    ground = -1.7
    elev = np.sort(np.deg2rad(rs.uniform(-25.0, 3.0, n_beams)))
    e = np.repeat(elev, per_beam)
    az = np.deg2rad(rs.uniform(0.0, 360.0, n_beams * per_beam))
    rng = np.clip(rs.lognormal(np.log(15.0), 0.6, n_beams * per_beam), 2.0, 80.0)
    jitter = rs.normal(0.0, 0.03, n_beams * per_beam)
    with np.errstate(divide="ignore"):
        t_ground = np.where(e < 0, ground / np.sin(e), np.inf)
    hit = t_ground < rng
    t = np.where(hit, t_ground, rng)
    x = t * np.cos(e) * np.cos(az)
    y = t * np.cos(e) * np.sin(az)
    z = np.where(hit, ground + jitter, t * np.sin(e))
    scan = np.stack([x, y, z], axis=1)
    boxes = []
    for _ in range(n_boxes):
        sides = rs.uniform(1.0, 5.0, 3)
        centre = rs.uniform(-60.0, 60.0, 2)
        boxes.append(_box_surface(rs, centre, sides, ground, per_box))
    pts = np.concatenate([scan] + boxes, axis=0)
    pts = pts[rs.permutation(len(pts))].astype(np.float32)
    return {"name": "lidar_scan", "clouds": [np.ascontiguousarray(pts)],
            "n_samples": n_samples,
            "range": (-80.0, 80.0, -80.0, 80.0, -4.0, 4.0, 32, 32, 8),
            "blocks": (32, 32, 8)}


def _shape_cloud(seed, n):
    """Half uniform in the unit ball, half on the unit sphere with N(0,0.01)
    jitter; 1% of rows overwritten with exact copies of other rows; shuffled."""
    rs = np.random.RandomState(seed)
    h = n // 2
    d = rs.normal(size=(h, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    ball = d * rs.uniform(0.0, 1.0, (h, 1)) ** (1.0 / 3.0)
    s = rs.normal(size=(n - h, 3))
    s /= np.linalg.norm(s, axis=1, keepdims=True)
    shell = s + rs.normal(0.0, 0.01, (n - h, 3))
    pts = np.concatenate([ball, shell], axis=0)
    n_dup = n // 100
    dst = rs.choice(n, n_dup, replace=False)
    src = rs.randint(0, n, n_dup)
    pts[dst] = pts[src]
    pts = pts[rs.permutation(n)].astype(np.float32)
    return np.ascontiguousarray(pts)


def batched_shapes(n_clouds=64, n=16384, n_samples=4096):
    """64 independent clouds x 16,384 points (cloud b uses seed 4000+b), 4,096
    samples per cloud, range from compute_bbox with 16^3 blocks."""
    clouds = [_shape_cloud(4000 + b, n) for b in range(n_clouds)]
    return {"name": "batched_shapes", "clouds": clouds, "n_samples": n_samples,
            "range": None, "blocks": (16, 16, 16)}


def clustered(n_clusters=256, per_cluster=32768, n_samples=524288):
    """8,388,608 points from 256 axis-aligned Gaussian clusters, seed 5:
    centres U[-500,500]^3, per-axis sigma = exp(U[ln 1, ln 30]); shuffled.
    Range [-600,600]^3 with 64^3 blocks."""
    rs = np.random.RandomState(5)
    centres = rs.uniform(-500.0, 500.0, (n_clusters, 3))
    sigmas = np.exp(rs.uniform(np.log(1.0), np.log(30.0), (n_clusters, 3)))
    pts = np.empty((n_clusters * per_cluster, 3))
    for c in range(n_clusters):
        pts[c * per_cluster:(c + 1) * per_cluster] = (
            centres[c] + rs.normal(size=(per_cluster, 3)) * sigmas[c])
    pts = pts[rs.permutation(len(pts))].astype(np.float32)
    return {"name": "clustered", "clouds": [np.ascontiguousarray(pts)],
            "n_samples": n_samples,
            "range": (-600.0, 600.0, -600.0, 600.0, -600.0, 600.0, 64, 64, 64),
            "blocks": (64, 64, 64)}


WORKLOADS = {
    "quickstart": quickstart,
    "uniform_cube": uniform_cube,
    "uniform_cube_30": uniform_cube_30,
    "lidar_scan": lidar_scan,
    "batched_shapes": batched_shapes,
    "clustered": clustered,
}


def make_workload(name, **kw):
    return WORKLOADS[name](**kw)
