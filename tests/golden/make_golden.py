"""Writes the golden fixtures of the FPS path from the reference itself.

The reference library is compiled from its own sources (src/yuezu_fps.cpp)
with FMA contraction off by ``make -C oracle ref`` into oracle/_ref/ -- this
script only runs in the container that holds the reference tree.  Outputs:

* tests/golden/cases.npz -- small cases: inputs (points, sample count, range
  or the compute_bbox flag) and the reference's output indices;
* tests/golden/configs.json -- for the workloads of ns_fps_amd/workloads.py:
  SHA-256 of the generated input and of the reference's int32 output per
  cloud, output length and the first indices;
* tests/golden/census.npz -- per-iteration algorithmic bytes of the same
  workloads.

Usage: python tests/golden/make_golden.py [--skip-large] [--workloads a,b]
(--workloads regenerates those workloads' entries only and keeps the others).
"""

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import Oracle, Reference  # noqa: E402
from ns_fps_amd.workloads import make_workload  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bbox_python(points, xb, yb, zb, margin=0.01):
    """test.py:10-28 compute_bbox_python (float32 arithmetic, NumPy 2 rules)."""
    mn = points.min(axis=0)
    mx = points.max(axis=0)
    pad = (mx - mn) * margin + 1e-4
    lo = mn - pad
    hi = mx + pad
    return (float(lo[0]), float(hi[0]), float(lo[1]), float(hi[1]), float(lo[2]), float(hi[2]),
            xb, yb, zb)


def small_cases():
    """(name, points float32 (N,3), n_samples, range 9-tuple or None, blocks)."""
    cases = []
    f32 = lambda a: np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1, 3))
    # hand-made known answers
    cases.append(("tie_bucket_order", f32([(0, 0, 0), (1, 0, 0), (-1, 0, 0)]), 2,
                  (-2, 2, -2, 2, -2, 2, 4, 4, 4), None))
    cases.append(("all_duplicates", f32([(1, 1, 1)] * 5), 3, (-2, 2, -2, 2, -2, 2, 4, 4, 4), None))
    cases.append(("identity_m_eq_n", f32([(0, 0, 0), (1, 2, 3), (3, 2, 1)]), 3,
                  (-4, 4, -4, 4, -4, 4, 4, 4, 4), None))
    cases.append(("identity_m_gt_n", f32([(0, 0, 0), (1, 2, 3), (3, 2, 1)]), 7,
                  (-4, 4, -4, 4, -4, 4, 4, 4, 4), None))
    cases.append(("single_sample", f32([(0, 0, 0), (1, 2, 3), (3, 2, 1)]), 1,
                  (-4, 4, -4, 4, -4, 4, 4, 4, 4), None))
    cases.append(("zero_samples", f32([(0, 0, 0), (1, 2, 3)]), 0,
                  (-4, 4, -4, 4, -4, 4, 4, 4, 4), None))
    cases.append(("empty_cloud", f32(np.zeros((0, 3))), 5, (-4, 4, -4, 4, -4, 4, 4, 4, 4), None))
    # test.py:94-101 (seed 42, drawn in order), ranges from compute_bbox_python
    rs = np.random.RandomState(42)
    tp = [("testpy_100_10", rs.randn(100, 3).astype(np.float32), 10),
          ("testpy_1k_100", rs.randn(1000, 3).astype(np.float32), 100),
          ("testpy_10k_1k", rs.randn(10000, 3).astype(np.float32), 1000),
          ("testpy_nonuniform_5k_500", rs.randn(5000, 3).astype(np.float32) * [10, 1, 0.1], 500)]
    for name, p, m in tp:
        p = np.ascontiguousarray(p, dtype=np.float32)
        cases.append((name, p, m, bbox_python(p, 16, 16, 16), None))
    # test.py:157-217 granularity sweep (seed 42, randn * 100, 500 samples)
    p = np.ascontiguousarray(np.random.RandomState(42).randn(5000, 3).astype(np.float32) * 100)
    for g in [(8, 8, 8), (16, 16, 16), (32, 32, 32), (64, 64, 64), (16, 8, 4), (4, 16, 64),
              (32, 16, 8)]:
        cases.append((f"granularity_{g[0]}x{g[1]}x{g[2]}", p, 500, bbox_python(p, *g), None))
    # test.py:220-273 manual ranges, including too-tight ones (clamped points)
    rs = np.random.RandomState(123)
    p = rs.randn(3000, 3).astype(np.float32)
    p[:, 0] = p[:, 0] * 50 + 100
    p[:, 1] = p[:, 1] * 20 - 30
    p[:, 2] = p[:, 2] * 5 + 10
    p = np.ascontiguousarray(p)
    cases.append(("manual_bbox_16x16x8", p, 300, bbox_python(p, 16, 16, 8), None))
    cases.append(("manual_includes_all", p, 300, (0, 200, -100, 0, 0, 20, 16, 16, 8), None))
    cases.append(("manual_y_too_tight", p, 300, (0, 200, -40, -20, 0, 20, 16, 16, 8), None))
    cases.append(("manual_z_too_tight", p, 300, (0, 200, -100, 0, 10, 15, 16, 16, 8), None))
    # test.py:276-305 step-by-step trace (seed 123, 100 points, 20 samples)
    p = np.ascontiguousarray(np.random.RandomState(123).randn(100, 3).astype(np.float32))
    cases.append(("trace_100_20", p, 20, bbox_python(p, 16, 16, 16), None))
    # compute_bbox path (range=None), yuezu_fps/yuezu_fps_pybind.cpp:74-76
    p = np.ascontiguousarray(np.random.RandomState(7).randn(4000, 3).astype(np.float32) * 3)
    cases.append(("bbox_default_16", p, 400, None, (16, 16, 16)))
    cases.append(("bbox_32x16x8", p, 400, None, (32, 16, 8)))
    # non-power-of-two and single-block axes: bucket = code % total_blocks aliases
    p = np.ascontiguousarray(np.random.RandomState(8).randn(3000, 3).astype(np.float32) * 4)
    for g in [(10, 10, 10), (4, 4, 1), (3, 5, 7), (1, 1, 1), (1, 8, 8), (12, 6, 2)]:
        cases.append((f"general_{g[0]}x{g[1]}x{g[2]}", p, 300, (-12, 12, -12, 12, -12, 12, *g),
                      None))
    # integer lattice: exact distance ties across different cells
    g = np.stack(np.meshgrid(np.arange(12), np.arange(12), np.arange(12), indexing="ij"), -1)
    g = g.reshape(-1, 3).astype(np.float32)
    g = np.ascontiguousarray(g[np.random.RandomState(9).permutation(len(g))])
    cases.append(("lattice_ties_16", g, 600, (-0.5, 11.5, -0.5, 11.5, -0.5, 11.5, 16, 16, 16),
                  None))
    cases.append(("lattice_ties_4", g, 900, (-0.5, 11.5, -0.5, 11.5, -0.5, 11.5, 4, 4, 4), None))
    # grid-aligned coordinates: points exactly on cell boundaries
    v = (np.arange(-8, 9) / 8.0).astype(np.float32)
    b = np.stack(np.meshgrid(v, v, v, indexing="ij"), -1).reshape(-1, 3)
    b = np.ascontiguousarray(b[np.random.RandomState(10).permutation(len(b))])
    cases.append(("boundary_aligned", b, 800, (-1, 1, -1, 1, -1, 1, 16, 16, 16), None))
    # tiny separations: subnormal squared distances
    t = np.random.RandomState(11).randn(500, 3).astype(np.float32) * np.float32(1e-21)
    t[250:] += np.float32(1e-19)
    t = np.ascontiguousarray(t)
    cases.append(("subnormal_distances", t, 200, (-1e-18, 1e-18, -1e-18, 1e-18, -1e-18, 1e-18,
                                                  8, 8, 8), None))
    # duplicates spread over a shell (ties inside buckets, batched-workload style)
    d = np.random.RandomState(12).randn(2000, 3)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    d[::7] = d[3]
    d = np.ascontiguousarray(d.astype(np.float32))
    cases.append(("shell_duplicates", d, 500, None, (16, 16, 16)))
    # a cloud whose early stop comes before n_samples (many duplicates)
    e = np.repeat(np.random.RandomState(13).randn(40, 3).astype(np.float32), 5, axis=0)
    e = np.ascontiguousarray(e[np.random.RandomState(14).permutation(len(e))])
    cases.append(("early_stop_duplicates", e, 150, (-4, 4, -4, 4, -4, 4, 8, 8, 8), None))
    # large magnitudes
    L = np.ascontiguousarray(np.random.RandomState(15).uniform(-1e6, 1e6, (3000, 3))
                             .astype(np.float32))
    cases.append(("large_magnitude", L, 300, (-1e6, 1e6, -1e6, 1e6, -1e6, 1e6, 32, 32, 32), None))
    # the quickstart workload in full (10,000 points -> 1,000 samples)
    w = make_workload("quickstart")
    cases.append(("quickstart_full", w["clouds"][0], w["n_samples"], w["range"], None))
    return cases


def census(wnames):
    """Algorithmic bytes of the reference's candidate rule per iteration:
    16 B per candidate point (12 B xyz + 4 B min-distance) and 8 B per
    candidate 16-point leaf (src/yuezu_fps.cpp:495-513, 560-597), entry 0 the
    first full pass.  The reference has no instrumentation, so the counts come
    from the oracle, whose outputs the fixtures above pin to the reference.
    Stored: exact prefix sums for the first 4,096 iterations and the total."""
    o = Oracle()
    path = os.path.join(HERE, "census.npz")
    out = {}
    if os.path.exists(path):  # entries of workloads not regenerated are kept
        with np.load(path, allow_pickle=False) as z:
            out = {k: z[k] for k in z.files if k.split("__")[0] not in wnames}
    for wname in wnames:
        w = make_workload(wname)
        tot = 0
        for b, P in enumerate(w["clouds"]):
            idx, _, pts, lv = o.fps_trace(P, w["n_samples"], w["range"], w["blocks"], leaves=True)
            per = 16 * pts.astype(np.uint64) + 8 * lv.astype(np.uint64)
            tot += int(per.sum())
            if b == 0:
                cum = np.concatenate([[0], np.cumsum(per, dtype=np.uint64)])
                out[f"{wname}__cum4096"] = cum[:4097]
                out[f"{wname}__iters"] = np.array([len(idx)], np.uint64)
        out[f"{wname}__total"] = np.array([tot], np.uint64)
        print(f"census {wname}: {tot / 1e9:.3f} GB", flush=True)
    np.savez_compressed(path, **out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-large", action="store_true",
                    help="skip the 8,388,608-point workload (about 4 minutes)")
    ap.add_argument("--census-only", action="store_true")
    ap.add_argument("--workloads", default="",
                    help="comma-separated workloads: regenerate only their census and hashes")
    args = ap.parse_args()
    wl = ["quickstart", "uniform_cube", "uniform_cube_30", "lidar_scan", "batched_shapes"]
    if not args.skip_large:
        wl.append("clustered")
    only = [n for n in args.workloads.split(",") if n]
    if only:
        wl = only
    census(wl)
    if args.census_only:
        return
    ref = Reference()
    if only:
        configs_for(ref, wl)
        return
    out = {}
    pool = {}  # identical point arrays are stored once: P<i>, referenced by <name>__pid
    for name, p, m, rng, blocks in small_cases():
        if rng is None:
            e = ref.fps(p, m, None, blocks)
            meta = np.array([m, 1, *blocks], dtype=np.float64)
            rr = np.zeros(9, np.float32)
        else:
            e = ref.fps(p, m, rng)
            meta = np.array([m, 0, 0, 0, 0], dtype=np.float64)
            rr = np.array(rng, dtype=np.float32)
        h = sha(p) + str(p.shape)
        if h not in pool:
            pool[h] = len(pool)
            out[f"P{pool[h]}"] = p
        out[f"{name}__pid"] = np.array([pool[h]], dtype=np.int64)
        out[f"{name}__range"] = rr
        out[f"{name}__meta"] = meta
        out[f"{name}__expected"] = e.astype(np.int32)
        print(f"{name:32s} n={len(p):6d} m={m:5d} -> {len(e)} samples", flush=True)
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **out)
    configs_for(ref, wl)


def configs_for(ref, wnames):
    cfg_path = os.path.join(HERE, "configs.json")
    configs = {}
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            configs = json.load(f)
    for wname in wnames:
        w = make_workload(wname)
        t = time.time()
        outs = [ref.fps(P, w["n_samples"], w["range"], w["blocks"]) for P in w["clouds"]]
        el = time.time() - t
        configs[wname] = {
            "input_sha256": sha(np.concatenate(w["clouds"])),
            "n_points": int(sum(len(P) for P in w["clouds"])),
            "n_clouds": len(w["clouds"]),
            "n_samples": w["n_samples"],
            "lengths": [int(len(o)) for o in outs],
            "output_sha256": [sha(o.astype(np.int32)) for o in outs],
            "head": [int(x) for x in outs[0][:16]],
            "reference_seconds": round(el, 2),
        }
        print(f"{wname}: {configs[wname]['lengths'][:4]} in {el:.1f}s", flush=True)
        with open(cfg_path, "w") as f:
            json.dump(configs, f, indent=1)


if __name__ == "__main__":
    main()
