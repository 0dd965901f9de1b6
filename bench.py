#!/usr/bin/env python3
"""Benchmark of the FPS path on one MI355X.

Metric: FPS ms per call and samples/s at 1,048,576 points -> 65,536 samples
(uniform cube in [-1,1]^3, 32^3 blocks, start index 0), plus the fraction of
the HBM roofline reached by the sampling pass.  A "step" is one complete FPS
call on device-resident input: structure build (cell keys, radix sorts,
leaves) + the whole sampling pass + the int32 indices written to device
memory.

Roofline: the sampling pass (speculative-run rounds: k_update, k_refine,
k_gather, k_run) moves the reference's algorithmic bytes -- 16 B per
candidate point and 8 B per candidate 16-point leaf of every iteration, the
per-iteration census in tests/golden/census.npz -- in the hipEvent-timed
sample_ms of the call.

Prints ONE JSON line (rank 0).  With --all it first prints one extra line per
workload (informational), the contract line always comes last.

  python bench.py [--gpus 1] [--steps 5] [--warmup 1] [--workload uniform_cube]
"""

import argparse
import json
import os
import re
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def workload_config(w, extra=None):
    P = w["clouds"]
    cfg = {
        "workload": w["name"],
        "points_per_cloud": int(len(P[0])),
        "clouds": len(P),
        "n_samples": int(w["n_samples"]),
        "blocks": list(w["blocks"]),
        "range": None if w["range"] is None else [float(v) for v in w["range"][:6]],
        "start_index": 0,
        "input": "device-resident float32 (N,3)" if len(P) == 1 else "host float32 (B,N,3)",
    }
    if extra:
        cfg.update(extra)
    return cfg


def load_census(wname):
    path = os.path.join(ROOT, "tests", "golden", "census.npz")
    if not os.path.exists(path):
        return None
    z = np.load(path, allow_pickle=False)
    if f"{wname}__total" not in z.files:
        return None
    return {"total": int(z[f"{wname}__total"][0]),
            "cum": z[f"{wname}__cum4096"] if f"{wname}__cum4096" in z.files else None}


def golden_hashes(wname):
    path = os.path.join(ROOT, "tests", "golden", "configs.json")
    with open(path) as f:
        return json.load(f).get(wname)


def profile_traffic(kernel="sampling", wname="uniform_cube"):
    """HBM bytes per call of the sampling pass from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE in KiB, calibrated by a copy kernel of
    known size); None when no summary was committed."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{wname}_pmc.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        text = f.read()
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    return float(m.group(1)) if m else None


def run_single(lib, hip, w, steps, warmup):
    import hashlib
    P = w["clouds"][0]
    m = int(w["n_samples"])
    d_xyz = hip.upload(P)
    d_out = hip.malloc(m * 4)
    try:
        for _ in range(warmup):
            lib.fps_device(d_xyz, len(P), m, w["range"], d_out)
        hip.synchronize()
        stats = []
        t0 = time.perf_counter()
        for _ in range(steps):
            n = lib.fps_device(d_xyz, len(P), m, w["range"], d_out)
            stats.append(lib.stats())
        hip.synchronize()
        t1 = time.perf_counter()
        out = hip.download(d_out, n, np.int32)
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
    digest = hashlib.sha256(out.astype(np.int32).tobytes()).hexdigest()
    return (t1 - t0) * 1e3 / steps, stats, out, digest


def run_batched(yf, w, steps, warmup):
    import hashlib
    P = np.stack(w["clouds"])
    for _ in range(warmup):
        yf.fps_batched(P, w["n_samples"], None, *w["blocks"])
    stats = []
    t0 = time.perf_counter()
    for _ in range(steps):
        idx, lens = yf.fps_batched(P, w["n_samples"], None, *w["blocks"])
        stats.append(yf.last_stats())
    t1 = time.perf_counter()
    digests = [hashlib.sha256(idx[b, :lens[b]].astype(np.int32).tobytes()).hexdigest()
               for b in range(len(lens))]
    return (t1 - t0) * 1e3 / steps, stats, digests


def cpu_baseline(w, budget_s=30.0):
    """The reference compiled from its own sources with its setup.py flags
    (oracle/_ref, kind "reference"), else the oracle ("port"); one core; the
    whole first cloud of the workload when it fits the budget, else the first
    iterations extrapolated linearly."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REF_ASBUILT_SO, Oracle, Reference
    P = w["clouds"][0]
    m = int(w["n_samples"])
    if os.path.exists(REF_ASBUILT_SO):
        runner, kind = Reference(REF_ASBUILT_SO), "reference"
    else:
        runner, kind = Oracle(), "port"
    t = time.perf_counter()
    runner.fps(P, m, w["range"], w["blocks"])
    el = time.perf_counter() - t
    base = {"value": round(m / el, 2), "unit": "samples/s", "cores": 1, "kind": kind,
            "ms_per_call": round(el * 1e3, 2),
            "sample": f"one full call on cloud 0 of {w['name']} ({len(P)} points -> {m} samples), "
                      f"single thread, {os.path.basename(getattr(runner, 'path', 'liboracle.so'))}"}
    o = Oracle()
    # our C restatement on the same call, one core, against the reference
    if kind == "reference":
        try:
            t = time.perf_counter()
            o.fps(P, m, w["range"], w["blocks"])
            el_port = time.perf_counter() - t
            base["port_ms_per_call"] = round(el_port * 1e3, 2)
            base["port_over_reference"] = round(el_port / el, 3)
        except Exception as e:  # informational only
            base["port_error"] = str(e)
    # naive O(N*M) FPS, first iterations extrapolated linearly (cost per
    # iteration is constant): one thread, then every core of the host
    try:
        k = max(16, min(m - 1, int(2e8 // max(len(P), 1))))
        t = time.perf_counter()
        o.fps_naive(P, m, tie="index", max_iters=k)
        el = time.perf_counter() - t
        base["naive_ms_extrapolated"] = round(el / k * (m - 1) * 1e3, 1)
        base["naive_sample"] = f"first {k} of {m - 1} iterations, single thread, extrapolated"
        nt = o.max_threads()
        k = max(16, min(m - 1, int(2e8 * nt // max(len(P), 1))))
        t = time.perf_counter()
        o.fps_naive_mt(P, m, max_iters=k, threads=nt)
        el = time.perf_counter() - t
        base["naive_mt_ms_extrapolated"] = round(el / k * (m - 1) * 1e3, 1)
        base["naive_mt_threads"] = nt
        base["naive_mt_sample"] = (f"first {k} of {m - 1} iterations, {nt} OpenMP threads, "
                                   "extrapolated")
    except Exception as e:  # the naive timings are informational only
        base["naive_error"] = str(e)
    return base


def run_ball_query(lib, hip, steps, radius=0.05, nsample=32):
    """The grouping step after FPS on the uniform cube: 65,536 FPS centers,
    ball query on device-resident buffers; 256 rows checked against the
    oracle's scan."""
    from ns_fps_amd.workloads import make_workload
    w = make_workload("uniform_cube")
    P = w["clouds"][0]
    idx = lib.fps(P, int(w["n_samples"]), w["range"])
    C = np.ascontiguousarray(P[idx])
    d_p, d_c = hip.upload(P), hip.upload(C)
    d_o = hip.malloc(len(C) * nsample * 4)
    try:
        lib.ball_query_device(d_p, len(P), d_c, len(C), radius, nsample, d_o)
        t0 = time.perf_counter()
        for _ in range(steps):
            lib.ball_query_device(d_p, len(P), d_c, len(C), radius, nsample, d_o)
        t1 = time.perf_counter()
        out = hip.download(d_o, len(C) * nsample, np.int32).reshape(len(C), nsample)
    finally:
        for b in (d_p, d_c, d_o):
            hip.free(b)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle, ball_query
    rows = np.linspace(0, len(C) - 1, 256).astype(np.int64)
    exact = bool(np.array_equal(out[rows], ball_query(Oracle(), P, C[rows], radius, nsample)))
    ms = (t1 - t0) * 1e3 / steps
    return {"workload": "ball_query_uniform_cube", "points": len(P), "centers": len(C),
            "radius": radius, "nsample": nsample, "ms_per_call": round(ms, 3),
            "centers_per_s": round(len(C) / (ms / 1e3), 1), "rows_checked_vs_oracle": len(rows),
            "exact": exact}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="uniform_cube")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--all", action="store_true", help="also print a line per workload")
    ap.add_argument("--ball-query", action="store_true",
                    help="time only the grouping step after FPS (ball query) and print its line")
    ap.add_argument("--calibrate", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device (a copy kernel of known size for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this FPS path runs on exactly one GPU: a single cloud's "
                                   "iterations are sequential and batched clouds are independent; "
                                   "run with --gpus 1"}))
        sys.exit(2)

    from ns_fps_amd.capi import Hip, Lib
    from ns_fps_amd.workloads import make_workload
    import ns_fps_amd.yuezu_fps_module as yf

    lib = Lib()
    if lib.device_count() < 1:
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    hip = Hip()
    if args.calibrate:
        nbytes = args.calibrate << 20
        src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
        hip.memcpy_d2d(dst, src, nbytes)
        hip.synchronize()
        hip.free(src)
        hip.free(dst)

    if args.ball_query:
        print(json.dumps(run_ball_query(lib, hip, args.steps)), flush=True)
        return

    if args.all:
        for wname in ["quickstart", "uniform_cube", "lidar_scan", "batched_shapes", "clustered"]:
            w = make_workload(wname)
            g = golden_hashes(wname)
            if len(w["clouds"]) == 1:
                steps = 1 if wname == "clustered" else 3
                ms, st, out, dg = run_single(lib, hip, w, steps, 1 if wname != "clustered" else 0)
                exact = g is not None and dg == g["output_sha256"][0]
                s = st[-1]
                line = {"workload": wname, "ms_per_call": round(ms, 3),
                        "device_ms": round(s["device_ms"], 3), "build_ms": round(s["build_ms"], 3),
                        "late_ms": round(s["late_ms"], 3), "wide_ms": round(s["wide_ms"], 3),
                        "samples_per_s": round(len(out) / (ms / 1e3), 1), "bit_exact": exact}
            else:
                ms, st, dgs = run_batched(yf, w, 3, 1)
                exact = g is not None and dgs == g["output_sha256"]
                s = st[-1]
                line = {"workload": wname, "ms_per_call": round(ms, 3),
                        "device_ms": round(s["device_ms"], 3), "e2e_ms": round(s["e2e_ms"], 3),
                        "samples_per_s": round(s["samples"] / (ms / 1e3), 1), "bit_exact": exact}
            census = load_census(wname)
            if census:
                line["alg_gb"] = round(census["total"] / 1e9, 3)
                line["alg_gbs_over_device_time"] = round(census["total"] / (line["device_ms"] * 1e6), 1)
            print(json.dumps(line), flush=True)

    w = make_workload(args.workload)
    if len(w["clouds"]) != 1:
        print(json.dumps({"error": "the contract line needs a single-cloud workload"}))
        sys.exit(2)
    ms, stats, out, digest = run_single(lib, hip, w, args.steps, args.warmup)
    m = int(w["n_samples"])
    g = golden_hashes(args.workload)
    exact = g is not None and digest == g["output_sha256"][0] and len(out) == g["lengths"][0]
    sample_ms = statistics.mean(s["sample_ms"] for s in stats)
    census = load_census(args.workload)
    roofline = None
    engine = "runs" if stats[-1].get("engine", 0) else "tree"
    if census is not None:
        alg = census["total"]  # every iteration, first pass included
        achieved = alg / (sample_ms * 1e6)  # GB/s
        roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6),
                    "traffic": profile_traffic("sampling", args.workload),
                    "kernel": "sampling pass (k_update+k_refine+k_gather+k_run rounds)"
                    if engine == "runs" else "k_wide_update+k_late_loop",
                    "alg_bytes_per_launch": alg, "kernel_ms": round(sample_ms, 3)}
    wide_iters = int(stats[-1]["wide_iters"])
    line = {
        "metric": "FPS ms/call & samples/s at 1M pts -> 65,536 samples; % of HBM roofline",
        "value": round(len(out) / (ms / 1e3), 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded uniform cube, NumPy RandomState(2))",
        "config": workload_config(w, {"engine": engine, "rounds": int(stats[-1].get("rounds", 0)),
                                      "wide_iters": wide_iters,
                                      "device_ms": round(statistics.mean(s["device_ms"] for s in stats), 3),
                                      "build_ms": round(statistics.mean(s["build_ms"] for s in stats), 3),
                                      "bit_exact_vs_reference": exact}),
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
