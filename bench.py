#!/usr/bin/env python3
"""Benchmark of the FPS path on one MI355X.

Metric: FPS ms per call and samples/s at 1,048,576 points -> 65,536 samples
(uniform cube in [-1,1]^3, 32^3 blocks, start index 0), plus the fraction of
the HBM roofline reached by the sampling pass.  A "step" is one complete FPS
call on device-resident input: structure build (cell keys, radix sorts,
leaves) + the whole sampling pass + the int32 indices written to device
memory.

Roofline: the sampling pass moves the reference's algorithmic bytes -- 16 B
per candidate point and 8 B per candidate 16-point leaf of every iteration,
the per-iteration census in tests/golden/census.npz -- in the hipEvent-timed
sample_ms of the call.

Besides the steady-state time of repeated calls (ms_per_step, and the
median of the same calls, each of which returns after its stream work), the
line reports the first call of a shape (first_call_ms: no replayed round
schedule), the host-buffer call with its PCIe copies (e2e_ms) and the
sampling of a prepared plan (plan_sample_ms).

The other four benchmark configurations (the 10,000-point quickstart, the
120,000-point LiDAR scan, 64 batched clouds of 16,384 points with per-cloud
compute_bbox, and the 8,388,608-point clustered cloud) each print one line
first -- median ms per call on device-resident input, samples/s, the
sampling pass's roofline and traffic, the reference CPU path on this host,
bit-exactness against the reference's hashes -- and the contract line
carries the same figures in its "configs" block.  --all adds the uniform
cube on a 30^3 grid (the general bucket path).  The contract line always
comes last.

  python bench.py [--gpus 1] [--steps 20] [--warmup 2] [--workload uniform_cube]
"""

import argparse
import hashlib
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
HEADLINE_METRIC = "FPS ms/call & samples/s at 1M pts -> 65,536 samples; % of HBM roofline"
ALL_WORKLOADS = ["quickstart", "uniform_cube", "uniform_cube_30", "lidar_scan", "batched_shapes",
                 "clustered"]
# the benchmark configurations besides the headline one, in their order
OTHER_CONFIGS = ["quickstart", "lidar_scan", "batched_shapes", "clustered"]


def metric_for(w):
    if w["name"] == "uniform_cube":
        return HEADLINE_METRIC
    n, m = len(w["clouds"][0]), int(w["n_samples"])
    per = f"{len(w['clouds'])} x " if len(w["clouds"]) > 1 else ""
    return (f"FPS ms/call & samples/s at {per}{n:,} pts -> {m:,} samples ({w['name']}); "
            "% of HBM roofline")


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
        "input": "device-resident float32 (N,3)" if len(P) == 1 else
                 "device-resident float32 (B,N,3)",
    }
    if extra:
        cfg.update(extra)
    return cfg


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "cpus_available": avail}


def load_census(wname):
    path = os.path.join(ROOT, "tests", "golden", "census.npz")
    if not os.path.exists(path):
        return None
    z = np.load(path, allow_pickle=False)
    if f"{wname}__total" not in z.files:
        return None
    return {"total": int(z[f"{wname}__total"][0])}


def golden_hashes(wname):
    path = os.path.join(ROOT, "tests", "golden", "configs.json")
    with open(path) as f:
        return json.load(f).get(wname)


def profile_traffic(kernel, wname):
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


def sha_i32(a):
    return hashlib.sha256(np.asarray(a, np.int32).tobytes()).hexdigest()


def roofline_of(wname, sample_ms, engine):
    census = load_census(wname)
    if census is None or not sample_ms or sample_ms <= 0:
        return None
    alg = census["total"]  # every iteration, first pass included
    achieved = alg / (sample_ms * 1e6)  # GB/s
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 6),
            "traffic": profile_traffic("sampling", wname),
            "kernel": "sampling pass (k_update+k_refine+k_gather+k_run rounds)"
            if engine == "runs" else "sampling pass (k_wide_update+k_late_loop)",
            "alg_bytes_per_launch": alg, "kernel_ms": round(sample_ms, 3)}


# ------------------------------------------------------------------ GPU legs

def run_single(lib, hip, w, steps, warmup):
    """Device-resident input.  Returns the steady-state ms per call, per-call
    statistics, the output and its digest, the digest of every timed call's
    output (each call writes its own buffer, hashed after the timed region),
    and the first call of the shape."""
    P = w["clouds"][0]
    m = int(w["n_samples"])
    d_xyz = hip.upload(P)
    d_out = hip.malloc(m * 4)
    d_outs = [hip.malloc(m * 4) for _ in range(steps)]
    try:
        # a call of another shape first, so that the timed first call replays
        # no round schedule
        lib.fps_device(d_xyz, len(P), m - 1, w["range"], d_out)
        hip.synchronize()
        t = time.perf_counter()
        lib.fps_device(d_xyz, len(P), m, w["range"], d_out)
        first_ms = (time.perf_counter() - t) * 1e3
        first_stats = lib.stats()
        for _ in range(warmup):
            lib.fps_device(d_xyz, len(P), m, w["range"], d_out)
        hip.synchronize()
        stats, per_call, lens = [], [], []
        # the range struct built once, and each call's statistics kept as the
        # C struct: Python conversions stay out of the timed calls
        from ns_fps_amd.capi import Range
        rng = Range.of(w["range"])
        t0 = time.perf_counter()
        for k in range(steps):
            tc = time.perf_counter()
            n = lib.fps_device(d_xyz, len(P), m, rng, d_outs[k])  # returns after the stream
            per_call.append((time.perf_counter() - tc) * 1e3)
            stats.append(lib.stats_raw())
            lens.append(n)
        hip.synchronize()
        t1 = time.perf_counter()
        stats = [st.as_dict() for st in stats]
        outs = [hip.download(d_outs[k], lens[k], np.int32) for k in range(steps)]
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
        for d in d_outs:
            hip.free(d)
    digests = [sha_i32(o) for o in outs]
    return {"ms": (t1 - t0) * 1e3 / steps, "median_ms": statistics.median(per_call),
            "stats": stats, "out": outs[-1], "digest": digests[-1], "digests": digests,
            "first_ms": first_ms, "first_stats": first_stats}


def run_host_buffers(lib, w, reps=3):
    """nsfps_fps on host buffers: upload, build, sampling, download."""
    P = w["clouds"][0]
    m = int(w["n_samples"])
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        out = lib.fps(P, m, w["range"])
        times.append((time.perf_counter() - t) * 1e3)
    return statistics.median(times), sha_i32(out)


def run_plan(lib, hip, w, steps):
    """A plan created once on device-resident input, sampled `steps` times."""
    if not hasattr(lib, "plan_create"):
        return None
    P = w["clouds"][0]
    m = int(w["n_samples"])
    d_xyz = hip.upload(P)
    d_out = hip.malloc(m * 4)
    plan = None
    try:
        t = time.perf_counter()
        plan = lib.plan_create(d_xyz, len(P), w["range"], on_device=True)
        create_ms = (time.perf_counter() - t) * 1e3
        lib.plan_sample(plan, m, d_out)
        hip.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            n = lib.plan_sample(plan, m, d_out)
        hip.synchronize()
        t1 = time.perf_counter()
        out = hip.download(d_out, n, np.int32)
    finally:
        if plan is not None:
            lib.plan_destroy(plan)
        hip.free(d_xyz)
        hip.free(d_out)
    return {"plan_create_ms": round(create_ms, 3),
            "plan_sample_ms": round((t1 - t0) * 1e3 / steps, 3), "digest": sha_i32(out)}


def run_batched(lib, hip, w, steps, warmup):
    """Device-resident clouds (B, N, 3) through nsfps_fps_batched_device:
    per-cloud compute_bbox (range=None) on the device, build and sampling of
    every cloud, the samples in device memory."""
    P = np.ascontiguousarray(np.stack(w["clouds"]))
    B, n, m = P.shape[0], P.shape[1], int(w["n_samples"])
    d_xyz, d_out = hip.upload(P), hip.malloc(B * m * 4)
    d_outs = [hip.malloc(B * m * 4) for _ in range(steps)]  # one per timed call
    try:
        # a call of another shape first, so that the timed first call replays
        # no round schedule
        lib.fps_batched_device(d_xyz, B, n, m - 1, d_out, w["range"], w["blocks"])
        t = time.perf_counter()
        lib.fps_batched_device(d_xyz, B, n, m, d_out, w["range"], w["blocks"])
        first_ms = (time.perf_counter() - t) * 1e3
        for _ in range(warmup):
            lib.fps_batched_device(d_xyz, B, n, m, d_out, w["range"], w["blocks"])
        stats, per_call, all_lens = [], [], []
        t0 = time.perf_counter()
        for k in range(steps):
            tc = time.perf_counter()
            lens = lib.fps_batched_device(d_xyz, B, n, m, d_outs[k], w["range"], w["blocks"])
            per_call.append((time.perf_counter() - tc) * 1e3)
            stats.append(lib.stats_raw())  # converted after the timed calls
            all_lens.append(lens)
        t1 = time.perf_counter()
        stats = [st.as_dict() for st in stats]
        outs = [hip.download(d_outs[k], B * m, np.int32).reshape(B, m) for k in range(steps)]
    finally:
        hip.free(d_xyz)
        hip.free(d_out)
        for d in d_outs:
            hip.free(d)
    calls = [[sha_i32(o[b, :ln[b]]) for b in range(B)] for o, ln in zip(outs, all_lens)]
    return {"ms": (t1 - t0) * 1e3 / steps, "median_ms": statistics.median(per_call),
            "stats": stats, "lens": all_lens[-1], "digests": calls[-1], "call_digests": calls,
            "first_ms": first_ms}


def run_batched_host(yf, w, reps=3):
    """The same clouds as host arrays through the module's fps_batched (copies
    to and from the device included)."""
    P = np.stack(w["clouds"])
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        idx, lens = yf.fps_batched(P, w["n_samples"], None, *w["blocks"])
        times.append((time.perf_counter() - t) * 1e3)
    return statistics.median(times), [sha_i32(idx[b, :lens[b]]) for b in range(len(lens))]


# ------------------------------------------------------------- CPU baseline

def cpu_baseline(w, budget_s=30.0):
    """The reference compiled from its own sources with its setup.py flags
    (oracle/_ref, kind "reference"), else the oracle ("port"); one core.

    A prefix of cloud 0's samples is timed first; when the whole workload (all
    clouds, every sample), extrapolated linearly from it, fits budget_s, the
    whole workload is timed, up to three times (median).  Otherwise the longest
    power-of-two prefix of cloud 0's sample sequence that fits the budget is
    timed once (a prefix costs more per sample than the whole call: early
    samples have the largest cubes)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import REF_ASBUILT_SO, Oracle, Reference
    clouds = w["clouds"]
    m = int(w["n_samples"])
    if os.path.exists(REF_ASBUILT_SO):
        runner, kind = Reference(REF_ASBUILT_SO), "reference"
    else:
        runner, kind = Oracle(), "port"
    rng, blocks = w["range"], w["blocks"]
    mp = min(m, max(64, m // 16))
    t = time.perf_counter()
    runner.fps(clouds[0], mp, rng, blocks)
    t_p = time.perf_counter() - t
    est = t_p * (m / mp) * len(clouds)
    info = cpu_info()
    if est <= budget_s:
        times = []
        while True:
            t = time.perf_counter()
            for P in clouds:
                runner.fps(P, m, rng, blocks)
            times.append(time.perf_counter() - t)
            if len(times) == 3 or (len(times) + 1) * times[0] > budget_s:
                break
        reps = len(times)
        el = statistics.median(times)
        done = m * len(clouds)
        what = (f"{'all ' + str(len(clouds)) + ' clouds' if len(clouds) > 1 else 'the whole call'} "
                f"of {w['name']} ({len(clouds[0])} points -> {m} samples"
                f"{' each' if len(clouds) > 1 else ''}), median of {reps}")
        sample_m = m
    else:
        sample_m = mp
        while sample_m * 2 <= m and t_p * (sample_m * 2 / mp) <= budget_s:
            sample_m *= 2
        t = time.perf_counter()
        runner.fps(clouds[0], sample_m, rng, blocks)
        el = time.perf_counter() - t
        done = sample_m
        what = (f"the first {sample_m} of {m} samples of cloud 0 of {w['name']} "
                f"({len(clouds[0])} points; a prefix of the same sample sequence), one run")
    base = {"value": round(done / el, 2), "unit": "samples/s", "cores": 1, "kind": kind,
            "ms_per_call": round(el * 1e3, 2) if sample_m == m else None,
            "ms_sample": round(el * 1e3, 2),
            "sample": f"{what}; single thread, "
                      f"{os.path.basename(getattr(runner, 'path', 'liboracle.so'))}",
            **info}
    if kind == "reference":
        # our C restatement (the oracle) on the same sample, one core
        try:
            o = Oracle()
            t = time.perf_counter()
            if sample_m == m:
                for P in clouds:
                    o.fps(P, m, rng, blocks)
            else:
                o.fps(clouds[0], sample_m, rng, blocks)
            el_port = time.perf_counter() - t
            base["port_ms_sample"] = round(el_port * 1e3, 2)
            base["port_over_reference"] = round(el_port / el, 3)
        except Exception as e:  # informational only
            base["port_error"] = str(e)
    return base


def naive_baselines(w):
    """Naive O(N*M) FPS on cloud 0, the first iterations extrapolated linearly
    (cost per iteration is constant): one thread, then every core."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from oracle import Oracle
    o = Oracle()
    P = w["clouds"][0]
    m = int(w["n_samples"])
    out = {}
    try:
        k = max(16, min(m - 1, int(2e8 // max(len(P), 1))))
        t = time.perf_counter()
        o.fps_naive(P, m, tie="index", max_iters=k)
        el = time.perf_counter() - t
        out["naive_ms_extrapolated"] = round(el / k * (m - 1) * 1e3, 1)
        out["naive_sample"] = f"first {k} of {m - 1} iterations, single thread, extrapolated"
        nt = o.max_threads()
        k = max(16, min(m - 1, int(2e8 * nt // max(len(P), 1))))
        t = time.perf_counter()
        o.fps_naive_mt(P, m, max_iters=k, threads=nt)
        el = time.perf_counter() - t
        out["naive_mt_ms_extrapolated"] = round(el / k * (m - 1) * 1e3, 1)
        out["naive_mt_threads"] = nt
        out["naive_mt_sample"] = (f"first {k} of {m - 1} iterations, {nt} OpenMP threads, "
                                  "extrapolated")
    except Exception as e:  # the naive timings are informational only
        out["naive_error"] = str(e)
    return out


# ---------------------------------------------------------------- grouping

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


# ------------------------------------------------------------ phase clocks

RUN_PHASES = ["load", "select", "gather", "phases", "apply", "tail", "big", "rank", "picks",
              "rounds", "hot_sets", "phase_count", "walk", "publish", "rt_load", "rt_total"]
PASS_COUNTERS = ["update_leaves", "update_points", "gather_leaves", "gather_points"]


def run_phases(lib, hip, w):
    """One call with NSFPS_PROFILE=1: the run kernel's phase clocks summed over
    rounds (s_memtime cycles of wave 0 between its barriers, and s_memrealtime
    ticks of 10 ns for the load and the whole kernel), per round and per hot
    set.  Batched clouds: one call of all of them, the counters of cloud 0
    (every kernel adds to its own cloud's words)."""
    os.environ["NSFPS_PROFILE"] = "1"
    try:
        P = np.ascontiguousarray(np.stack(w["clouds"]))
        B, n, m = P.shape[0], P.shape[1], int(w["n_samples"])
        d_xyz = hip.upload(P)
        d_out = hip.malloc(B * m * 4)
        try:
            if B == 1:
                lib.fps_device(d_xyz, n, m, w["range"], d_out)
            else:
                lib.fps_batched_device(d_xyz, B, n, m, d_out, w["range"], w["blocks"])
            st = lib.stats()
            words = lib.loop_profile()
        finally:
            hip.free(d_xyz)
            hip.free(d_out)
    finally:
        del os.environ["NSFPS_PROFILE"]
    v = dict(zip(RUN_PHASES, words[:16]))
    ctr = dict(zip(PASS_COUNTERS, words[24:28]))
    ctr.update(zip(["up_t_picks", "up_t_leaves", "up_t_flush", "up_groups"], words[32:36]))
    ctr.update(zip(["up_t_load", "up_t_zero", "up_t_hits", "up_t_points"], words[40:44]))
    ctr.update(zip(["ga_t_select", "ga_t_records", "ga_t_points_claim", "ga_t_writes", "ga_groups"],
                   words[44:49]))
    ctr.update(zip(["up_w_points_max", "up_w_points_sum", "up_w_loop_max", "up_w_loop_sum"],
                   words[49:53]))
    ctr.update(zip(["update_touched_leaves", "update_touched_points"], words[53:55]))
    ctr.update(zip(["up_w_hits_max", "up_w_hits_sum"], words[55:57]))
    ctr.update(zip(["window_keys", "listed", "window_keys_max"], words[57:60]))
    v["walk_wait"], v["alias"], v["alias_entries"] = words[28], words[29], words[30]
    rounds = max(1, v["rounds"])
    hot = max(1, v["hot_sets"])
    cycles = {k: v[k] for k in ["load", "select", "gather", "rank", "phases", "walk", "walk_wait",
                                "alias", "apply", "big", "publish", "tail"]}
    cyc_total = sum(cycles.values())
    rt_us = v["rt_total"] * 0.01
    clock_ghz = cyc_total / (rt_us * 1e3) if rt_us else None
    return {"workload": w["name"], "profile": "run kernel phase clocks (NSFPS_PROFILE=1)",
            "rounds": v["rounds"], "hot_sets": v["hot_sets"], "picks": v["picks"],
            "phases": v["phase_count"], "samples_per_hot_set": round(v["picks"] / hot, 2),
            "phases_per_hot_set": round(v["phase_count"] / hot, 2),
            "multi_cell_entries_per_hot_set": round(v["alias_entries"] / hot, 1),
            "run_kernel_us_per_round": round(rt_us / rounds, 2),
            "load_us_per_round": round(v["rt_load"] * 0.01 / rounds, 2),
            "run_kernel_us_total": round(rt_us, 1),
            "s_memtime_ghz": round(clock_ghz, 3) if clock_ghz else None,
            "cycles_per_hot_set": {k: round(cycles[k] / hot, 1) for k in cycles
                                   if k not in ("load", "tail")},
            "cycles_per_round": {"load": round(cycles["load"] / rounds, 1),
                                 "tail": round(cycles["tail"] / rounds, 1)},
            "sample_ms": round(st["sample_ms"], 3), "device_ms": round(st["device_ms"], 3),
            "passes": pass_counts(w["name"], ctr, rounds)}


def pass_counts(wname, ctr, rounds):
    """The grid-wide passes' device-counted reads against the census: leaves
    (64-point) and points whose data the update and gather passes read, per
    round and in total, and their bytes at the census's own prices (16 B per
    point, 8 B per leaf) beside the census's total (16 B per candidate point,
    8 B per candidate 16-point leaf of the reference's iterations)."""
    out = {k: int(ctr[k]) for k in PASS_COUNTERS}
    out.update({k + "_per_round": round(ctr[k] / rounds, 1) for k in PASS_COUNTERS})
    census = load_census(wname)
    dev = 16 * (ctr["update_points"] + ctr["gather_points"]) + \
        8 * (ctr["update_leaves"] + ctr["gather_leaves"])
    out["device_bytes_at_census_prices"] = int(dev)
    if ctr.get("up_groups"):
        ng = ctr["up_groups"]
        out["update_pass_us_per_workgroup"] = {
            "state_node_picks": round(ctr["up_t_picks"] * 0.01 / ng, 2),
            "leaves": round(ctr["up_t_leaves"] * 0.01 / ng, 2),
            "node_key_flush": round(ctr["up_t_flush"] * 0.01 / ng, 2),
            "workgroups_per_round": round(ng / rounds, 1),
            "touched_leaves_per_round": round(ctr.get("update_touched_leaves", 0) / rounds, 1),
            "touched_points_per_round": round(ctr.get("update_touched_points", 0) / rounds, 1),
            # parts of the first two: the first reads, clearing the histogram,
            # finding the touched leaves, their points' reads
            "first_reads": round(ctr.get("up_t_load", 0) * 0.01 / ng, 2),
            "hist_clear": round(ctr.get("up_t_zero", 0) * 0.01 / ng, 2),
            "touched_leaves": round(ctr.get("up_t_hits", 0) * 0.01 / ng, 2),
            "point_reads": round(ctr.get("up_t_points", 0) * 0.01 / ng, 2),
            # over the 16 waves, from the picks' barrier: points in, loop done
            "waves_touched_found_latest": round(ctr.get("up_w_hits_max", 0) * 0.01 / ng, 2),
            "waves_touched_found_mean": round(ctr.get("up_w_hits_sum", 0) * 0.01 / ng / 16, 2),
            "waves_points_in_latest": round(ctr.get("up_w_points_max", 0) * 0.01 / ng, 2),
            "waves_points_in_mean": round(ctr.get("up_w_points_sum", 0) * 0.01 / ng / 16, 2),
            "waves_loop_done_latest": round(ctr.get("up_w_loop_max", 0) * 0.01 / ng, 2),
            "waves_loop_done_mean": round(ctr.get("up_w_loop_sum", 0) * 0.01 / ng / 16, 2)}
    if ctr.get("window_keys"):
        out["window_keys_per_round"] = round(ctr["window_keys"] / rounds, 1)
        out["listed_per_round"] = round(ctr["listed"] / rounds, 1)
        out["window_keys_max"] = int(ctr["window_keys_max"])
    if ctr.get("ga_groups"):
        ng = ctr["ga_groups"]
        out["gather_pass_us_per_workgroup"] = {  # the first node chunk of each workgroup
            "selection": round(ctr["ga_t_select"] * 0.01 / ng, 2),
            "leaf_records": round(ctr["ga_t_records"] * 0.01 / ng, 2),
            "points_and_claim": round(ctr["ga_t_points_claim"] * 0.01 / ng, 2),
            "writes": round(ctr["ga_t_writes"] * 0.01 / ng, 2),
            "workgroups_per_round": round(ng / rounds, 1)}
    if census is not None:
        out["census_alg_bytes"] = census["total"]
        out["device_over_census"] = round(dev / census["total"], 4)
    return out


# --------------------------------------------------------------------- lines

def workload_line(lib, hip, yf, wname, budget_s, steps, warmup, with_cpu=True):
    """One line per workload: median ms per call on device-resident input,
    samples/s, the sampling pass's roofline (with the committed traffic
    profile), the reference's CPU time on this host, bit-exactness."""
    from ns_fps_amd.workloads import make_workload
    w = make_workload(wname)
    g = golden_hashes(wname)
    if len(w["clouds"]) == 1:
        big = wname == "clustered"
        r = run_single(lib, hip, w, min(steps, 5) if big else steps, min(warmup, 1) if big else warmup)
        s = r["stats"][-1]
        exact = g is not None and all(d == g["output_sha256"][0] for d in r["digests"])
        samples = len(r["out"])
        line = {"workload": wname, "metric": metric_for(w),
                "ms_per_call": round(r["median_ms"], 3), "ms_mean": round(r["ms"], 3),
                "calls": len(r["stats"]), "first_call_ms": round(r["first_ms"], 3),
                "device_ms": round(s["device_ms"], 3), "build_ms": round(s["build_ms"], 3),
                "sample_ms": round(s["sample_ms"], 3), "rounds": int(s["rounds"]),
                "samples_per_s": round(samples / (r["median_ms"] / 1e3), 1), "bit_exact": exact,
                "calls_checked": len(r["digests"])}
        if not big:
            e2e, dg = run_host_buffers(lib, w)
            line["e2e_ms"] = round(e2e, 3)
            line["e2e_bit_exact"] = g is not None and dg == g["output_sha256"][0]
        engine = "runs" if s["engine"] else "tree"
    else:
        r = run_batched(lib, hip, w, steps, warmup)
        s = r["stats"][-1]
        exact = g is not None and all(c == g["output_sha256"] for c in r["call_digests"])
        samples = int(sum(r["lens"]))
        e2e, dg = run_batched_host(yf, w)
        line = {"workload": wname, "metric": metric_for(w),
                "ms_per_call": round(r["median_ms"], 3), "ms_mean": round(r["ms"], 3),
                "calls": len(r["stats"]), "first_call_ms": round(r["first_ms"], 3),
                "device_ms": round(s["device_ms"], 3), "build_ms": round(s["build_ms"], 3),
                "sample_ms": round(s["sample_ms"], 3), "rounds": int(s["rounds"]),
                "samples_per_s": round(samples / (r["median_ms"] / 1e3), 1), "bit_exact": exact,
                "calls_checked": len(r["call_digests"]),
                "input": "device-resident float32 (B,N,3); range=None: per-cloud compute_bbox "
                         "on the device",
                "e2e_ms": round(e2e, 3),
                "e2e_bit_exact": g is not None and dg == g["output_sha256"],
                "e2e_input": "host float32 (B,N,3) through the module's fps_batched"}
        engine = "runs" if s["engine"] else "tree"
    line["mixed_leaves"] = bool(s.get("mixed", 0))
    line["roofline"] = roofline_of(wname, statistics.mean(x["sample_ms"] for x in r["stats"]),
                                   engine)
    if with_cpu:
        line["cpu_baseline"] = cpu_baseline(w, budget_s)
        cb = line["cpu_baseline"]
        if cb.get("ms_per_call"):
            line["speedup_vs_cpu_baseline"] = round(cb["ms_per_call"] / line["ms_per_call"], 1)
    return line


def config_summary(line):
    """The compact form of a workload line carried in the contract line."""
    rf = line.get("roofline") or {}
    cb = line.get("cpu_baseline") or {}
    out = {"ms_per_call": line["ms_per_call"], "samples_per_s": line["samples_per_s"],
           "sample_ms": line["sample_ms"], "bit_exact": line["bit_exact"],
           "roofline": {k: rf.get(k) for k in ("achieved", "frac", "traffic")} if rf else None}
    if cb:
        out["cpu_baseline"] = {"ms_per_call": cb.get("ms_per_call"), "ms_sample": cb.get("ms_sample"),
                               "samples_per_s": cb.get("value"), "kind": cb.get("kind"),
                               "cores": cb.get("cores"), "sample": cb.get("sample")}
        if line.get("speedup_vs_cpu_baseline"):
            out["speedup_vs_cpu_baseline"] = line["speedup_vs_cpu_baseline"]
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="uniform_cube")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=30.0,
                    help="seconds of reference CPU work per workload (default 30)")
    ap.add_argument("--all", action="store_true",
                    help="also print the uniform cube on a 30^3 grid (the general bucket path) "
                         "among the per-workload lines")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-workload lines (the contract line alone)")
    ap.add_argument("--no-contract", action="store_true",
                    help="stop after the per-workload lines (profiler runs of one workload)")
    ap.add_argument("--only", default="",
                    help="comma-separated workloads for the per-workload lines instead of the "
                         "benchmark configurations")
    ap.add_argument("--ball-query", action="store_true",
                    help="time only the grouping step after FPS (ball query) and print its line")
    ap.add_argument("--phases", action="store_true",
                    help="print the run kernel's phase clocks of one profiled call and exit")
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
    import yuezu_fps.yuezu_fps_module as yf

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
    if args.phases:
        print(json.dumps(run_phases(lib, hip, make_workload(args.workload))), flush=True)
        return

    configs = {}
    if not args.no_configs:
        names = [n for n in args.only.split(",") if n] or (
            OTHER_CONFIGS + (["uniform_cube_30"] if args.all else []))
        for wname in names:
            line = workload_line(lib, hip, yf, wname, args.cpu_budget, args.steps, args.warmup,
                                 with_cpu=not args.no_cpu_baseline)
            print(json.dumps(line), flush=True)
            configs[wname] = config_summary(line)
    if args.no_contract:
        return

    w = make_workload(args.workload)
    if len(w["clouds"]) != 1:
        print(json.dumps({"error": "the contract line needs a single-cloud workload"}))
        sys.exit(2)
    r = run_single(lib, hip, w, args.steps, args.warmup)
    stats = r["stats"]
    configs_done = dict(configs)
    g = golden_hashes(args.workload)
    exact = (g is not None and len(r["out"]) == g["lengths"][0]
             and all(d == g["output_sha256"][0] for d in r["digests"]))
    sample_ms = statistics.mean(s["sample_ms"] for s in stats)
    engine = "runs" if stats[-1].get("engine", 0) else "tree"
    e2e_ms, e2e_digest = run_host_buffers(lib, w)
    plan = run_plan(lib, hip, w, max(3, args.steps // 2))
    line = {
        "metric": metric_for(w),
        "value": round(len(r["out"]) / (r["ms"] / 1e3), 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 3),
        "ms_median": round(r["median_ms"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded, NumPy RandomState; the workload's generator in "
                "ns_fps_amd/workloads.py)",
        "config": workload_config(w, {
            "engine": engine, "rounds": int(stats[-1].get("rounds", 0)),
            "device_ms": round(statistics.mean(s["device_ms"] for s in stats), 3),
            "build_ms": round(statistics.mean(s["build_ms"] for s in stats), 3),
            "sample_ms": round(sample_ms, 3),
            "bit_exact_vs_reference": exact, "calls_checked": len(r["digests"])}),
        "first_call_ms": round(r["first_ms"], 3),
        "e2e_ms": round(e2e_ms, 3),
        "e2e_bit_exact": g is not None and e2e_digest == g["output_sha256"][0],
        "roofline": roofline_of(args.workload, sample_ms, engine),
    }
    if plan is not None:
        line["plan_sample_ms"] = plan["plan_sample_ms"]
        line["plan_create_ms"] = plan["plan_create_ms"]
        line["plan_bit_exact"] = g is not None and plan["digest"] == g["output_sha256"][0]
    if not args.no_cpu_baseline:
        cb = cpu_baseline(w, args.cpu_budget)
        cb.update(naive_baselines(w))
        line["cpu_baseline"] = cb
    # the other benchmark configurations, measured above in this run
    if configs_done:
        line["configs"] = configs_done
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
