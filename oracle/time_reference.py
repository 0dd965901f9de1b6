"""Times the reference library built from its own sources (oracle/_ref) on one
seeded workload, single-threaded, and prints one JSON line: the whole call
(every cloud, every sample) or, with --samples K, the first K samples of cloud
0 (a prefix of the same sample sequence).

Test infrastructure, like the rest of oracle/: a CPU baseline for reports, not
part of the product path.

    python oracle/time_reference.py clustered [--asbuilt] [--samples K]
"""

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import REF_ASBUILT_SO, REF_SO, Reference  # noqa: E402
from ns_fps_amd.workloads import make_workload  # noqa: E402


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("workload")
    ap.add_argument("--asbuilt", action="store_true",
                    help="the reference built with its setup.py flags (default: -ffp-contract=off)")
    ap.add_argument("--samples", type=int, default=0, help="time a prefix of cloud 0's samples")
    args = ap.parse_args()
    w = make_workload(args.workload)
    ref = Reference(REF_ASBUILT_SO if args.asbuilt else REF_SO)
    clouds = w["clouds"][:1] if args.samples else w["clouds"]
    m = args.samples or int(w["n_samples"])
    t = time.perf_counter()
    outs = [ref.fps(P, m, w["range"], w["blocks"]) for P in clouds]
    el = time.perf_counter() - t
    print(json.dumps({
        "workload": w["name"], "library": os.path.basename(ref.path), "clouds": len(clouds),
        "points_per_cloud": int(len(clouds[0])), "samples": m, "seconds": round(el, 3),
        "samples_per_s": round(m * len(clouds) / el, 1), "threads": 1, "cpu_model": cpu_model(),
        "output_sha256_cloud0": hashlib.sha256(outs[0].astype(np.int32).tobytes()).hexdigest()}),
        flush=True)


if __name__ == "__main__":
    main()
