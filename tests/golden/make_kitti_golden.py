"""Writes the KITTI fixtures of the FPS path from the reference itself.

Inputs are the reference's own scans (eval/kitti_data): the 16,384-point cut
of frame 0 (16k_000000.bin, stride 4) and the six full frames
000000-000005.bin.  The samples come from the reference
library compiled from its own sources (oracle/_ref, ``make -C oracle ref``)
and are checked against the CPU restatement (oracle/) before they are written.
The two sampling runs are those of the reference's drivers:

* "cmp": eval/src_cpu/compare_cpu_test_kitti.cpp:195-240 -- keep z >= -5,
  range over the bounds widened by 1e-6 (float32), 128 x 128 x 2 blocks,
  samples reported as the file's record numbers;
* "ex": semantickitti_example.py:15-37 -- the exact bounds, 128 x 128 x 2.

Outputs (only this script writes them; it runs where the reference tree is):

* tests/golden/kitti.npz -- the cut's x, y, z and, per case, sample
  count, range and expected samples (case lowz: the cut with every 997th
  point's z set to -7.5);
* tests/golden/kitti.json -- per full frame: SHA-256 of the file, points
  kept, and per sample count the output length, SHA-256 of the int64 record
  numbers and the first ones.

Usage: python tests/golden/make_kitti_golden.py
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import Oracle, Reference  # noqa: E402

DATA = "/root/reference/eval/kitti_data"


def sha(b):
    return hashlib.sha256(b).hexdigest()


def read(path, stride):
    """x, y, z of whole records, as the C++ reader keeps them."""
    raw = np.fromfile(path, dtype=np.float32)
    n = raw.size // stride
    return np.ascontiguousarray(raw[:n * stride].reshape(n, stride)[:, :3])


def rng_of(p, eps):
    """Exact float32 bounds (the C++ loop's std::min/std::max from point 0;
    the scans hold no NaN), then -/+ eps in float32."""
    lo = [np.float32(p[:, a].min()) for a in range(3)]
    hi = [np.float32(p[:, a].max()) for a in range(3)]
    e = np.float32(eps)
    return (float(lo[0] - e), float(hi[0] + e), float(lo[1] - e), float(hi[1] + e),
            float(lo[2] - e), float(hi[2] + e), 128, 128, 2)


def lowz(k16):
    """Frame 0's cut with every 997th point moved below z = -5: the filter
    drops them and the samples keep the file's record numbers."""
    low = k16.copy()
    low[::997, 2] = np.float32(-7.5)
    return low


def run(ref, orc, pts, n, rng, tag):
    want = ref.fps(pts, n, rng)
    got = orc.fps(pts, n, rng)
    if not np.array_equal(want, got):
        raise SystemExit(f"{tag}: restatement and reference differ")
    return want


def cmp_flow(ref, orc, p, n, tag):
    rows = np.flatnonzero(p[:, 2] >= np.float32(-5.0))
    kept = np.ascontiguousarray(p[rows])
    rng = rng_of(kept, 1e-6)
    return rows[run(ref, orc, kept, n, rng, tag)].astype(np.int64), rng, len(kept)


def main():
    ref, orc = Reference(), Oracle()
    k16 = read(os.path.join(DATA, "16k_000000.bin"), 4)
    z = {"k16_xyz": k16}
    for name, pts, ns in (("k16", k16, (100, 1024, 4096)), ("lowz", lowz(k16), (1024,))):
        for n in ns:
            out, rng, _ = cmp_flow(ref, orc, pts, n, f"{name}_cmp_{n}")
            z[f"{name}_cmp_{n}__n"] = np.array(n, np.int64)
            z[f"{name}_cmp_{n}__range"] = np.array(rng, np.float64)
            z[f"{name}_cmp_{n}__expected"] = out
            print(f"{name}_cmp_{n}: {len(out)} samples", flush=True)
    rng = rng_of(k16, 0.0)
    z["k16_ex_1024__n"] = np.array(1024, np.int64)
    z["k16_ex_1024__range"] = np.array(rng, np.float64)
    z["k16_ex_1024__expected"] = run(ref, orc, k16, 1024, rng, "k16_ex_1024").astype(np.int64)
    np.savez_compressed(os.path.join(HERE, "kitti.npz"), **z)

    frames = {}
    for f in range(6):
        name = f"{f:06d}.bin"
        path = os.path.join(DATA, name)
        p = read(path, 4)
        rec = {"file_sha256": sha(open(path, "rb").read()), "points": int(len(p))}
        for n in (1024, 16384):
            out, rng, kept = cmp_flow(ref, orc, p, n, f"{name}_{n}")
            rec["kept"] = kept
            rec["range"] = list(rng)
            rec[str(n)] = {"len": int(len(out)), "sha256": sha(out.astype(np.int64).tobytes()),
                           "head": [int(v) for v in out[:8]]}
            print(f"{name} n={n}: kept {kept}, {len(out)} samples", flush=True)
        frames[name] = rec
    with open(os.path.join(HERE, "kitti.json"), "w") as fh:
        json.dump(frames, fh, indent=1)


if __name__ == "__main__":
    main()
