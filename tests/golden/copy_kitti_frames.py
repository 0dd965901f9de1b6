"""Copies the reference's six full KITTI frames (eval/kitti_data/000000.bin ..
000005.bin, about 12 MB) into tests/golden/kitti_frames/, checking each
against the SHA-256 recorded in tests/golden/kitti.json.

The frames are input data of the reference's own evaluation; they are too
large to keep in the repository's history, so the directory is git-ignored
but travels with the working tree to the machine that runs the GPU tests
(test_kitti.py's full-frame test reads it).  __graft_entry__.build() runs
this script where the reference tree is present.

Usage: python tests/golden/copy_kitti_frames.py [SOURCE_DIR]
"""

import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
DEST = os.path.join(HERE, "kitti_frames")
DEFAULT_SOURCE = "/root/reference/eval/kitti_data"


def main(src=DEFAULT_SOURCE):
    with open(os.path.join(HERE, "kitti.json")) as f:
        frames = json.load(f)
    if not os.path.isdir(src):
        print(f"no KITTI source directory at {src}; nothing copied")
        return 0
    os.makedirs(DEST, exist_ok=True)
    copied = 0
    for name, rec in sorted(frames.items()):
        dst = os.path.join(DEST, name)
        if os.path.exists(dst):
            with open(dst, "rb") as fh:
                if hashlib.sha256(fh.read()).hexdigest() == rec["file_sha256"]:
                    continue
        with open(os.path.join(src, name), "rb") as fh:
            data = fh.read()
        if hashlib.sha256(data).hexdigest() != rec["file_sha256"]:
            raise RuntimeError(f"{name}: SHA-256 differs from tests/golden/kitti.json")
        tmp = dst + ".tmp"
        with open(tmp, "wb") as fh:
            fh.write(data)
        os.replace(tmp, dst)
        copied += 1
    print(f"KITTI frames in {DEST}: {len(frames)} ({copied} copied)")
    return 0


if __name__ == "__main__":
    sys.exit(main(*sys.argv[1:]))
