"""Builds the native parts in-tree (no JIT cache, nothing installed).

* ``libnsfps.so`` -- HIP kernels (gfx950) + C++ host library behind the C ABI
  of include/nsfps.h, compiled by hipcc.
* ``yuezu_fps_module*.so`` -- the pybind11 module, linked against libnsfps.so
  with an $ORIGIN rpath.

Run ``python -m ns_fps_amd.build`` (or ``__graft_entry__.build()``).
"""

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NSFPS_OFFLOAD_ARCH", "gfx950")

LIB = os.path.join(HERE, "libnsfps.so")

# Exact fp32: no contraction, IEEE division/sqrt, denormals kept.  Packed fp32
# instructions are disabled for all device code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def module_path():
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(HERE, "yuezu_fps_module" + suffix)


def build_lib():
    srcs = [os.path.join(CSRC, f) for f in ("nsfps_build.hip", "nsfps_sample.hip", "nsfps_runs.hip", "nsfps_group.hip",
                                             "nsfps_host.cpp")]
    tmp = LIB + ".tmp"
    _run([HIPCC, *DEVICE_FLAGS, "-shared", "-I", INCLUDE, "-I", CSRC, *srcs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


def build_module():
    import pybind11
    out = module_path()
    tmp = out + ".tmp"
    pyinc = sysconfig.get_paths()["include"]
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          "-I", INCLUDE, "-I", pybind11.get_include(), "-I", pyinc,
          os.path.join(CSRC, "yuezu_fps_pybind.cpp"),
          "-L", HERE, "-lnsfps", "-Wl,-rpath,$ORIGIN", "-o", tmp])
    os.replace(tmp, out)
    return out


def build_all():
    build_lib()
    build_module()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for w in what:
        {"lib": build_lib, "module": build_module, "all": build_all}[w]()
