"""Builds the native parts in-tree (no JIT cache, nothing installed).

* ``ns_fps_amd/libnsfps.so`` -- HIP kernels (gfx950) + C++ host library
  behind the C ABI of include/nsfps.h, compiled by hipcc.
* ``yuezu_fps/yuezu_fps_module*.so`` -- the pybind11 module under the
  reference's own import path (``import yuezu_fps.yuezu_fps_module as yf``),
  linked against libnsfps.so with an $ORIGIN-relative rpath.

* ``_build/sanitize/`` -- the same two, host code built with AddressSanitizer
  and UndefinedBehaviorSanitizer (device code as usual), for
  ``python -m ns_fps_amd.sanitize``, which runs the CPU tests of the host
  library under them.

Run ``python -m ns_fps_amd.build`` (or ``__graft_entry__.build()``);
``python -m ns_fps_amd.build sanitize`` builds the sanitized pair.
"""

import os
import re
import subprocess
import sys
import sysconfig
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
MODULE_DIR = os.path.join(ROOT, "yuezu_fps")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NSFPS_OFFLOAD_ARCH", "gfx950")

LIB = os.path.join(HERE, "libnsfps.so")
SOURCES = ("nsfps_build.hip", "nsfps_sample.hip", "nsfps_runs.hip", "nsfps_group.hip",
           "nsfps_host.cpp")

# Exact fp32: no contraction, IEEE division/sqrt, denormals kept.
# "-packed-fp32-ops" turns off the gfx950 packed fp32 instructions
# (v_pk_add/mul/fma_f32) in the device pass.  The same -Xclang pair also
# reaches hipcc's x86 host pass, which does not know the feature and prints
# "not a recognized feature" once per translation unit; the driver cannot
# forward an option with an argument to the device pass alone
# (-Xarch_device refuses it), so that host-pass warning is filtered from the
# build output and the device assembly is checked instead (check_no_packed_fp32).
# The backend's atomic optimizer is off: by default it turns an atomic whose
# address is the same in every lane into a loop over the active lanes (a
# read-lane and a scalar step each) ahead of one atomic, and in these kernels
# such atomics have few active lanes on the run kernel's critical path (the
# largest key left unaccepted, the lowered copies' masks and bounds).  With
# one LDS atomic per lane instead, per call on one MI355X, bit-exact: 1M-point
# uniform cube 7.20-7.22 -> 6.99-7.01 ms, quickstart 0.71 -> 0.65-0.66,
# LiDAR scan 3.91 -> 3.77-3.80, batched clouds 2.05 -> 1.93-1.98, clustered
# cloud 60.2-60.3 -> 59.5.  Its DPP form (a reduction across lanes in place of
# the loop) measured in between: uniform cube 7.16-7.23, quickstart 0.67-0.69.
# The machine scheduler favours instruction-level parallelism (max-ilp): the
# run kernel is latency-bound with two waves per SIMD.  Per call, two runs on
# each of two boxes, bit-exact, against the default strategy: uniform cube
# 7.01-7.02 -> 6.96-7.00 ms, LiDAR scan 3.77-3.79 -> 3.67-3.69, batched
# clouds 1.99-2.00 -> 1.89-1.94, clustered cloud 59.5-59.8 -> 58.3-58.6,
# quickstart 0.66-0.68 -> 0.65-0.66.  The others measured: max-memory-clause
# slower everywhere (uniform cube 7.04-7.05), iterative-ilp and
# iterative-maxocc in between (uniform cube 6.95-6.97 and 7.00-7.01,
# clustered 58.7 and 58.9-59.0).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-mllvm", "-amdgpu-sched-strategy=max-ilp",
    "-Wall", "-Wno-unused-result",
]
HOST_PASS_WARNING = "'-packed-fp32-ops' is not a recognized feature for this target"
PACKED_FP32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")


def _run(cmd, cwd=None):
    print("+", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = p.stdout.splitlines()
    kept = [ln for ln in lines if HOST_PASS_WARNING not in ln]
    if kept:
        print("\n".join(kept), flush=True)
    if len(kept) != len(lines):
        print(f"  ({len(lines) - len(kept)} host-pass notes about -packed-fp32-ops omitted; "
              "the device pass applies the feature)", flush=True)
    if p.returncode != 0:
        raise subprocess.CalledProcessError(p.returncode, cmd)


def check_no_packed_fp32(asm_dir):
    """Fails when the gfx950 assembly of this build holds a packed fp32
    add/mul/fma instruction."""
    found = []
    n_files = 0
    for name in sorted(os.listdir(asm_dir)):
        if not (name.endswith(".s") and f"amdgcn-amd-amdhsa-{ARCH}" in name):
            continue
        n_files += 1
        with open(os.path.join(asm_dir, name)) as f:
            for ln in f:
                if PACKED_FP32.search(ln):
                    found.append(f"{name}: {ln.strip()}")
    if n_files == 0:
        raise RuntimeError("no device assembly was written; cannot check for packed fp32")
    if found:
        raise RuntimeError("packed fp32 instructions in the device code:\n" + "\n".join(found[:20]))
    print(f"  device assembly of {n_files} translation units: no v_pk_add/mul/fma_f32", flush=True)


def module_path():
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(MODULE_DIR, "yuezu_fps_module" + suffix)


SAN_DIR = os.path.join(ROOT, "_build", "sanitize")
# host code only: each -fsanitize= right after -Xarch_host, device code unsanitized
SAN_HOST_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all",
                  "-fno-gpu-sanitize", "-g"]


def build_lib(out=LIB, extra=()):
    srcs = [os.path.join(CSRC, f) for f in SOURCES]
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    with tempfile.TemporaryDirectory(prefix="nsfps_build_") as td:
        # -save-temps keeps each translation unit's gfx950 assembly in td
        _run([HIPCC, *DEVICE_FLAGS, *extra, "-save-temps", "-shared", "-I", INCLUDE, "-I", CSRC,
              *srcs, "-o", tmp], cwd=td)
        check_no_packed_fp32(td)
    os.replace(tmp, out)
    return out


def build_module(out=None, lib_dir=HERE, cxx="g++", extra=()):
    import pybind11
    out = out or module_path()
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    pyinc = sysconfig.get_paths()["include"]
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", *extra,
          "-I", INCLUDE, "-I", pybind11.get_include(), "-I", pyinc,
          os.path.join(CSRC, "yuezu_fps_pybind.cpp"),
          "-L", lib_dir, "-lnsfps", "-Wl,-rpath,$ORIGIN/../ns_fps_amd", "-o", tmp])
    os.replace(tmp, out)
    if out == module_path():
        # an older build placed the module inside the package: remove it so
        # that only one copy of the bindings exists
        old = os.path.join(HERE, os.path.basename(out))
        if os.path.exists(old):
            os.remove(old)
    return out


def build_sanitized():
    """libnsfps.so and the module with ASan + UBSan host code, under
    _build/sanitize/ (ns_fps_amd/ and yuezu_fps/, as in the tree).  Both use
    clang's sanitizer runtime, which the process preloads."""
    lib = build_lib(os.path.join(SAN_DIR, "ns_fps_amd", "libnsfps.so"), SAN_HOST_FLAGS)
    clangxx = os.path.join(os.path.dirname(os.path.realpath(HIPCC)), "..", "llvm", "bin", "clang++")
    if not os.path.exists(clangxx):
        clangxx = "/opt/rocm/llvm/bin/clang++"
    mod = build_module(os.path.join(SAN_DIR, "yuezu_fps", os.path.basename(module_path())),
                       os.path.dirname(lib), clangxx,
                       ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        "-fno-omit-frame-pointer", "-shared-libasan", "-g"])
    return lib, mod


def build_all():
    build_lib()
    build_module()


if __name__ == "__main__":
    what = sys.argv[1:] or ["all"]
    for w in what:
        {"lib": build_lib, "module": build_module, "all": build_all,
         "sanitize": build_sanitized}[w]()
