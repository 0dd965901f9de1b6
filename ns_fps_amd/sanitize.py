"""Runs the host library's CPU tests under AddressSanitizer and
UndefinedBehaviorSanitizer.

    python -m ns_fps_amd.sanitize [--no-build] [pytest arguments]

Builds (unless --no-build) the library and the module with sanitized host
code into _build/sanitize/ (ns_fps_amd/build.py: build_sanitized), then runs
pytest in a child process with clang's sanitizer runtime preloaded,
NSFPS_LIB / NSFPS_MODULE naming the sanitized builds, and every sanitizer
report fatal.  By default it runs the CPU tests that drive the host library
(range derivation and thresholds, compute_bbox on the worker pool including
a fork, argument checks and error statuses, the module's surface, guards and
conversions); without a GPU the compute calls end at the device check, with
one they run too.  Exits with pytest's status; a sanitizer report aborts the
test process and fails the run.
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
DEFAULT_TESTS = ["tests/test_host_api.py", "tests/test_dropin.py", "tests/test_bench_cli.py",
                 "tests/test_plan.py", "tests/test_device_bbox.py",
                 "tests/test_failure_injection.py"]


def runtime_path():
    """clang's ASan runtime (it carries the UBSan handlers too)."""
    for clang in ("/opt/rocm/llvm/bin/clang", "clang"):
        try:
            p = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"],
                               stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True)
        except OSError:
            continue
        path = p.stdout.strip()
        if p.returncode == 0 and os.path.isabs(path) and os.path.exists(path):
            return path
    raise RuntimeError("clang's AddressSanitizer runtime (libclang_rt.asan-x86_64.so) not found")


REPORTS = os.path.join(ROOT, "_build", "sanitize", "reports")


def sanitized_env():
    from ns_fps_amd import build as b
    lib = os.path.join(b.SAN_DIR, "ns_fps_amd", "libnsfps.so")
    mod = os.path.join(b.SAN_DIR, "yuezu_fps", os.path.basename(b.module_path()))
    for f in (lib, mod):
        if not os.path.exists(f):
            raise RuntimeError(f"{f} is missing: run python -m ns_fps_amd.build sanitize")
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": runtime_path(),
        "NSFPS_LIB": lib,
        "NSFPS_MODULE": mod,
        # the interpreter itself is not instrumented: its allocations at exit
        # are not ours to report; every report from our code is fatal.
        # Reports go to files (pytest captures the test's stderr, and an
        # aborted test process would lose it).
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1:"
                        f"detect_odr_violation=0:log_path={REPORTS}/asan",
        "UBSAN_OPTIONS": f"halt_on_error=1:print_stacktrace=1:log_path={REPORTS}/ubsan",
    })
    return env


def reports():
    """The sanitizer reports the last run wrote (file name, text)."""
    if not os.path.isdir(REPORTS):
        return []
    out = []
    for f in sorted(os.listdir(REPORTS)):
        with open(os.path.join(REPORTS, f), errors="replace") as fh:
            out.append((f, fh.read()))
    return out


def run(pytest_args=(), build=True):
    if build:
        from ns_fps_amd import build as b
        b.build_sanitized()
    args = list(pytest_args) or ["-m", "not gpu", *DEFAULT_TESTS]
    os.makedirs(REPORTS, exist_ok=True)
    for f in os.listdir(REPORTS):
        os.remove(os.path.join(REPORTS, f))
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", *args]
    p = subprocess.run(cmd, cwd=ROOT, env=sanitized_env(), stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True)
    return p.returncode, p.stdout


def main(argv):
    build = "--no-build" not in argv
    args = [a for a in argv if a != "--no-build"]
    rc, out = run(args, build)
    print(out, end="")
    found = reports()
    for name, text in found:
        print(f"---- sanitizer report {name}:\n{text[:4000]}")
    return (rc or 1) if found else rc


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
