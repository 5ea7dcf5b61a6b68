"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

Builds the library's host-only sources (error handling, RNG and rotary
tables, SHA-256, the safetensors reader/writer, token shards and the batcher)
into midman-ai_amd/_build/asan/libmidman_host_asan.so, and the CPU oracle into
oracle/libmm_oracle_asan.so, both with g++/gcc -fsanitize=address,undefined
(no HIP code is involved: nothing here is compiled for the GPU). Then runs the
host test files against those builds: the Python bindings load them through
MMH_LIB_PATH and MM_ORACLE_LIB, with the ASan runtime preloaded into the
interpreter and every sanitizer report fatal.

    python midman-ai_amd/build_sanitized.py build
    python midman-ai_amd/build_sanitized.py run [pytest args...]

The reference runs its C-ABI consumer the same way under ASan and UBSan
(.github/workflows/midman-api-ffi.yml:170-204).
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build", "asan")
HOST_LIB = os.path.join(OUT_DIR, "libmidman_host_asan.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "libmm_oracle_asan.so")

SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
# The host test files: checkpoint reader/writer (bit flips, truncations, lying
# sizes), shards/sequences/batcher, schedule and optimizer host logic, and
# the oracle's own pins.
HOST_TESTS = ["tests/test_checkpoint_host.py", "tests/test_data_host.py",
              "tests/test_train_host.py", "tests/test_oracle.py", "tests/test_oracle_train.py"]


def _run(cmd, **kw):
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, **kw)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{p.stdout}")
    return p.stdout


def build() -> None:
    sys.path.insert(0, HERE)
    import build as pkg_build  # the same host source list as the product build

    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = [os.path.join(CSRC, s) for s in pkg_build.HOST_SOURCES]
    _run(["g++", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-Wall", "-Wextra",
          *SAN, "-o", HOST_LIB + ".tmp", *srcs, "-lpthread"])
    os.replace(HOST_LIB + ".tmp", HOST_LIB)
    _run(["make", "-B", "-C", ORACLE_DIR, "asan"])


def runtime_libraries() -> str:
    """The ASan runtime, and libstdc++ beside it: the interpreter does not
    link libstdc++, and ASan's exception interceptor finds the real
    __cxa_throw only if libstdc++ is loaded when ASan starts."""
    asan = _run(["g++", "-print-file-name=libasan.so"]).strip()
    cxx = _run(["g++", "-print-file-name=libstdc++.so.6"]).strip()
    return f"{asan} {cxx}"


def environment() -> dict:
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": runtime_libraries(),
        # CPython's own allocations are not freed at exit by design
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1:"
                        "detect_stack_use_after_return=1:strict_string_checks=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "MMH_LIB_PATH": HOST_LIB,
        "MM_ORACLE_LIB": ORACLE_LIB,
        "PYTHONDONTWRITEBYTECODE": "1",
    })
    return env


def run(extra=()) -> int:
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
           *HOST_TESTS, *extra]
    return subprocess.call(cmd, cwd=ROOT, env=environment())


def main():
    what = sys.argv[1] if len(sys.argv) > 1 else "build"
    if what == "build":
        build()
        print(HOST_LIB)
        print(ORACLE_LIB)
        return 0
    if what == "run":
        return run(sys.argv[2:])
    raise SystemExit(f"unknown command {what!r} (build | run)")


if __name__ == "__main__":
    sys.exit(main())
