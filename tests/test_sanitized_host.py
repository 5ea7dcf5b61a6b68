"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only):
midman-ai_amd/build_sanitized.py builds the library's host-only sources and
the oracle with -fsanitize=address,undefined (every report fatal) and runs the
host test files against those builds: the safetensors reader on the
reference's fixtures, every truncation and bit flip, lying sizes; token
shards, sequences and the batcher; the schedule; the oracle's pins. The
reference runs its C-ABI consumer the same way
(.github/workflows/midman-api-ffi.yml:170-204)."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "midman-ai_amd", "build_sanitized.py")


@pytest.mark.slow
def test_host_code_is_clean_under_asan_and_ubsan():
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("no g++/make")
    b = subprocess.run([sys.executable, SCRIPT, "build"], cwd=ROOT, capture_output=True,
                       text=True, timeout=600)
    assert b.returncode == 0, b.stdout + b.stderr
    r = subprocess.run([sys.executable, SCRIPT, "run"], cwd=ROOT, capture_output=True,
                       text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "runtime error" not in out and "ERROR: AddressSanitizer" not in out
    assert " passed" in out, out[-2000:]
