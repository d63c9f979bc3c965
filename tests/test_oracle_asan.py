"""The oracle under AddressSanitizer and UBSan (CPU).

`make -C oracle asan` builds the same oracle.c with -fsanitize=address,undefined into
oracle/_asan/liboracle.so.  This test runs the oracle's pin tests (reference golden vectors,
the float64 / closed-form pins, the HLO host ops) and the chained-runtime checks in a child
Python with libasan preloaded and SHP_ORACLE_LIB pointing at that build; any out-of-bounds
access, use after free or undefined behaviour in the oracle aborts the child and fails here.
Leak checking is off: the child is a whole Python interpreter."""
import os
import pathlib
import shutil
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def _libasan():
    gcc = shutil.which("gcc")
    if gcc is None:
        return None
    p = subprocess.run([gcc, "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = p.stdout.strip()
    return path if path and os.path.isabs(path) and os.path.exists(path) else None


def test_oracle_pins_under_asan_and_ubsan():
    asan = _libasan()
    if asan is None:
        pytest.skip("gcc's libasan is not available")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"], check=True)
    env = dict(os.environ, LD_PRELOAD=asan, SHP_ORACLE_LIB=str(ROOT / "oracle/_asan/liboracle.so"),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
           "tests/test_oracle_golden.py", "tests/test_oracle_math.py",
           "tests/test_oracle_hlo_ops.py", "tests/test_chained_run.py"]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, tail
    print(r.stdout.strip().splitlines()[-1])
