"""The oracle's own test suites against its AddressSanitizer +
UndefinedBehaviorSanitizer build (oracle/Makefile `asan`, gcc, CPU only).

The oracle is the checker every parity claim rests on, so an out-of-bounds
read or an undefined operation inside it would make those claims unsound.
This runs the oracle KATs, property tests and golden fixtures in a child
process with the sanitizer runtime preloaded; any report fails the test.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SUITES = ["tests/test_oracle_kat.py", "tests/test_oracle_properties.py", "tests/test_golden.py",
          "tests/test_oracle_linear.py", "tests/test_oracle_lm_head.py"]


def runtime(name: str) -> str:
    out = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else ""


def test_oracle_suites_are_clean_under_asan_and_ubsan():
    asan = runtime("libasan.so")
    if not asan:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"], check=True)
    lib = ROOT / "oracle" / "_build" / "libspissa_oracle_asan.so"
    assert lib.exists()
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": asan,
        "SPISSA_ORACLE_LIB": str(lib),
        # the interpreter itself is not instrumented: report only the oracle's errors
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *SUITES],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = res.stdout + res.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert res.returncode == 0, out[-4000:]
    assert " passed" in res.stdout
