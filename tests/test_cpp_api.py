"""The reference's own Rust tests, restated in C++ against include/spissa.hpp
(tests/cpp/reference_tests.cpp), run through the C ABI. The host-only subset
(argument validation, pure functions) runs on the CPU; the full set is marked
gpu."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BIN = ROOT / "tests" / "cpp" / "_build" / "reference_tests"
LIB = ROOT / "spissa_amd" / "_lib" / "libspissa_hip.so"


def _run(*args: str) -> subprocess.CompletedProcess:
    res = subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=110)
    print(res.stdout, res.stderr, flush=True)
    return res


def test_cpp_reference_tests_host_only():
    if not BIN.exists():
        if not LIB.exists():
            pytest.skip("libspissa_hip.so is not built (python -m spissa_amd.build)")
        subprocess.run(["make", "-s", "-C", str(ROOT / "tests" / "cpp")], check=True)
    res = _run("--host")
    assert res.returncode == 0, res.stdout
    assert "test result: ok" in res.stdout


@pytest.mark.gpu
def test_cpp_reference_tests_on_gpu(gpu):
    assert BIN.exists(), f"{BIN} is not built (make -C tests/cpp)"
    listed = [l for l in _run("--list").stdout.splitlines() if l.strip()]
    res = _run()
    assert res.returncode == 0, res.stdout
    assert f"test result: ok. {len(listed)} passed; 0 failed" in res.stdout
