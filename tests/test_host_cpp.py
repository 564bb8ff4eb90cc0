"""Runs the C++ host-layer tests (tests/cpp/host_tests.cpp) one case per
pytest item.  Cases named gpu_* drive the gfx950 library through the C ABI
and are marked gpu; the others are host logic and run on the CPU."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "cpp", "_build", "host_tests")


def _ensure_built() -> None:
    if not os.path.exists(BINARY):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)


def _cases():
    _ensure_built()
    out = subprocess.run([BINARY, "--list"], check=True, capture_output=True, text=True).stdout
    names = [n for n in out.split() if n]
    return [pytest.param(n, marks=pytest.mark.gpu) if n.startswith("gpu_") else n for n in names]


@pytest.mark.parametrize("case", _cases())
def test_host_cpp(case):
    r = subprocess.run([BINARY, case], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"PASS {case}" in r.stdout
