"""Runs the C++ host-layer tests (tests/cpp/host_tests.cpp, the portable
backend and kernel configuration; tests/cpp/store_tests.cpp, the ColdStore
and region store) one case per pytest item.  Cases named gpu_* drive the gfx950 library through the C ABI
and are marked gpu; the others are host logic and run on the CPU."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BINARIES = [os.path.join(HERE, "cpp", "_build", name) for name in ("host_tests", "store_tests")]


def _ensure_built() -> None:
    # make is a no-op when the binaries are newer than their sources.
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)


def _cases():
    _ensure_built()
    cases = []
    for binary in BINARIES:
        out = subprocess.run([binary, "--list"], check=True, capture_output=True, text=True).stdout
        for name in out.split():
            param = (os.path.basename(binary), name)
            marks = [pytest.mark.gpu] if name.startswith("gpu_") else []
            cases.append(pytest.param(*param, marks=marks, id=f"{param[0]}:{name}"))
    return cases


@pytest.mark.parametrize("binary,case", _cases())
def test_host_cpp(binary, case):
    r = subprocess.run([os.path.join(HERE, "cpp", "_build", binary), case], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"PASS {case}" in r.stdout
