import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "vk-shei_amd"), os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_terminal_summary(terminalreporter):
    """Per-check error of GPU outputs against the oracle (max abs and BF16 ulp
    distance), collected by _data.check_bf16."""
    from _data import ERROR_LEDGER

    if not ERROR_LEDGER:
        return
    tr = terminalreporter
    from _data import ULP_FLOOR

    tr.write_sep("-", f"BF16 outputs against the oracle: max abs; ulp distance where |ref| >= {ULP_FLOOR}")
    by_label = {}
    for label, n, err, nbig, umax, over in ERROR_LEDGER:
        e = by_label.setdefault(label, [0, 0.0, 0, 0, 0])
        e[0] += n
        e[1] = max(e[1], err)
        e[2] += nbig
        e[3] = max(e[3], umax)
        e[4] += over
    for label, (n, err, nbig, umax, over) in by_label.items():
        tr.write_line(f"{label:56s} n={n:9d} max abs {err:.4g} | n={nbig:8d} max ulp {umax} >1 ulp {over}")


@pytest.fixture(scope="session")
def ctx():
    """One gfx950 context on torch's current stream for the whole GPU session."""
    import torch
    import mslim_attn

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = mslim_attn.Context()
    c.use_torch_stream()
    yield c
    c.synchronize()
    c.close()
