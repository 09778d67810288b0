import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "bonsai-pot_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    torch.cuda.init()
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Per-config margins of the attention comparisons (max-abs against 2e-3,
    rel-L2 against 1e-3, and the f16-ulp distance from f16 of the oracle's f32
    result, which separates the kernel's own error from the f16 store's
    rounding), so the headroom to the bar is visible in every run."""
    try:
        from helpers import MARGINS, TOL_MAX_ABS, TOL_REL_L2, ULP_MIN_MAG
    except Exception:
        return
    if not MARGINS:
        return
    tr = terminalreporter
    tr.write_sep("-", f"attention margins ({len(MARGINS)} comparisons; bar max_abs {TOL_MAX_ABS}, rel_l2 {TOL_REL_L2})")
    for what, ma, rl, mu, n_off, n_big in MARGINS:
        tr.write_line(f"{what:60s} max_abs {ma:.2e} ({ma / TOL_MAX_ABS:5.1%} of bar)  "
                      f"rel_l2 {rl:.2e} ({rl / TOL_REL_L2:5.1%} of bar)  "
                      f"|out| >= {ULP_MIN_MAG}: max {mu} ulp from f16(oracle), {n_off} of {n_big} off")
    worst = max(MARGINS, key=lambda x: max(x[1] / TOL_MAX_ABS, x[2] / TOL_REL_L2))
    tr.write_line(f"worst: {worst[0]} at {max(worst[1] / TOL_MAX_ABS, worst[2] / TOL_REL_L2):.1%} of the bar")
    wu = max(MARGINS, key=lambda x: x[3])
    tr.write_line(f"largest distance from f16(oracle): {wu[3]} ulp ({wu[0]})")
