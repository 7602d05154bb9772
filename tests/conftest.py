"""Shared fixtures.  ``gpu`` marks tests that need an MI355X and the built
HIP library; everything else runs on the CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU and libzorse_amd.so")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from zorse_amd import _abi
    _abi.lib()  # raises if the library is missing: GPU tests never run without it
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter):
    """Which bound each 16-bit loss check passed under, and how many matched
    checks fell back to the reference layer's own error for the scaled bar
    (tests/_tol.py)."""
    try:
        from tests._tol import RECORDS
    except ImportError:
        return
    if not RECORDS:
        return
    tr = terminalreporter
    losses = [r for r in RECORDS if r["kind"] == "loss"]
    matched = [r for r in RECORDS if r["kind"] == "matched"]
    tr.write_sep("-", "tolerance record (tests/_tol.py)")
    literal = sum(r["bound"].startswith("1e-3") for r in losses)
    tr.write_line(f"loss checks: {len(losses)}, within the literal 1e-3: {literal}")
    for r in losses:
        if not r["bound"].startswith("1e-3"):
            tr.write_line(f"  {r['what']}: rel err {r['rel_err']:.2e} (reference layer "
                          f"{r['rel_err_reference_layer']:.2e}) passes under: {r['bound']}")
    own = [r for r in matched if r["scaled_bar"] != "2e-2 scaled"]
    tr.write_line(f"precision-matched checks: {len(matched)}, scaled bar within 1.5x of the "
                  f"reference layer's own error (matched bar applied): {len(own)}")
    for r in own:
        tr.write_line(f"  {r['what']}: hip {r['diff']:.3e}, reference layer {r['low']:.3e}, "
                      f"max|ref| {r['scale']:.3e}")
