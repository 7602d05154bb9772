"""Pre-tuned hipBLASLt / rocBLAS solution choices for the projection GEMMs.

The decoder layer's q|k|v, o, gate|up and down projections (and their
backward GEMMs) run through torch.mm / torch.addmm, i.e. hipBLASLt.  Its
default heuristic does not always pick the fastest solution for these shapes
on gfx950; ``tunableop_gfx950.csv`` records, per GEMM shape, the solution
PyTorch's TunableOp measured fastest on an MI355X for the Llama-2-7B layer
(bf16, 4096 tokens), tuned with a 1 GiB rotating input buffer so that the
operands are not cache-resident, as in a stage step.  ``use_tuned_gemms()`` loads that table with tuning
switched OFF, so nothing is benchmarked at run time; shapes not in the table
use the library default.  The table is validated by TunableOp against the
torch / HIP / hipBLASLt versions it was recorded with and ignored on a
mismatch.
"""
from __future__ import annotations

import os

TUNED_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tunableop_gfx950.csv")


def use_tuned_gemms(enable: bool = True) -> bool:
    """Enable (or disable) the recorded GEMM solutions; returns whether the
    table was loaded."""
    import torch.cuda.tunable as tun
    if not enable:
        tun.enable(False)
        return False
    tun.enable(True)
    tun.tuning_enable(False)
    tun.record_untuned_enable(False)
    return bool(tun.read_file(TUNED_FILE))
