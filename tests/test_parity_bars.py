"""The parity bars have teeth -- CPU only.

The GPU tests hold the kernels to two bars: the north-star bar against the
f64 oracle (2e-2 of max|ref| in bf16) and a tight bar against the oracle with
the GPU path's storage roundings (_gpu.TIGHT).  Here one lost 16-byte operand
fragment of one gate/up MFMA block (8 of the 1024 input columns missing from
16 of the 8192 hidden units, for every row) is planted in the oracle (on the CPU) and offered as if it
were the GPU's output: the tight bar must reject it, the loose one lets it
through -- the reason the tight bar exists.
"""
import numpy as np

import oracle as O
from _common import rounded, small_case
from _gpu import TIGHT, TOL, rel_err, tight_metrics
from nomas_moe import workloads as wl


def test_tight_bar_catches_a_lost_fragment_the_loose_bar_misses():
    rows, D, E, k, H = 64, 1024, 4, 2, 8192  # the headline hidden: 256 k steps of 32
    t, x = small_case(rows, D, E, k, H, 31, bias=False)
    rt, rx = rounded(t, x, "bf16")
    p, _ = wl.oracle_params(rt, E)
    ref = O.forward_sparse_rounded(rx, p, k, "bf16")
    f64, _, _, _ = O.forward_sparse(rx, p, k)
    try:
        O.set_mutation(O.KERNEL_FAULTS["gate_up_loses_fragment"])
        planted = O.forward_sparse_rounded(rx, p, k, "bf16")
    finally:
        O.set_mutation(0)
    loose = rel_err(planted, f64)
    m, r = tight_metrics(planted, ref)
    print(f"lost fragment: vs f64 {loose:.3e} (bar {TOL['bf16']}), vs rounded max {m:.3e}, "
          f"worst row rms {r:.3e} (bars {TIGHT['bf16']})")
    assert loose <= TOL["bf16"]                       # passes the north-star bar ...
    assert m > TIGHT["bf16"][0] or r > TIGHT["bf16"][1]  # ... but not the tight one
    # and the unplanted output passes both
    assert rel_err(ref, f64) <= TOL["bf16"]
    m0, r0 = tight_metrics(ref, ref)
    assert m0 == 0 and r0 == 0
