"""The exact RMSNorm's shortcut, pinned on the CPU.

The exact-mode norm kernels sum the squares in parallel and keep that sum
only when every value within 4*(n+4)*2^-53 of it, relatively, gives the same
float(ss/n); otherwise they run the reference's serial chain
(sml/sml-run.c:147-152). Here the rule is checked against the serial chain
itself: on random vectors of every norm width the rule's float is the
chain's whenever the rule gives one, and on vectors built so that the chain
ends on a rounding midpoint the rule refuses (and a tree sum alone would
have rounded the other way)."""
import numpy as np
import pytest

import norm_cases as nc
from oracle import bind as ob


@pytest.mark.parametrize("n", [64, 1536, 4096, 8960, 14336])
def test_window_agrees_with_serial_chain(n):
    rng = np.random.default_rng(n)
    kept = 0
    for trial in range(300):
        scale = np.float32(10.0 ** rng.uniform(-3, 3))
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        if trial % 3 == 0:
            x[rng.integers(0, n)] *= np.float32(1e3)   # one dominant element
        got = nc.mean_alike(nc.tree_ss(x), n)
        want = np.float32(nc.serial_ss(x) / n)
        if got is not None:
            kept += 1
            assert got == want, (n, trial)
    assert kept >= 295                                 # the serial chain is rare


@pytest.mark.parametrize("n", [1536, 4096, 8960, 14336])
def test_boundary_vectors_fall_back(n):
    x = nc.boundary_vector(n, np.random.default_rng(n + 1))
    ss, ts = nc.serial_ss(x), nc.tree_ss(x)
    assert np.float32(ss / n) != np.float32(ts / n)    # the orders disagree
    assert nc.mean_alike(ts, n) is None                # so the rule refuses
    # and the oracle's chain is the serial one
    w = np.ones(n, np.float32)
    out = np.zeros(n, np.float32)
    ob.oracle().orc_rms_norm(out.ctypes.data, x.ctypes.data, w.ctypes.data, n, np.float32(0.0))
    sc = np.float32(1) / np.sqrt(np.float32(ss / n))
    assert out[0] == x[0] * sc
