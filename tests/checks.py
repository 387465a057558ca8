"""The output gate of the GPU tests: every f32 output within the f32 error bound of the f64 reference."""

import numpy as np

from oracle import oracle as O


def outputs_ok(fmt, y, ws, xd, s, r):
    """True when every output of y lies within oracle.output_error_bound of the f64 reference r, computed from the
    exact block dots s, the weight scale plane ws and the activation scales xd the kernel used; otherwise an
    AssertionError naming the worst output (and the norm-wise relative error, which only reports)."""
    y = np.asarray(y, dtype=np.float64)
    ok, worst = O.output_check(fmt, y, ws, xd, s, r)
    if not ok:
        r = np.asarray(r, dtype=np.float64).reshape(y.shape)
        bound = O.output_error_bound(fmt, ws, xd, s).reshape(y.shape)
        i = np.unravel_index(int(np.argmax(np.abs(y - r) - bound)), y.shape)
        raise AssertionError(f"{fmt}: output {i} = {y[i]!r}, reference {r[i]!r}, bound {bound[i]:.3g} "
                             f"(worst {worst:.3g} of the bound; relerr {O.relerr(y, r):.2e})")
    return True
