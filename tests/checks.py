"""The output gate of the GPU tests: every f32 output within the f32 error bound of the f64 reference, and the
norm-wise relative error within the reference's 1e-5 rule."""

import numpy as np

from oracle import oracle as O

# the reference's f32 output rule: relerr(Y, reference) <= 1e-5 (src/komp/verify.py:28, :135-137)
TOL = 1e-5


def gate(fmt, y, ws, xd, s, r, tol=TOL):
    """(ok, message).  ok when both halves of the gate hold:
      * every output of y lies within oracle.output_error_bound of the f64 reference r, computed from the exact block
        dots s, the weight scale plane ws and the activation scales xd the kernel used;
      * the norm-wise relative error, max|y - r| / max|r| (oracle.relerr) and ||y - r|| / ||r|| (oracle.relerr2), is at
        most tol.
    The bound alone grows with the block count (at 448 Q4_0 blocks a row it admits about 2e-4 norm-wise), so the
    second half is what holds long rows to the reference's rule; the first is what holds small outputs next to a large
    one.  message names the worst output and the relative error."""
    y = np.asarray(y, dtype=np.float64)
    r64 = np.asarray(r, dtype=np.float64).reshape(y.shape)
    bound_ok, worst = O.output_check(fmt, y, ws, xd, s, r)
    # both norm-wise forms: KURN's relerr is one of them (tests/test_relerr_form.py), whichever norm it takes
    err = max(O.relerr(y, r64), O.relerr2(y, r64))
    rel_ok = bool(err <= tol)
    if bound_ok and rel_ok:
        return True, f"{fmt}: worst output {worst:.3g} of its bound, relerr {err:.2e}"
    bound = O.output_error_bound(fmt, ws, xd, s).reshape(y.shape)
    dev = np.abs(y - r64)
    dev = np.where(np.isfinite(dev), dev, np.inf)
    i = np.unravel_index(int(np.argmax(dev - bound)), y.shape)
    why = [] if bound_ok else [f"an output past its bound ({worst:.3g} of it)"]
    why += [] if rel_ok else [f"relerr {err:.2e} > {tol:g}"]
    return False, (f"{fmt}: {' and '.join(why)}; output {i} = {y[i]!r}, reference {r64[i]!r}, bound {bound[i]:.3g}, "
                   f"relerr {err:.2e}")


def outputs_ok(fmt, y, ws, xd, s, r):
    """True when gate(...) holds; otherwise an AssertionError with its message."""
    ok, msg = gate(fmt, y, ws, xd, s, r)
    if not ok:
        raise AssertionError(msg)
    return True
