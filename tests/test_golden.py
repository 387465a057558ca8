"""The oracle against the committed golden vectors (expected values from exact arithmetic and brute force)."""

import numpy as np

from oracle import oracle as O
from tests.golden import fixtures as G

V = G.load()


def test_q8_0_golden():
    x = np.stack([G.f32(b) for b in V["q8_0"]["x_bits"]]).reshape(1, -1)
    xq, xd = O.quant_q8_0(x)
    assert np.array_equal(xq.reshape(-1, 32).astype(int), np.asarray(V["q8_0"]["q"]))
    assert np.array_equal(xd.reshape(-1).view(np.uint32), np.asarray(V["q8_0"]["d_bits"], np.uint32))


def test_q8_K_golden():
    x = np.stack([G.f32(b) for b in V["q8_K"]["x_bits"]]).reshape(1, -1)
    xq, xd, xb = O.quant_q8_K(x)
    assert np.array_equal(xq.reshape(-1, 256).astype(int), np.asarray(V["q8_K"]["q"]))
    assert np.array_equal(xd.reshape(-1).view(np.uint32), np.asarray(V["q8_K"]["d_bits"], np.uint32))
    assert np.array_equal(xb.reshape(-1, 16).astype(int), np.asarray(V["q8_K"]["bsums"]))


def test_dp4a_golden():
    t = np.asarray(V["dp4a"], np.int64)
    assert np.array_equal(O.dp4a(t[:, 0], t[:, 1], t[:, 2]).astype(np.int64), t[:, 3])


def test_gemv_golden():
    for c in V["gemv"]:
        fmt, n, k, m, W, xq, xd, S, Y = G.gemv_case(c)
        wq, ws = O.split(fmt, W, n, k)
        r, s = O.gemv(fmt, wq, ws, xq, xd, n, k)
        assert np.array_equal(s, S)
        assert np.array_equal(r, Y)  # same f64 operations in the same order: bit-identical
