"""Loader for tests/golden/vectors.json (written by make_golden.py)."""

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load():
    with open(os.path.join(HERE, "vectors.json")) as fh:
        return json.load(fh)


def f32(bits):
    return np.asarray(bits, dtype=np.uint32).view(np.float32)


def gemv_case(c):
    """-> (fmt, n, k, m, W bytes, xq int8 [m][k], xd f32 [m][nb], S int64 [m][n][nb], Y f64 [m][n])."""
    n, k, m = c["n"], c["k"], c["m"]
    xq = np.asarray(c["xq"], np.int8)
    xd = np.stack([f32(r) for r in c["xd_bits"]])
    S = np.asarray(c["S"], np.int64).reshape(m, n, -1)
    Y = np.asarray(c["Y"], np.float64).reshape(m, n)
    return c["fmt"], n, k, m, bytes.fromhex(c["W"]), xq, xd, S, Y
