"""The C restatement of the oracle (oracle/oracle.c) and the numpy one (oracle/oracle.py) agree exactly: quantizer
bytes, exact block dots, the f64 block-order reference; the C f32 GEMV (the kernels' arithmetic) is within 1e-5."""

import numpy as np
import pytest

from oracle import coracle as C
from oracle import oracle as O


def test_f16_conversions_all_patterns():
    lib = C.lib()
    for b in range(0, 65536, 7):
        f = float(O.f16_bits_to_f32(np.array([b], np.uint16).view(np.int16))[0])
        g = lib.oracle_f16_to_f32(b)
        assert (np.isnan(f) and np.isnan(g)) or f == g
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 3e4, 5000), rng.normal(0, 1e-5, 5000),
                         [65504, 65519, 65520, 65536, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0]]).astype(np.float32)  # fmt: skip
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([lib.oracle_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("extreme", [False, True])
def test_quantizers_agree(extreme):
    rng = np.random.default_rng(1 + extreme)
    x = O.activations(rng, 256 * 12, 3, block=32, extreme=extreme, outliers=0.02)
    q, d = C.quant_q8_0(x)
    rq, rd = O.quant_q8_0(x)
    assert np.array_equal(q, rq) and np.array_equal(d.view(np.uint32), rd.view(np.uint32))
    x = O.activations(rng, 256 * 12, 3, block=256, extreme=extreme, outliers=0.02)
    q, d, b = C.quant_q8_K(x)
    rq, rd, rb = O.quant_q8_K(x)
    assert np.array_equal(q, rq) and np.array_equal(d.view(np.uint32), rd.view(np.uint32)) and np.array_equal(b, rb)


@pytest.mark.parametrize("fmt,n,k,m", [("q4_0", 37, 416, 3), ("q4_0", 64, 4096, 1), ("tq2_0", 37, 768, 3),
                                       ("tq2_0", 19, 2816, 2)])  # fmt: skip
@pytest.mark.parametrize("extreme", [False, True])
def test_gemv_references_agree(fmt, n, k, m, extreme):
    W, x = O.problem(fmt, n, k, m, 5 + extreme, extreme)
    wq, ws = O.split(fmt, W, n, k)
    xq, xd, _ = O.quantize(fmt, x)
    s = C.block_dots(fmt, wq, xq, n, k)
    assert np.array_equal(s, O.block_dots(fmt, wq, xq, n, k))
    r = C.reference_dot(fmt, ws, xd, s)
    assert np.array_equal(r, O.reference_dot(fmt, ws, xd, s))
    y = C.gemv_f32(fmt, wq, ws, xq, xd, n, k)
    assert O.output_check(fmt, y, ws, xd, s, r)[0]  # the C f32 evaluation stays within the per-output bound
