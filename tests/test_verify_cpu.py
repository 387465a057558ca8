"""The verify module's CPU parts: the dp4a definition, the weight values, exact int dots, the bit-identical rebuild, the
per-output bound and the report line grammar (src/komp/verify.py:37-41, 94-120, 145-149)."""

import random

import numpy as np
import pytest

from comp_amd import host, verify
from oracle import oracle as O


def test_dp4a_expected_matches_oracle():
    rng = np.random.default_rng(0)
    a, b, c = (rng.integers(-(2**31), 2**31, size=2000).astype(np.int32) for _ in range(3))
    a[:10] = np.asarray(verify.DP4A_EDGE_WORDS, np.int64).astype(np.int32)
    assert np.array_equal(verify.dp4a_expected(a, b, c), O.dp4a(a, b, c))


@pytest.mark.parametrize("fmt,n,k,m", [("q4_0", 37, 416, 3), ("tq2_0", 29, 1792, 3)])
@pytest.mark.parametrize("extreme", [False, True])
def test_output_bound_is_the_oracles(fmt, n, k, m, extreme):
    """verify's per-output bound (the product package cannot import the oracle) equals oracle.output_error_bound."""
    from kurn.gpu import ref

    W, x = ref.problem(fmt, n, k, m, 3 + extreme, extreme)
    xq, xd, _ = O.quantize(fmt, x)
    wq, ws = host.split(fmt, W, n, k)
    s = O.block_dots(fmt, wq, xq, n, k)
    got = verify._output_bound(fmt, W, host.act_blocks(fmt, xq, xd), s, n, m)
    assert np.allclose(got, O.output_error_bound(fmt, ws, xd, s), rtol=1e-12, atol=0)


def test_weight_values_are_the_oracles():
    from kurn.gpu import ref

    for fmt, k in (("q4_0", 416), ("tq2_0", 768)):
        W = ref.weights(fmt, random.Random(4), 9, k, True)
        v = verify.weight_values(fmt, W).reshape(9, k)
        assert np.array_equal(v, O.weight_values(fmt, O.split(fmt, W, 9, k)[0], 9, k))


@pytest.mark.parametrize("fmt,n,k,m", [("q4_0", 37, 416, 3), ("tq2_0", 5, 1280, 2)])
@pytest.mark.parametrize("extreme", [False, True])
def test_exact_idots_rebuild_and_reference(fmt, n, k, m, extreme):
    from kurn.gpu import ref

    W, x = ref.problem(fmt, n, k, m, 1 + extreme, extreme)
    xq, xd, xb = O.quantize(fmt, x)
    s = verify.exact_idots(fmt, W, xq, n, k)
    wq, ws = host.split(fmt, W, n, k)
    assert np.array_equal(s, O.block_dots(fmt, wq, xq, n, k))
    xblocks = host.act_blocks(fmt, xq, xd)
    assert xblocks == ref.act_blocks(fmt, x)
    rf = ref.reference(fmt, W, xblocks, n, k, m)
    assert verify.rebuild_reference(fmt, W, xblocks, s, n, k, m) == list(rf)
    assert np.array_equal(np.asarray(rf).reshape(m, n), O.reference_dot(fmt, ws, xd, s))
    # one wrong block dot (in a block whose scale product is nonzero) changes the rebuilt reference
    dwx = O.f16_bits_to_f32(ws)[None, :, :].astype(np.float64) * xd[:, None, :].astype(np.float64)
    i, r, b = np.unravel_index(np.argmax(np.abs(dwx)), dwx.shape)
    s2 = s.copy()
    s2[i, r, b] += 1000
    assert verify.rebuild_reference(fmt, W, xblocks, s2, n, k, m) != list(rf)


def test_line_grammar():
    r = {"fmt": "q4_0", "n": 64, "k": 512, "m": 1, "quant": True, "idots": True, "rebuilt": True, "relerr": 1.234e-7,
         "ok": True}  # fmt: skip
    assert verify.line(r, 32, 4, 4, 2) == ("ok   q4_0  gemv dp4a-sdot4    block_n=32 nb=4 warps=4 n=64 k=512 m=1 "
                                           "quant=exact idots=exact reference_dot=bit-identical relerr=1.2e-07")  # fmt: skip
    r.update(ok=False, quant=False, rebuilt=False)
    assert verify.line(r, 32, 4, 4, 0).startswith("FAIL q4_0  gemv bytes") and "MISMATCH" in verify.line(r, 32, 4, 4, 0)


def test_run_all_check_count():
    assert 1 + 4 + 2 * 3 * len(verify.CONFIGS["q4_0"]) * len(verify.PROBLEMS["q4_0"]) * 2 == 113


def test_check_gemv_needs_a_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("device present")
    with pytest.raises(RuntimeError, match="HIP device"):
        verify.check_gemv("q4_0", 5, 96, 2)
