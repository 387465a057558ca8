"""Pins of oracle.output_error_bound, the per-output gate of every device output.

Any f32 evaluation of a GEMV output (products of the exact block dot and the two scales, summed in any order) must
stay within the bound; plausible mistakes of a kernel (a shifted scale index, a dropped block, subnormal scales
flushed to zero, a flipped sign, another column's d_x) must break it.  The evaluations below are f32 simulations in
numpy, where every operation rounds to nearest-even as the GPU's do."""

import functools

import numpy as np
import pytest

from oracle import coracle as C
from oracle import oracle as O
from tests.checks import gate

FORMATS = ("q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k")
SHAPES = {"q4_0": (37, 416, 3), "q8_0": (37, 416, 3), "iq4_nl": (37, 416, 3), "tq2_0": (29, 1792, 3),
          "q4_k": (29, 1792, 3)}


def _problem(fmt, seed, extreme):
    n, k, m = SHAPES[fmt]
    W, x = O.problem(fmt, n, k, m, seed=seed, extreme=extreme)
    wq, ws = O.split(fmt, W, n, k)
    xq, xd, _ = O.quantize(fmt, x)
    r, s = O.gemv(fmt, wq, ws, xq, xd, n, k)
    return ws, xd, s, r


def _f32_terms(fmt, ws, xd, s, dw_shift=0, flip=None, col_shift=0, flush=False):
    """The f32 products of the device, [M][N][T] float32 (q4_k: two terms per block), with optional planted
    mistakes."""
    dx = np.asarray(xd, np.float32)
    if col_shift:
        dx = np.roll(dx, col_shift, axis=0)
    if fmt == "q4_k":
        meta = np.ascontiguousarray(ws, dtype=np.int16).reshape(ws.shape[0], -1, 8)
        d = O.f16_bits_to_f32(meta[:, :, 0])
        dmin = O.f16_bits_to_f32(meta[:, :, 1])
        if flush:
            d = np.where(np.abs(d) < 2.0**-14, np.float32(0), d)
            dmin = np.where(np.abs(dmin) < 2.0**-14, np.float32(0), dmin)
        d, dmin = np.roll(d, dw_shift, axis=1), np.roll(dmin, dw_shift, axis=1)
        sd = s[..., 0].astype(np.float32)
        sm = s[..., 1].astype(np.float32)
        t1 = sd * (d[None] * dx[:, None, :])
        t2 = -(sm * (dmin[None] * dx[:, None, :]))
        t = np.concatenate([t1, t2], axis=-1)
    else:
        dw = O.f16_bits_to_f32(ws)
        if flush:
            dw = np.where(np.abs(dw) < 2.0**-14, np.float32(0), dw)
        dw = np.roll(dw, dw_shift, axis=1)
        sf = s.astype(np.float32)
        if fmt == "tq2_0":
            t = (dx[:, None, :] * dw[None]) * sf  # kernels.py:141 order
        else:
            t = (sf * dw[None]) * dx[:, None, :]  # kernels.py:93 order
    if flip is not None:
        t = t.copy()
        t[..., flip] = -t[..., flip]
    return t.astype(np.float32)


def _sum_sequential(t):
    acc = np.zeros(t.shape[:-1], np.float32)
    for i in range(t.shape[-1]):
        acc = acc + t[..., i]
    return acc


def _sum_reversed(t):
    return _sum_sequential(t[..., ::-1])


def _sum_pairwise(t):
    v = t
    while v.shape[-1] > 1:
        if v.shape[-1] % 2:
            v = np.concatenate([v, np.zeros(v.shape[:-1] + (1,), np.float32)], axis=-1)
        v = v[..., 0::2] + v[..., 1::2]
    return v[..., 0] if v.shape[-1] else np.zeros(t.shape[:-1], np.float32)


def _sum_lanes(t, lanes=8):
    """Lane l adds terms l, l + lanes, ... in order, then a butterfly tree over the lanes (the kernels' shape)."""
    pad = (-t.shape[-1]) % lanes
    v = np.concatenate([t, np.zeros(t.shape[:-1] + (pad,), np.float32)], axis=-1)
    v = v.reshape(*t.shape[:-1], -1, lanes)
    acc = np.zeros(t.shape[:-1] + (lanes,), np.float32)
    for i in range(v.shape[-2]):
        acc = acc + v[..., i, :]
    return _sum_pairwise(acc)


def _sum_fma(fmt, ws, xd, s):
    """acc = fma(f32(s), dw * dx, acc): the product dw * dx in f32, then one rounding of s * that + acc (f64 holds
    f32(s) * f32 exactly, so the only double rounding left is the sum's)."""
    dx = np.asarray(xd, np.float32)
    if fmt == "q4_k":
        meta = np.ascontiguousarray(ws, dtype=np.int16).reshape(ws.shape[0], -1, 8)
        d = O.f16_bits_to_f32(meta[:, :, 0])
        dmin = O.f16_bits_to_f32(meta[:, :, 1])
        acc = np.zeros(s.shape[:2], np.float32)
        for b in range(s.shape[2]):
            p1 = (d[None, :, b] * dx[:, None, b]).astype(np.float64)
            acc = (s[:, :, b, 0].astype(np.float64) * p1 + acc.astype(np.float64)).astype(np.float32)
            p2 = (dmin[None, :, b] * dx[:, None, b]).astype(np.float64)
            acc = (-s[:, :, b, 1].astype(np.float64) * p2 + acc.astype(np.float64)).astype(np.float32)
        return acc
    dw = O.f16_bits_to_f32(ws)
    acc = np.zeros(s.shape[:2], np.float32)
    for b in range(s.shape[2]):
        p = (dx[:, None, b] * dw[None, :, b]).astype(np.float64)
        acc = (s[:, :, b].astype(np.float64) * p + acc.astype(np.float64)).astype(np.float32)
    return acc


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("extreme", [False, True])
def test_f32_evaluations_stay_within_the_bound(fmt, extreme):
    for seed in (1, 2, 3):
        ws, xd, s, r = _problem(fmt, seed, extreme)
        t = _f32_terms(fmt, ws, xd, s)
        for name, y in (("sequential", _sum_sequential(t)), ("reversed", _sum_reversed(t)),
                        ("pairwise", _sum_pairwise(t)), ("lanes", _sum_lanes(t)),
                        ("fma", _sum_fma(fmt, ws, xd, s))):  # fmt: skip
            ok, worst = O.output_check(fmt, y, ws, xd, s, r)
            assert ok, f"{fmt} seed {seed} extreme {extreme}: {name} order exceeds the bound ({worst:.3g})"


@pytest.mark.parametrize("fmt", FORMATS)
def test_planted_mistakes_break_the_bound(fmt):
    ws, xd, s, r = _problem(fmt, 5, False)
    nterms = s.shape[2] * (2 if fmt == "q4_k" else 1)
    mistakes = {
        "shifted scale index": _f32_terms(fmt, ws, xd, s, dw_shift=1),
        "dropped last block": np.concatenate(
            [_f32_terms(fmt, ws, xd, s)[..., : nterms - (2 if fmt == "q4_k" else 1)]], axis=-1),
        "flipped sign": _f32_terms(fmt, ws, xd, s, flip=s.shape[2] // 2),
        "another column's d_x": _f32_terms(fmt, ws, xd, s, col_shift=1),
    }
    for name, t in mistakes.items():
        ok, worst = O.output_check(fmt, _sum_sequential(t), ws, xd, s, r)
        assert not ok, f"{fmt}: the bound misses a {name} (worst {worst:.3g})"


@pytest.mark.parametrize("fmt", FORMATS)
def test_flushed_subnormal_scales_break_the_bound(fmt):
    """Rows whose weight scales are all f16 subnormals: a kernel that flushes them to zero gives 0 there."""
    ws, xd, s, r = _problem(fmt, 7, False)
    rng = np.random.default_rng(7)
    ws = np.array(ws, copy=True)
    if fmt == "q4_k":
        meta = ws.reshape(ws.shape[0], -1, 8)
        meta[:4, :, 0] = rng.integers(1, 1024, size=meta[:4, :, 0].shape)  # d subnormal, dmin kept
        ws = meta.reshape(ws.shape)
    else:
        ws[:4] = rng.integers(1, 1024, size=ws[:4].shape)
    n, k, _ = SHAPES[fmt]
    r = O.reference_dot(fmt, ws, xd, s)
    y_good = _sum_sequential(_f32_terms(fmt, ws, xd, s))
    assert O.output_check(fmt, y_good, ws, xd, s, r)[0]
    ok, worst = O.output_check(fmt, _sum_sequential(_f32_terms(fmt, ws, xd, s, flush=True)), ws, xd, s, r)
    assert not ok, f"{fmt}: the bound misses flushed subnormal scales (worst {worst:.3g})"


@pytest.mark.parametrize("fmt", FORMATS)
def test_bound_is_tight_on_random_data(fmt):
    """Not vacuous: the bound of a typical output is far below the output itself, so an error of 1e-4 of |r| in
    any single output of magnitude at least the median fails."""
    ws, xd, s, r = _problem(fmt, 9, False)
    bound = O.output_error_bound(fmt, ws, xd, s)
    big = np.abs(r) >= np.median(np.abs(r))
    assert np.all(bound[big] < 1e-4 * np.abs(r[big]))
    y = _sum_sequential(_f32_terms(fmt, ws, xd, s)).astype(np.float64)
    i = np.flatnonzero(big.reshape(-1))[0]
    y.reshape(-1)[i] += 1e-4 * abs(r.reshape(-1)[i])
    assert not O.output_check(fmt, y, ws, xd, s, r)[0]


def test_zero_terms_need_exact_zero():
    ws, xd, s, r = _problem("q4_0", 11, False)
    s = np.zeros_like(s)
    r = O.reference_dot("q4_0", ws, xd, s)
    y = np.zeros(r.shape, np.float32)
    assert O.output_check("q4_0", y, ws, xd, s, r) == (True, 0.0)
    y[0, 0] = np.float32(1e-30)
    assert not O.output_check("q4_0", y, ws, xd, s, r)[0]
    y[0, 0] = np.nan
    assert not O.output_check("q4_0", y, ws, xd, s, r)[0]


# ---------------------------------------------------------------------------------------------------------------------
# the combined gate (tests/checks.py: per-output bound and relerr <= 1e-5) at the workloads' long rows


@functools.lru_cache(maxsize=4)
def _long_row_problem(n, k, seed):
    """Q4_0 W [n][k] ~ N(0, 0.02) by ggml's q4_0 rule and one column x ~ N(0, 1) with 1% of entries x20 (the
    Llama-3-8B layer's activations), from the C oracle: (ws, xd, s [1][n][k/32], r)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    wq, ws = O.split("q4_0", C.quantize_q4_0_weights(w), n, k)
    x = rng.standard_normal((1, k), dtype=np.float32)
    x = np.where(rng.random((1, k)) < 0.01, x * np.float32(20), x).astype(np.float32)
    xq, xd = C.quant_q8_0(x)
    s = C.block_dots("q4_0", wq, xq, n, k)
    return ws, xd, s, C.reference_dot("q4_0", ws, xd, s)


def _round_mantissa(p, bits):
    """f32 p rounded to nearest (ties away) at `bits` fraction bits: a kernel keeping a short scale product."""
    u = np.ascontiguousarray(p, np.float32).view(np.uint32).astype(np.uint64)
    shift = 23 - bits
    u = ((u + (1 << (shift - 1))) >> shift) << shift
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("k", [4096, 8192, 14336])
def test_gate_is_tight_at_long_rows(k):
    """Not vacuous at 128-448 blocks a row, where the per-output bound alone admits 1e-4 of |r| and more: the f32
    evaluations pass the combined gate, and an error of 1e-4 of |r| in one output at or above the median fails it."""
    ws, xd, s, r = _long_row_problem(512, k, 31)
    t = _f32_terms("q4_0", ws, xd, s)
    for name, y in (("sequential", _sum_sequential(t)), ("lanes", _sum_lanes(t)), ("fma", _sum_fma("q4_0", ws, xd, s))):
        ok, msg = gate("q4_0", y, ws, xd, s, r)
        assert ok, f"k={k} {name}: {msg}"
    y = _sum_sequential(t).astype(np.float64)
    big = np.flatnonzero((np.abs(r) >= np.median(np.abs(r))).reshape(-1))
    for i in big[:: max(1, big.size // 16)]:
        yp = y.copy()
        yp.reshape(-1)[i] += 1e-4 * abs(r.reshape(-1)[i])
        assert not gate("q4_0", yp, ws, xd, s, r)[0], f"k={k}: an error of 1e-4 |r| at output {i} passes"


@pytest.mark.parametrize("bits", [12, 13, 14])
def test_short_scale_product_fails_the_gate_at_4096x14336(bits):
    """A kernel that keeps only 12-14 fraction bits of each block's scale product d_w * d_x, summing in f32, stays
    within the per-output bound at the Llama-3-8B down projection (448 Q4_0 blocks a row), so only the relerr half of
    the gate catches it; the full-precision f32 evaluation passes both halves."""
    ws, xd, s, r = _long_row_problem(4096, 14336, 37)
    dw = O.f16_bits_to_f32(ws)
    dx = np.asarray(xd, np.float32)
    good = _sum_sequential((s.astype(np.float32) * dw[None]) * dx[:, None, :])
    assert gate("q4_0", good, ws, xd, s, r)[0]
    short = _sum_sequential(s.astype(np.float32) * _round_mantissa(dw[None] * dx[:, None, :], bits))
    bound_ok, _ = O.output_check("q4_0", short, ws, xd, s, r)
    ok, msg = gate("q4_0", short, ws, xd, s, r)
    assert not ok and "relerr" in msg, f"{bits} bits: {msg}"
    if bits == 12:
        assert bound_ok, "the per-output bound alone was expected to admit the 12-bit scale product here"
