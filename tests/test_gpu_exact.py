"""Outputs that f32 arithmetic must reproduce bit for bit: every weight scale an f16 subnormal (k * 2**-24), power-of-two
activation scales, and integer dots small enough that every term and every partial sum is an exact f32.  Then any
summation order gives the exact value, so the device Y must equal the f64 reference bit for bit, on every route
(the general kernel in the three modes, the lean dp4a kernels, the fused launch, the matrix-core GEMM).  A kernel that
flushed subnormal scales to zero (patch:33-36 decodes them exactly), read a wrong scale or d_x, or rounded a term
twice would fail here even where the output is tiny next to its row's other outputs."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O

FORMATS = ("q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k")
K = {"q4_0": 1024, "q8_0": 1024, "iq4_nl": 512, "tq2_0": 2048, "q4_k": 512}
E = -2  # activation scale 2**E


def exact_problem(fmt, n, m, seed):
    """(W ggml block bytes, x f32 [m][K]) with the properties above.  Weights take the values 0 and +-1 (iq4_nl: its
    table's 1 and -10; q4_k: nibbles 0 and 1 with 6-bit scales and mins below 4); every activation block holds one
    127 * 2**E, whose weight is 0 (iq4_nl: 1), among values of at most 15 * 2**E in magnitude, so the block's d is
    +-2**E."""
    rng = np.random.default_rng(seed)
    k = K[fmt]
    blk = O.FORMATS[fmt]["block"]
    nb = k // blk
    kmax = 511 if fmt in ("iq4_nl", "q4_k") else 1023
    sub = rng.integers(1, kmax + 1, size=(n, nb)).astype(np.uint16)  # f16 subnormal bit patterns
    ablk = O.ACT_BLOCK[O.FORMATS[fmt]["act"]]
    amax = 15 if ablk == 32 else 7
    q = rng.integers(-amax, amax + 1, size=(m, k))
    peak = rng.integers(0, ablk, size=(m, k // ablk)) + np.arange(k // ablk) * ablk
    for i in range(m):
        q[i, peak[i]] = 127
    x = (q * 2.0**E).astype(np.float32)
    zero = np.zeros(k, bool)
    zero[peak.reshape(-1)] = True  # weight 0 at every column's peak position
    if fmt in ("q4_0", "iq4_nl"):
        lo, hi = (7, 9) if fmt == "q4_0" else (7, 8)  # q4_0: -1, 0, +1; iq4_nl: table values -10, 1
        nib = rng.integers(lo, hi + 1, size=(n, k)).astype(np.uint8)
        nib[:, zero] = 8  # q4_0: 0; iq4_nl: 1 (its table has no 0)
        return O.pack_q4_0(nib, sub), x
    if fmt == "q8_0":
        v = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
        v[:, zero] = 0
        return O.pack_q8_0(v, sub), x
    if fmt == "tq2_0":
        c = rng.integers(0, 3, size=(n, k)).astype(np.uint8)
        c[:, zero] = 1
        return O.pack_tq2_0(c, sub), x
    nib = rng.integers(0, 2, size=(n, k)).astype(np.uint8)
    nib[:, zero] = 0
    sc = rng.integers(0, 4, size=(n, nb, 8)).astype(np.uint8)
    mn = rng.integers(0, 4, size=(n, nb, 8)).astype(np.uint8)
    sc12 = np.zeros((n, nb, 12), np.uint8)
    sc12[:, :, 0:4] = sc[:, :, 0:4]
    sc12[:, :, 4:8] = mn[:, :, 0:4]
    sc12[:, :, 8:12] = sc[:, :, 4:8] | (mn[:, :, 4:8] << 4)
    dmin = rng.integers(1, kmax + 1, size=(n, nb)).astype(np.uint16)
    return O.pack_q4_k(nib, sub, dmin, sc12), x


def exact_reference(fmt, W, x, n):
    k = x.shape[1]
    wq, ws = O.split(fmt, W, n, k)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    return wq, ws, rq, rd, r, rs


@pytest.mark.parametrize("fmt", FORMATS)
def test_exact_problem_is_exact(fmt):
    """CPU check of the construction: the scales are f16 subnormals, |d_x| = 2**E, and the integer parts of the terms
    sum to less than 2**24 in magnitude, so every term and partial sum is an exact f32 and r is an f32 value."""
    n, m = 40, 3
    W, x = exact_problem(fmt, n, m, 1)
    wq, ws, rq, rd, r, rs = exact_reference(fmt, W, x, n)
    assert np.all(np.abs(rd) == 2.0**E)
    scales = ws.reshape(n, -1, 8)[:, :, :2] if fmt == "q4_k" else ws
    bits = np.asarray(scales).astype(np.uint16)
    assert np.all((bits & 0x7C00) == 0) and np.all(bits != 0)  # every f16 scale subnormal
    terms, _ = O.output_terms(fmt, ws, rd, rs)
    units = np.abs(terms) / 2.0 ** (E - 24)
    assert np.all(units == np.round(units)) and np.all(units.sum(-1) < 2**24)
    assert np.array_equal(r.astype(np.float32).astype(np.float64), r)
    assert np.count_nonzero(r) > 0.9 * r.size


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def bits_equal(y, r):
    return np.array_equal(np.asarray(y, np.float32).view(np.uint32), r.astype(np.float32).view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("m", [1, 3])
def test_gemv_routes_bit_exact(fmt, m):
    n = 300
    W, x = exact_problem(fmt, n, m, 10 + m)
    wq, ws, rq, rd, r, rs = exact_reference(fmt, W, x, n)
    k = x.shape[1]
    wq_d, ws_d, xq_d, xd_d = dev(wq), dev(ws), dev(rq), dev(rd)
    runs = {}
    for mode in (0, 1, 2):
        for knobs in ((32, 4, 4), (128, 2, 8)):
            runs[f"mode {mode} knobs {knobs}"] = host.gemv(fmt, wq_d, ws_d, xq_d, xd_d, n, k, *knobs[:2], mode, knobs[2])[0]
    runs["library plan"] = host.gemv(fmt, wq_d, ws_d, xq_d, xd_d, n, k, block_n=None, mode=2)[0]
    runs["fused, library plan"] = host.gemv_f32(fmt, wq_d, ws_d, dev(x), n, k)[0]
    runs["fused, knobs (16, 2, 2)"] = host.gemv_f32(fmt, wq_d, ws_d, dev(x), n, k, 16, 2, 2, 2)[0]
    torch.cuda.synchronize()
    for name, y in runs.items():
        assert bits_equal(y.cpu().numpy(), r), f"{fmt} m={m} {name}: Y differs from the exact value"


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
def test_gemm_bit_exact(fmt):
    n, m = 200, 20
    W, x = exact_problem(fmt, n, m, 30)
    wq, ws, rq, rd, r, rs = exact_reference(fmt, W, x, n)
    y, s = host.gemm(fmt, dev(wq), dev(ws), dev(rq), dev(rd), n, x.shape[1], store_s=True)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert bits_equal(y.cpu().numpy(), r), f"{fmt}: GEMM Y differs from the exact value"


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0"])
@pytest.mark.parametrize("act", [-128, 127])
@pytest.mark.parametrize("m", [1, 3])
def test_bytes_mode_sums_at_their_largest(fmt, act, m):
    """The largest integer dots the formats allow: every nibble 15 (Q4_0 value +7) or every crumb 3 (TQ2_0 value
    +2) against activations all -128 or all 127, q8 bytes given directly (the quantizers never produce -128; the C ABI
    takes any bytes).  Bytes mode keeps 16-bit partial sums (at most 16 Q4_0 products of 15 x 128 or 32 TQ2_0 products
    of 3 x 128 in a half), so this is where they would overflow: S must equal the exact dots in every mode, on the lean
    and general kernels, and Y the exact reference."""
    n, k = 300, K[fmt]
    blk, qb = (32, 16) if fmt == "q4_0" else (256, 64)
    nb = k // blk
    wq = np.full((n, nb * qb), 0xFF, np.uint8)
    ws = np.full((n, nb), 0x3C00, np.uint16).view(np.int16)  # d_w = 1
    xq = np.full((m, k), act, np.int8)
    xd = np.full((m, nb), 0.5, np.float32)
    r, rs = O.gemv(fmt, wq, ws, xq, xd, n, k)
    assert (rs == (7 if fmt == "q4_0" else 2) * act * blk).all()  # the oracle's decode: nibble 15 -> 7, crumb 3 -> 2
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    wq_d, ws_d, xq_d, xd_d = dev(wq), dev(ws), dev(xq), dev(xd)
    runs = []
    for mode in (0, 1, 2):  # bytes, emulated dp4a (the general kernel), dp4a
        for bn, nb_, nw in ((None, 4, 4), (64, 1, 4), (16, 4, 4)):  # auto (lean), knob sets (lean / general)
            print(f"{fmt} act={act} m={m} mode={mode} block_n={bn} nb={nb_} num_warps={nw}", flush=True)
            runs.append((mode, host.gemv(fmt, wq_d, ws_d, xq_d, xd_d, n, k, bn, nb_, mode, nw, store_s=True)))
    torch.cuda.synchronize()
    for mode, (y, s) in runs:
        assert np.array_equal(s.cpu().numpy().astype(np.int64), rs), mode
        # every term and partial sum is an integer below 2**24, exact in f32: Y equals the reference in any order
        assert np.array_equal(y.cpu().numpy().astype(np.float64), r), mode
