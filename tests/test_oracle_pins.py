"""Pins of the CPU oracle (oracle/oracle.py) against what fixes each function independently of it: the reference's
own edge words, layouts and known answers, exhaustive enumeration, exact rational arithmetic with explicit IEEE
rounding (tests/exact.py), brute force on tiny inputs, and algebraic invariants.  Each check is chosen so that a
plausible mistake (a swapped nibble, a wrong crumb shift, a missing f16 rounding, the f16 d used for q, round-half-even
where half-away is meant, last-index ties, a dropped -8 offset, a different block order) fails it."""

import math
import random
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from tests import exact as X

# ---------------------------------------------------------------------------------------------------------------------
# f16 bits -> f32 (patch:33-36): all 65536 patterns vs the binary16 field definition


def test_f16_bits_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(bits.view(np.int16))
    for b in range(65536):
        want = X.f16_from_bits(b)
        g = float(got[b])
        if isinstance(want, float) and math.isnan(want):
            assert math.isnan(g)
        else:
            assert g == (want if isinstance(want, float) else float(want)), hex(b)
    assert float(got[0x7BFF]) == 65504.0 and float(got[0x0001]) == 2.0**-24


# ---------------------------------------------------------------------------------------------------------------------
# decode (patch:16-19, 39-63): every byte value at every position, with arithmetic other than the oracle's masks


def test_q4_0_every_byte_every_position():
    for pos in range(16):
        qs = np.zeros((256, 16), np.uint8)
        qs[:, pos] = np.arange(256)
        v = O.q4_0_values(qs)
        for b in range(256):
            lo, hi = b % 16, b // 16
            assert v[b, pos] == lo - 8 and v[b, pos + 16] == hi - 8
        # every other value decodes byte 0 -> -8
        others = [i for i in range(32) if i not in (pos, pos + 16)]
        assert (v[:, others] == -8).all()


def test_q8_0_every_byte_every_position():
    for pos in (0, 13, 31):
        qs = np.zeros((256, 32), np.uint8)
        qs[:, pos] = np.arange(256)
        v = O.q8_0_values(qs)
        for b in range(256):
            assert v[b, pos] == struct.unpack("<b", bytes([b]))[0]
        assert (np.delete(v, pos, axis=1) == 0).all()


def test_iq4_nl_every_byte_every_position():
    # value i = table[low nibble of byte i], value i+16 = table[high nibble of byte i]; decoded here through the table
    # held in a dict keyed by nibble, one byte at a time
    table = dict(enumerate(int(t) for t in O.IQ4_NL_VALUES))
    for pos in (0, 7, 15):
        qs = np.full((256, 16), 0x88, np.uint8)  # nibble 8 -> table[8] elsewhere
        qs[:, pos] = np.arange(256)
        v = O.iq4_nl_values(qs)
        for b in range(256):
            assert v[b, pos] == table[b & 15] and v[b, pos + 16] == table[b >> 4]
        others = [i for i in range(32) if i not in (pos, pos + 16)]
        assert (v[:, others] == table[8]).all()
    # the table is a non-uniform 4-bit grid inside int8: 16 strictly increasing entries spanning -127 .. 113
    t = O.IQ4_NL_VALUES
    assert t.size == 16 and (np.diff(t) > 0).all() and t[0] == -127 and t[-1] == 113 and len(set(t.tolist())) == 16


def test_new_format_blocks_from_ggml_bytes():
    # block_q8_0 / block_iq4_nl bytes built with struct, decoded value by value
    rng = np.random.default_rng(21)
    d = struct.pack("<e", 0.25)
    q = [int(v) for v in rng.integers(-128, 128, size=32)]
    blk = d + struct.pack("<32b", *q)
    wq, ws = O.split("q8_0", blk, 1, 32)
    assert ws[0, 0].tobytes() == d and O.weight_values("q8_0", wq, 1, 32).tolist() == [q]
    idx = [int(v) for v in rng.integers(0, 16, size=32)]
    blk = d + bytes((idx[i] | (idx[i + 16] << 4)) for i in range(16))
    wq, ws = O.split("iq4_nl", blk, 1, 32)
    assert O.weight_values("iq4_nl", wq, 1, 32).tolist() == [[int(O.IQ4_NL_VALUES[i]) for i in idx]]


def test_q4_k_every_byte_every_position():
    # ggml dequantize_row_q4_K order: for each 32-byte group j: 32 low nibbles (values 64j..64j+31), then the 32 high
    # nibbles of the same bytes (values 64j+32..64j+63)
    for pos in (0, 31, 32, 77, 127):
        qs = np.full((256, 128), 0x53, np.uint8)
        qs[:, pos] = np.arange(256)
        v = O.q4_k_values(qs)
        j, l = divmod(pos, 32)
        for b in range(256):
            assert v[b, 64 * j + l] == b & 15 and v[b, 64 * j + 32 + l] == b >> 4
        others = [i for i in range(256) if i not in (64 * j + l, 64 * j + 32 + l)]
        assert ((v[:, others] == 3) | (v[:, others] == 5)).all()
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, size=(3, 128), dtype=np.uint8)
    want = []
    for row in qs:  # the loop of the dequantizer, value by value
        out = []
        for j in range(4):
            out += [int(row[32 * j + l]) & 15 for l in range(32)] + [int(row[32 * j + l]) >> 4 for l in range(32)]
        want.append(out)
    assert O.q4_k_values(qs).tolist() == want


def _q4_k_scales_bits(sc12):
    """The 6-bit fields read out of the 96-bit little-endian integer of the 12 bytes: sub-block i < 4 at bits 8i
    (scale) and 32 + 8i (min); i >= 4: bits 64 + 8(i-4) (low 4 scale bits), 68 + 8(i-4) (low 4 min bits), and the
    two top bits of bytes i-4 (scale) and i (min) as bits 4..5."""
    v = int.from_bytes(bytes(sc12), "little")
    bits = lambda at, w: (v >> at) & ((1 << w) - 1)  # noqa: E731
    sc = [bits(8 * i, 6) for i in range(4)] + [bits(64 + 8 * i, 4) | (bits(8 * i + 6, 2) << 4) for i in range(4)]
    mn = [bits(32 + 8 * i, 6) for i in range(4)] + [bits(68 + 8 * i, 4) | (bits(32 + 8 * i + 6, 2) << 4) for i in range(4)]
    return sc, mn


def _q4_k_scales_words(sc12):
    """The same fields as ggml's vec_dot unpacks them: three little-endian dwords u0..u2 rearranged with byte masks
    into the 8 scales (bytes of two dwords) and the 8 mins."""
    u0, u1, u2 = struct.unpack("<3I", bytes(sc12))
    s_lo = u0 & 0x3F3F3F3F
    s_hi = (u2 & 0x0F0F0F0F) | (((u0 >> 6) & 0x03030303) << 4)
    m_lo = u1 & 0x3F3F3F3F
    m_hi = ((u2 >> 4) & 0x0F0F0F0F) | (((u1 >> 6) & 0x03030303) << 4)
    return list(struct.pack("<2I", s_lo, s_hi)), list(struct.pack("<2I", m_lo, m_hi))


def test_q4_k_scales_every_byte_every_position():
    rng = np.random.default_rng(5)
    for pos in range(12):
        base = rng.integers(0, 256, size=12, dtype=np.uint8)
        sc12 = np.tile(base, (256, 1))
        sc12[:, pos] = np.arange(256)
        sc, mn = O.q4_k_scales(sc12)
        for b in range(256):
            want = _q4_k_scales_bits(sc12[b])
            assert (sc[b].tolist(), mn[b].tolist()) == want
            assert want == _q4_k_scales_words(sc12[b])
    assert O.q4_k_scales(np.full(12, 0xFF, np.uint8))[0].tolist() == [63] * 8  # every field at its maximum


def test_q4_k_block_dots_are_the_dequantized_dot():
    # ggml dequantizes value l of sub-block i to d * sc_i * q_l - dmin * m_i; the oracle's (sd, sm) must give exactly
    # sum_l (that value) * (dx * x_l), checked here with exact rationals on blocks built with struct
    from fractions import Fraction

    rng = np.random.default_rng(6)
    n, k, m = 3, 512, 2
    W = O.weights("q4_k", rng, n, k, extreme=True)
    wq, ws = O.split("q4_k", W, n, k)
    xq = rng.integers(-128, 128, size=(m, k)).astype(np.int8)
    xd = rng.uniform(0.001, 0.1, size=(m, k // 256)).astype(np.float32)
    s = O.block_dots("q4_k", wq, xq, n, k, ws)
    assert s.shape == (m, n, k // 256, 2)
    for r in range(n):
        for b in range(k // 256):
            raw = W[(r * (k // 256) + b) * 144 :][:144]
            d, dmin = (Fraction(float(v)) for v in struct.unpack_from("<2e", raw, 0))
            sc, mn = _q4_k_scales_bits(raw[4:16])
            q = [raw[16 + 32 * (v // 64) + v % 32] >> (4 * ((v % 64) // 32)) & 15 for v in range(256)]
            for i in range(m):
                xs = [int(t) for t in xq[i, 256 * b : 256 * (b + 1)]]
                sd = sum(sc[v // 32] * q[v] * xs[v] for v in range(256))
                sm = sum(mn[v // 32] * xs[v] for v in range(256))
                assert tuple(s[i, r, b]) == (sd, sm)
                dx = Fraction(float(xd[i, b]))
                deq = sum((d * sc[v // 32] * q[v] - dmin * mn[v // 32]) * dx * xs[v] for v in range(256))
                assert deq == d * dx * sd - dmin * dx * sm


def test_q4_k_known_answer():
    # one block: d = 0.5, dmin = 0.25, every scale 2 and every min 1, quant nibbles all 3; x = 1 everywhere, dx = 1:
    # each value dequantizes to 0.5 * 2 * 3 - 0.25 * 1 = 2.75.  Scales 0..3 sit in bytes 0..3, mins 0..3 in bytes
    # 4..7, sub-blocks 4..7 in bytes 8..11 (scale in the low nibble, min in the high nibble; top bits 0)
    sc12 = bytes([2, 2, 2, 2, 1, 1, 1, 1, 0x12, 0x12, 0x12, 0x12])
    blk = struct.pack("<2e", 0.5, 0.25) + sc12 + bytes([0x33] * 128)
    wq, ws = O.split("q4_k", blk, 1, 256)
    xq = np.ones((1, 256), np.int8)
    y, s = O.gemv("q4_k", wq, ws, xq, np.ones((1, 1), np.float32), 1, 256)
    assert tuple(s[0, 0, 0]) == (2 * 3 * 256, 256) and y[0, 0] == 2.75 * 256


def test_tq2_0_every_byte_every_position():
    # ggml dequantize_row_tq2_0 order: for j in (0, 32): for l in 0..3: for m in 0..31: y = crumb(qs[j+m], l) - 1
    rng = np.random.default_rng(0)
    qs = rng.integers(0, 256, size=(8, 64), dtype=np.uint8)
    qs[0] = np.arange(64, dtype=np.uint8) * 4  # + every byte value across rows 0..3
    qs[1:5] = np.arange(256, dtype=np.uint8).reshape(4, 64)
    got = O.tq2_0_values(qs)
    for r in range(qs.shape[0]):
        want = []
        for j in (0, 32):
            for l in range(4):
                for m in range(32):
                    want.append((int(qs[r, j + m]) // 4**l) % 4 - 1)
        assert list(got[r]) == want


def test_tq2_0_pack_round_trip():
    rng = np.random.default_rng(1)
    crumbs = rng.integers(0, 4, size=(3, 512), dtype=np.uint8)
    d = np.full((3, 2), 0x3C00, np.uint16)
    wq, ws = O.split("tq2_0", O.pack_tq2_0(crumbs, d), 3, 512)
    assert np.array_equal(O.weight_values("tq2_0", wq, 3, 512), crumbs.astype(np.int32) - 1)
    assert (ws.view(np.uint16) == 0x3C00).all()


def test_q4_0_ggml_quantize_round_trip():
    # ggml quantize_row_q4_0_ref: d = max / -8 with max the signed value of largest |x|; x = q * d with q in -8..7 and
    # a -8 in every block (so max = -8 d) must come back as exactly q after decode
    rng = np.random.default_rng(2)
    n, k = 4, 256
    q = rng.integers(-8, 8, size=(n, k))
    q.reshape(n, k // 32, 32)[:, :, 5] = -8
    d = np.float32(0.015625)  # a power of two: x = q d and x / d are exact
    w = (q * d).astype(np.float32)
    wq, ws = O.split("q4_0", O.quantize_q4_0_weights(w), n, k)
    assert np.array_equal(O.weight_values("q4_0", wq, n, k), q)
    assert (O.f16_bits_to_f32(ws) == d).all()


# ---------------------------------------------------------------------------------------------------------------------
# dp4a (patch:66-81; src/komp/verify.py:37-47)

EDGE = [0, -1, 0x7F7F7F7F, -0x7F7F7F80, 0x01010101, 0x0F0F0F0F, 0x03030303, 2**31 - 1, -(2**31), 0x80000000 - 2**32]


def _dp4a_struct(a, b, c):
    sa = struct.unpack("<4b", struct.pack("<i", a))
    sb = struct.unpack("<4b", struct.pack("<i", b))
    r = c + sum(x * y for x, y in zip(sa, sb))
    return struct.unpack("<i", struct.pack("<I", r & 0xFFFFFFFF))[0]


def test_dp4a_edge_and_random_words():
    rng = random.Random(3)
    a = [rng.choice(EDGE) if rng.random() < 0.3 else rng.randrange(-(2**31), 2**31) for _ in range(1024)]
    b = [rng.choice(EDGE) if rng.random() < 0.3 else rng.randrange(-(2**31), 2**31) for _ in range(1024)]
    c = [rng.randrange(-(2**20), 2**20) for _ in range(1024)]
    got = O.dp4a(np.array(a), np.array(b), np.array(c))
    assert [int(v) for v in got] == [_dp4a_struct(x, y, z) for x, y, z in zip(a, b, c)]
    for x in EDGE:
        for y in EDGE:
            assert int(O.dp4a(x, y, 0)) == _dp4a_struct(x, y, 0)


def test_dp4a_known_answers():
    assert int(O.dp4a(0x7F7F7F7F, 0x7F7F7F7F, 0)) == 4 * 127 * 127
    assert int(O.dp4a(-0x7F7F7F80, -0x7F7F7F80, 0)) == 4 * 128 * 128  # 0x80808080: four -128s
    assert int(O.dp4a(-1, -1, 5)) == 9
    assert int(O.dp4a(0x01010101, 0x04FF02FE, 0)) == 4 - 1 + 2 - 2
    assert int(O.dp4a(0x7F7F7F7F, 0x7F7F7F7F, 2**31 - 1)) == 2**31 - 1 + 64516 - 2**32  # int32 wraparound


# ---------------------------------------------------------------------------------------------------------------------
# rounding (patch:84-101)


def test_rounding_known_answers():
    xs = np.array([0.5, 1.5, 2.5, -0.5, -2.5, 3.5, 0.49999997, -0.49999997, 8388609.0, 1e30, 1e-45, -0.0, 126.5],
                  np.float32)  # fmt: skip
    assert list(O.round_half_away(xs)) == [1, 2, 3, -1, -3, 4, 0, 0, 8388609, np.float32(1e30), 0, 0, 127]
    assert list(O.round_half_even(xs)) == [0, 2, 2, 0, -2, 4, 0, 0, 8388609, np.float32(1e30), 0, 0, 126]


def test_rounding_vs_exact_rationals():
    rng = np.random.default_rng(4)
    xs = np.concatenate([rng.normal(0, 100, 4000), (rng.integers(-300, 300, 2000) + 0.5)]).astype(np.float32)
    ha, he = O.round_half_away(xs), O.round_half_even(xs)
    for x, a, e in zip(xs, ha, he):
        assert a == X.round_half_away(X.f32(x)) and e == X.round_half_even(X.f32(x))
        assert e == round(float(x))  # Python's round() on floats is half-to-even


# ---------------------------------------------------------------------------------------------------------------------
# q8_0 (patch:104-114; kernels.py:22-33)


def _q8_0_exact(x):
    m, k = x.shape
    q = np.zeros((m, k), np.int64)
    d = np.zeros((m, k // 32), np.float64)
    for i in range(m):
        for b in range(k // 32):
            qq, dd = X.q8_0_block(x[i, b * 32 : (b + 1) * 32])
            q[i, b * 32 : (b + 1) * 32] = qq
            d[i, b] = dd
    return q, d


@pytest.mark.parametrize("extreme", [False, True])
def test_q8_0_vs_exact_arithmetic(extreme):
    x = O.activations(np.random.default_rng(5 + extreme), 32 * 24, 2, block=32, extreme=extreme, outliers=0.05)
    x[0, :32] = np.linspace(-1, 1, 32, dtype=np.float32) * np.float32(1e-36)  # d is an f32 subnormal, 1/d finite
    x[1, 32:64] = np.float32(3e-6)  # f16(d) is an f16 subnormal
    xq, xd = O.quant_q8_0(x)
    q, d = _q8_0_exact(x)
    assert np.array_equal(xq.astype(np.int64), q)
    assert np.array_equal(xd.astype(np.float64), d)


def test_q8_0_known_answers():
    x = np.zeros((1, 96), np.float32)
    x[0, :32] = np.arange(-16, 16)
    x[0, 31] = 127.0  # amax 127 -> d = 1 exactly, q == x
    x[0, 32:64] = np.arange(32) - np.float32(15.5)  # d = 15.5 / 127
    xq, xd = O.quant_q8_0(x)
    assert list(xq[0, :32]) == list(x[0, :32].astype(int)) and xd[0, 0] == 1.0
    assert xd[0, 2] == 0.0 and (xq[0, 64:] == 0).all()
    assert xq[0, 32] == -127 and xq[0, 63] == 127
    # the stored d is f16-rounded, q uses the unrounded d: 15.5/127 is not an f16 value
    assert xd[0, 1] == np.float32(np.float32(15.5) / np.float32(127)).astype(np.float16).astype(np.float32)
    assert xd[0, 1] != np.float32(15.5) / np.float32(127)


def test_q8_0_overflowing_scale_is_inf():
    x = np.full((1, 32), np.float32(1e38))
    _, xd = O.quant_q8_0(x)
    assert np.isinf(xd[0, 0])


# ---------------------------------------------------------------------------------------------------------------------
# q8_K (patch:117-131; host.py:50)


@pytest.mark.parametrize("extreme", [False, True])
def test_q8_K_vs_exact_arithmetic(extreme):
    x = O.activations(np.random.default_rng(6 + extreme), 256 * 6, 2, block=256, extreme=extreme, outliers=0.05)
    x[1, 256:512] *= np.float32(1e-35)  # tiny inputs (some subnormal after scaling), iscale finite
    xq, xd, xb = O.quant_q8_K(x)
    for i in range(2):
        for b in range(6):
            q, d, bs = X.q8_K_block(x[i, b * 256 : (b + 1) * 256])
            assert list(xq[i, b * 256 : (b + 1) * 256].astype(int)) == q
            assert float(xd[i, b]) == d
            assert list(xb[i, b * 16 : (b + 1) * 16].astype(int)) == bs


def test_q8_K_first_index_tie_and_zero_block():
    x = np.zeros((1, 512), np.float32)
    x[0, 3] = 2.0
    x[0, 9] = -2.0  # same |x|, later: the first (positive) one sets the sign
    x[0, 10] = 1.0
    xq, xd, xb = O.quant_q8_K(x)
    assert xq[0, 3] == -127 and xq[0, 9] == 127 and xq[0, 10] == -64  # -127/2 * 1 = -63.5 -> -64 (half to even)
    assert xd[0, 0] == np.float32(1) / (np.float32(-127) / np.float32(2))
    assert xd[0, 1] == 0.0 and (xq[0, 256:] == 0).all() and (xb[0, 16:] == 0).all()
    assert xb[0, 0] == -127 + 127 - 64
    assert xq.min() >= -127  # the docstring's -128 cannot occur


# ---------------------------------------------------------------------------------------------------------------------
# split planes and ggml blocks (host.py:16-56; tests/test_komp.py:69-82)


def test_split_layout_is_kurns():
    rng = np.random.default_rng(7)
    n, k = 3, 96
    W = O.weights("q4_0", rng, n, k)
    wq, ws = O.split("q4_0", W, n, k)
    for r in range(n):
        for b in range(k // 32):
            blk = W[(r * (k // 32) + b) * 18 : (r * (k // 32) + b + 1) * 18]
            assert bytes(wq[r, b * 16 : b * 16 + 16]) == blk[2:18]
            assert ws[r, b].tobytes() == blk[:2]
    assert wq.dtype == np.uint8 and ws.dtype == np.int16
    W = O.weights("tq2_0", rng, n, 512)
    wq, ws = O.split("tq2_0", W, n, 512)
    for r in range(n):
        for b in range(2):
            blk = W[(r * 2 + b) * 66 : (r * 2 + b + 1) * 66]
            assert bytes(wq[r, b * 64 : b * 64 + 64]) == blk[:64] and ws[r, b].tobytes() == blk[64:66]
    assert O.join("tq2_0", wq, ws) == W


def test_act_block_layouts():
    xq = np.arange(-16, 16, dtype=np.int8).reshape(1, 32)
    xd = np.array([[0.5]], np.float32)
    blk = O.q8_0_blocks(xq, xd)
    assert len(blk) == 34 and struct.unpack_from("<e", blk, 0)[0] == 0.5
    assert struct.unpack_from("<32b", blk, 2) == tuple(range(-16, 16))
    xq = np.tile(np.arange(16, dtype=np.int8), 16).reshape(1, 256)
    blk = O.q8_K_blocks(xq, np.array([[0.25]], np.float32))
    assert len(blk) == 292 and struct.unpack_from("<f", blk, 0)[0] == 0.25
    assert struct.unpack_from("<16h", blk, 260) == (120,) * 16


# ---------------------------------------------------------------------------------------------------------------------
# GEMV references (verify.py:94-120)


@pytest.mark.parametrize("fmt,k", [("q4_0", 96), ("tq2_0", 512), ("q8_0", 96), ("iq4_nl", 96)])  # q4_k: above
def test_block_dots_brute_force(fmt, k):
    rng = np.random.default_rng(8)
    n, m = 5, 2
    W = O.weights(fmt, rng, n, k, extreme=True)
    wq, _ = O.split(fmt, W, n, k)
    xq = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    s = O.block_dots(fmt, wq, xq, n, k)
    blk = O.FORMATS[fmt]["block"]
    # values straight from the ggml block bytes, one at a time
    for r in range(n):
        for b in range(k // blk):
            raw = W[(r * (k // blk) + b) * O.FORMATS[fmt]["nbytes"] :][: O.FORMATS[fmt]["nbytes"]]
            if fmt == "q4_0":
                vals = [(raw[2 + i % 16] >> (4 * (i // 16))) % 16 - 8 for i in range(32)]
            elif fmt == "q8_0":
                vals = list(struct.unpack("<32b", bytes(raw[2:34])))
            elif fmt == "iq4_nl":
                vals = [int(O.IQ4_NL_VALUES[(raw[2 + i % 16] >> (4 * (i // 16))) % 16]) for i in range(32)]
            else:
                vals = [(raw[(v // 128) * 32 + v % 32] >> (2 * ((v % 128) // 32))) % 4 - 1 for v in range(256)]
            for i in range(m):
                want = sum(int(a) * int(q) for a, q in zip(vals, xq[i, b * blk : (b + 1) * blk]))
                assert s[i, r, b] == want


def test_block_dots_bilinear():
    rng = np.random.default_rng(9)
    n, k = 7, 1024
    W = O.weights("tq2_0", rng, n, k)
    wq, _ = O.split("tq2_0", W, n, k)
    a = rng.integers(-60, 60, size=(1, k)).astype(np.int8)
    b = rng.integers(-60, 60, size=(1, k)).astype(np.int8)
    assert np.array_equal(O.block_dots("tq2_0", wq, a + b, n, k),
                          O.block_dots("tq2_0", wq, a, n, k) + O.block_dots("tq2_0", wq, b, n, k))  # fmt: skip


def test_reference_dot_exact_with_power_of_two_scales():
    # all products and partial sums are exact: the f64 result equals the exact rational sum
    rng = np.random.default_rng(10)
    s = rng.integers(-5000, 5000, size=(2, 3, 9))
    ws = np.full((3, 9), 0x3400, np.uint16).view(np.int16)  # f16 0.25
    xd = np.full((2, 9), 0.125, np.float32)
    r = O.reference_dot("q4_0", ws, xd, s)
    assert np.array_equal(r, s.sum(axis=2) * 0.25 * 0.125)


def test_reference_dot_follows_block_order():
    # terms 2^60, 1, -2^60: sequential order gives 0; any order that adds 1 last gives 1
    ws = np.array([[0x3C00, 0x3C00, 0x3C00]], np.uint16).view(np.int16)
    xd = np.array([[2.0**30, 1.0, 2.0**30]], np.float32)
    s = np.array([[[2**30, 1, -(2**30)]]])
    assert O.reference_dot("tq2_0", ws, xd, s)[0, 0] == 0.0
    assert sum((Fraction(2**60), Fraction(1), Fraction(-(2**60)))) == 1  # the exact sum, which the order loses


def test_reference_dot_error_bound_random():
    rng = np.random.default_rng(11)
    fmt, n, k, m = "q4_0", 9, 32 * 40, 2
    W, x = O.problem(fmt, n, k, m, 12)
    wq, ws = O.split(fmt, W, n, k)
    xq, xd = O.quant_q8_0(x)
    r, s = O.gemv(fmt, wq, ws, xq, xd, n, k)
    dw = [[X.f16_from_bits(int(v)) for v in row] for row in ws.view(np.uint16)]
    for i in range(m):
        for j in range(n):
            terms = [dw[j][b] * X.f32(xd[i, b]) * int(s[i, j, b]) for b in range(k // 32)]
            exact_sum = sum(terms, Fraction(0))
            bound = len(terms) * 2.0**-52 * float(sum(abs(t) for t in terms))
            assert abs(float(Fraction(r[i, j]) - exact_sum)) <= bound
