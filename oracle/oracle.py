"""CPU oracle for COMP's decode path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the thing measured or shipped: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it.  The product path (`comp_amd`) never imports anything under `oracle/`
and fails loudly when its HIP library is missing.

It restates, in numpy, the arithmetic of the reference decode path (COMP, package `komp`):

  * the format helpers of `triton.language.extra.kurn`   patches/0001-language-extra-kurn.patch:33-131
  * the split layouts and ggml block packing               src/komp/host.py:9-56
  * the exact integer block dots and the f64 rebuild       src/komp/verify.py:37-41, 57-67, 94-120
  * the GEMV arithmetic (int32 block dot, then f32 scale)  src/komp/kernels.py:48-142
  * the synthetic problem generators of the workload list (seeded numpy; the reference's own generators live in the
    absent `kurn.gpu.ref`, so the random streams are this repository's own)

How each function is pinned (tests/test_oracle_pins.py):

  f16_bits_to_f32        all 65536 bit patterns vs IEEE binary16 decoded from its fields with exact rationals
  q4_0_values            all 256 byte values vs the per-value formula; ggml q4_0 quantize->decode round trip
  q8_0_values            all 256 byte values vs struct's signed-byte decode of ggml block_q8_0 bytes
  iq4_nl_values          all 256 byte values at both nibble positions vs a per-byte loop over ggml block_iq4_nl
                         bytes; the table itself (ggml's kvalues_iq4nl) is parity unpinned: KURN, where COMP's
                         formats would be defined, is absent, so the table restates ggml's published constant
  tq2_0_values           all 256 byte values at every crumb position vs a per-value loop over the layout text
  q4_k_values            all 256 byte values at 5 positions vs the dequantizer's loop order; random blocks
  q4_k_scales            all 256 values of each of the 12 bytes vs two independent formulations (bit fields of the
                         96-bit integer; ggml vec_dot's dword masks)
  q4_k_block_dots        (sd, sm) vs brute-force loops over struct-built block_q4_K bytes, and d*dx*sd - dmin*dx*sm
                         equal, in exact rationals, to the dot of the dequantized weights; a known-answer block
  dp4a                   the reference's 11 edge words + random words vs an independent struct-based byte dot
  round_half_*           vs Python's round()/Fraction on ties, negatives, huge and subnormal values
  quant_q8_0 / q8_K      vs an exact-rational (fractions.Fraction) implementation with explicit IEEE f32 rounding,
                         plus known answers (amax 127 -> d 1, ties, zero blocks, first-index ties, spikes)
  block_dots             vs brute-force Python integer loops on tiny shapes, plus bilinearity
  reference_dot          each term is exact in f64 (proved in the docstring) so tests compare the sum against
                         math.fsum-free sequential Fraction sums rounded per step
  relerr                 parity unpinned: KURN's `relerr` formula is in the absent `kurn` package; it is only
                         reported (the reference's `komp verify` line prints it), no output check rests on it
  output_error_bound     every device output is gated by it: f32 simulations in five summation orders (sequential,
                         reversed, pairwise, lane-strided like the kernels, fused multiply-add) stay within it on
                         random and extreme problems, and planted mistakes (a shifted scale index, a dropped block,
                         flushed subnormal scales, a flipped sign, another column's d_x) break it
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------------------------------------------------
# formats (src/komp/host.py:9-13)

FORMATS = {
    "q4_0": dict(block=32, nbytes=18, qoff=2, qbytes=16, soff=0, act="q8_0"),
    "tq2_0": dict(block=256, nbytes=66, qoff=0, qbytes=64, soff=64, act="q8_K"),
    # ggml formats the reference lists as next (README.md:143), restated from ggml's published block layouts
    # (ggml-common.h: block_q8_0 = f16 d + 32 int8; block_iq4_nl = f16 d + 16 bytes of 4-bit table indices)
    "q8_0": dict(block=32, nbytes=34, qoff=2, qbytes=32, soff=0, act="q8_0"),
    "iq4_nl": dict(block=32, nbytes=18, qoff=2, qbytes=16, soff=0, act="q8_0"),
    # block_q4_K = f16 d, f16 dmin, 12 bytes of 6-bit sub-block scales and mins, 128 quant bytes; its split keeps the
    # first 16 bytes (d, dmin, scales) as the scale plane: WS int16 [n][8 * blocks]
    "q4_k": dict(block=256, nbytes=144, qoff=16, qbytes=128, soff=0, sbytes=16, act="q8_K"),
}
for _f in FORMATS.values():
    _f.setdefault("sbytes", 2)  # scale-plane bytes per block
# ggml's IQ4_NL value table (ggml-common.h kvalues_iq4nl): a fixed non-uniform 4-bit grid
IQ4_NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int32)
ACT_BLOCK = {"q8_0": 32, "q8_K": 256}


def f16_bits_to_f32(bits):
    """int16/uint16 fp16 bit patterns -> f32, exact (patch:33-36)."""
    return np.asarray(bits).astype(np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------------------------------------------------
# weight decode (patch:16-19, 39-63; src/komp/verify.py:57-67)


def q4_0_values(qs):
    """[..., 16] q4_0 quant bytes -> [..., 32] int32: value i = (byte i & 15) - 8, value i+16 = (byte i >> 4) - 8."""
    qs = np.asarray(qs, dtype=np.uint8)
    lo = (qs & 15).astype(np.int32) - 8
    hi = (qs >> 4).astype(np.int32) - 8
    return np.concatenate([lo, hi], axis=-1)


def q8_0_values(qs):
    """[..., 32] q8_0 quant bytes -> [..., 32] int32: value i = byte i as a signed int8 (ggml dequantize_row_q8_0)."""
    return np.asarray(qs, dtype=np.uint8).view(np.int8).astype(np.int32)


def iq4_nl_values(qs):
    """[..., 16] iq4_nl quant bytes -> [..., 32] int32: value i = table[byte i & 15], value i+16 = table[byte i >> 4]
    (ggml dequantize_row_iq4_nl: the Q4_0 nibble order with the non-uniform table in place of nibble - 8)."""
    qs = np.asarray(qs, dtype=np.uint8)
    return np.concatenate([IQ4_NL_VALUES[qs & 15], IQ4_NL_VALUES[qs >> 4]], axis=-1)


def q4_k_values(qs):
    """[..., 128] q4_k quant bytes -> [..., 256] int32 in 0..15: byte 32j + l holds value 64j + l in its low nibble
    and value 64j + 32 + l in its high nibble (ggml dequantize_row_q4_K)."""
    qs = np.asarray(qs, dtype=np.uint8)
    g = qs.reshape(*qs.shape[:-1], 4, 32)
    v = np.stack([g & 15, g >> 4], axis=-2)  # [.., j, half, l] -> value 64j + 32 half + l
    return v.reshape(*qs.shape[:-1], 256).astype(np.int32)


def q4_k_scales(sc12):
    """[..., 12] packed scale bytes of block_q4_K -> (scales [..., 8], mins [..., 8]) int32 in 0..63, ggml's
    get_scale_min_k4: sub-block i < 4 takes the low 6 bits of byte i (scale) and byte i + 4 (min); i >= 4 takes the
    low (scale) / high (min) nibble of byte i + 4 and, as bits 4..5, the top two bits of byte i - 4 (scale) / byte i
    (min)."""
    q = np.asarray(sc12, dtype=np.uint8).astype(np.int32)
    sc = np.empty(q.shape[:-1] + (8,), dtype=np.int32)
    mn = np.empty_like(sc)
    for i in range(8):
        if i < 4:
            sc[..., i] = q[..., i] & 63
            mn[..., i] = q[..., i + 4] & 63
        else:
            sc[..., i] = (q[..., i + 4] & 0xF) | ((q[..., i - 4] >> 6) << 4)
            mn[..., i] = (q[..., i + 4] >> 4) | ((q[..., i] >> 6) << 4)
    return sc, mn


def tq2_0_values(qs):
    """[..., 64] tq2_0 quant bytes -> [..., 256] int32.

    Byte h*32+i holds value h*128 + j*32 + i at bits 2j..2j+1; value = crumb - 1 (crumb 3 decodes to +2)."""
    qs = np.asarray(qs, dtype=np.uint8)
    q = qs.reshape(*qs.shape[:-1], 2, 1, 32).astype(np.int32)  # [.., h, 1, i]
    sh = (2 * np.arange(4, dtype=np.int32)).reshape(1, 4, 1)  # [1, j, 1]
    v = ((q >> sh) & 3) - 1  # [.., h, j, i] -> value h*128 + j*32 + i
    return v.reshape(*qs.shape[:-1], 256)


# ---------------------------------------------------------------------------------------------------------------------
# dp4a (patch:66-81; src/komp/verify.py:37-41)


def dp4a(a, b, c):
    """c + sum of the four signed-byte products of int32 words a and b, with int32 wraparound (dp4a.s32.s32)."""
    a = np.asarray(a, dtype=np.int64) & 0xFFFFFFFF
    b = np.asarray(b, dtype=np.int64) & 0xFFFFFFFF
    r = np.asarray(c, dtype=np.int64).copy()
    for i in range(4):
        sa = (a >> (8 * i)) & 0xFF
        sb = (b >> (8 * i)) & 0xFF
        sa = np.where(sa >= 128, sa - 256, sa)
        sb = np.where(sb >= 128, sb - 256, sb)
        r = r + sa * sb
    return (((r + 2**31) % 2**32) - 2**31).astype(np.int32)


# ---------------------------------------------------------------------------------------------------------------------
# exact rounding (patch:84-101), in f32


def round_half_away(x):
    """roundf(): nearest integer, halfway cases away from zero, exact for every f32 (patch:84-90)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x)
    f = np.floor(a)
    r = np.where(a - f >= np.float32(0.5), f + np.float32(1.0), f)
    return np.where(x < 0, -r, r).astype(np.float32)


def round_half_even(x):
    """nearbyint() in round-to-nearest-even mode, exact for every f32 (patch:93-101)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x)
    f = np.floor(a)
    d = a - f
    odd = (f - np.float32(2.0) * np.floor(f * np.float32(0.5))) != 0
    r = np.where((d > np.float32(0.5)) | ((d == np.float32(0.5)) & odd), f + np.float32(1.0), f)
    return np.where(x < 0, -r, r).astype(np.float32)


# ---------------------------------------------------------------------------------------------------------------------
# activation quantizers (patch:104-131; src/komp/kernels.py:22-45; src/komp/host.py:43-52)


def quant_q8_0(x):
    """f32 [M][K] -> (XQ int8 [M][K], XD f32 [M][K/32]) as ggml quantize_row_q8_0_ref.

    Per block of 32: amax = max|x|; d = amax / 127 (f32, round to nearest); id = 1/d (0 when d == 0);
    q = roundf(x * id) computed with the unrounded d; XD stores f32(f16(d)) (patch:104-114, kernels.py:33)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    assert k % 32 == 0
    xb = x.reshape(m, k // 32, 32)
    amax = np.max(np.abs(xb), axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    nz = d != 0
    idv = np.where(nz, np.float32(1.0) / np.where(nz, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    q = round_half_away((xb * idv[:, :, None]).astype(np.float32))
    xq = q.astype(np.int32).astype(np.int8).reshape(m, k)
    with np.errstate(over="ignore"):
        xd = d.astype(np.float16).astype(np.float32)
    return xq, xd


def quant_q8_K(x):
    """f32 [M][K] -> (XQ int8 [M][K], XD f32 [M][K/256], XB int16 [M][K/16]) as ggml quantize_row_q8_K_ref.

    Per block of 256: amax = max|x|, mx = x at the FIRST index where |x| == amax; all-zero block -> q = 0, d = 0;
    else iscale = -127 / mx, q = min(127, nearest-even(iscale * x)), d = 1 / iscale (patch:117-131).
    XB are the bsums, the sums of each 16 consecutive q (src/komp/host.py:50)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    assert k % 256 == 0
    xb = x.reshape(m, k // 256, 256)
    ax = np.abs(xb)
    amax = ax.max(axis=2)
    first = np.argmax(ax == amax[:, :, None], axis=2)  # argmax returns the first True
    mx = np.take_along_axis(xb, first[:, :, None], axis=2)[:, :, 0]
    nz = amax != 0
    iscale = (np.float32(-127.0) / np.where(nz, mx, np.float32(1.0))).astype(np.float32)
    q = np.minimum(round_half_even((iscale[:, :, None] * xb).astype(np.float32)), np.float32(127.0))
    q = np.where(nz[:, :, None], q, np.float32(0.0)).astype(np.int32)
    d = np.where(nz, (np.float32(1.0) / iscale).astype(np.float32), np.float32(0.0)).astype(np.float32)
    xq = q.astype(np.int8).reshape(m, k)
    xbs = q.reshape(m, k // 16, 16).sum(axis=2).astype(np.int16)
    return xq, d, xbs


# ---------------------------------------------------------------------------------------------------------------------
# split planes and ggml blocks (src/komp/host.py:16-56)


def split(fmt, W, n, k):
    """ggml weight blocks (bytes, n rows) -> (WQ uint8 [n][quant bytes per row], WS int16 [n][blocks])."""
    f = FORMATS[fmt]
    nb = k // f["block"]
    blocks = np.frombuffer(bytes(W), dtype=np.uint8).reshape(n, nb, f["nbytes"])
    wq = np.ascontiguousarray(blocks[:, :, f["qoff"] : f["qoff"] + f["qbytes"]]).reshape(n, nb * f["qbytes"])
    sb = f["sbytes"]
    ws = np.ascontiguousarray(blocks[:, :, f["soff"] : f["soff"] + sb]).view(np.int16).reshape(n, nb * sb // 2)
    return wq, ws


def join(fmt, wq, ws):
    """Inverse of split: split planes -> ggml block bytes."""
    f = FORMATS[fmt]
    sb = f["sbytes"]
    n = ws.shape[0]
    nb = ws.shape[1] * 2 // sb
    out = np.zeros((n, nb, f["nbytes"]), dtype=np.uint8)
    out[:, :, f["qoff"] : f["qoff"] + f["qbytes"]] = np.asarray(wq, np.uint8).reshape(n, nb, f["qbytes"])
    out[:, :, f["soff"] : f["soff"] + sb] = np.ascontiguousarray(ws, dtype=np.int16).view(np.uint8).reshape(n, nb, sb)
    return out.tobytes()


def q8_0_blocks(xq, xd):
    """q8_0 split planes -> ggml q8_0 blocks: f16 d then 32 int8 per block (34 bytes)."""
    xq = np.asarray(xq, np.int8)
    m, k = xq.shape
    out = np.empty((m, k // 32, 34), dtype=np.uint8)
    out[:, :, :2] = np.asarray(xd, np.float32).astype(np.float16).view(np.uint8).reshape(m, k // 32, 2)
    out[:, :, 2:] = xq.view(np.uint8).reshape(m, k // 32, 32)
    return out.tobytes()


def q8_K_blocks(xq, xd, xb=None):
    """q8_K split planes -> ggml q8_K blocks: f32 d, 256 int8, 16 int16 bsums (292 bytes)."""
    xq = np.asarray(xq, np.int8)
    m, k = xq.shape
    nb = k // 256
    out = np.empty((m, nb, 292), dtype=np.uint8)
    out[:, :, :4] = np.asarray(xd, np.float32).view(np.uint8).reshape(m, nb, 4)
    out[:, :, 4:260] = xq.view(np.uint8).reshape(m, nb, 256)
    if xb is None:
        xb = xq.astype(np.int32).reshape(m, nb, 16, 16).sum(-1).astype(np.int16)
    out[:, :, 260:] = np.ascontiguousarray(xb, dtype=np.int16).view(np.uint8).reshape(m, nb, 32)
    return out.tobytes()


def act_blocks(fmt, xq, xd, xb=None):
    if FORMATS[fmt]["act"] == "q8_0":
        return q8_0_blocks(xq, xd)
    return q8_K_blocks(xq, xd, xb)


# ---------------------------------------------------------------------------------------------------------------------
# GEMV references (src/komp/verify.py:94-120; src/komp/kernels.py:48-142)


def weight_values(fmt, wq, n, k):
    """Split quant plane -> int32 weight values [n][k]."""
    wq = np.asarray(wq, np.uint8).reshape(n, -1)
    if fmt == "q4_0":
        return q4_0_values(wq[:, : k // 2].reshape(n, k // 32, 16)).reshape(n, k)
    if fmt == "iq4_nl":
        return iq4_nl_values(wq[:, : k // 2].reshape(n, k // 32, 16)).reshape(n, k)
    if fmt == "q8_0":
        return q8_0_values(wq[:, :k]).reshape(n, k)
    if fmt == "q4_k":
        return q4_k_values(wq[:, : k // 2].reshape(n, k // 256, 128)).reshape(n, k)
    return tq2_0_values(wq[:, : k // 4].reshape(n, k // 256, 64)).reshape(n, k)


def q4_k_block_dots(wq, ws, xq, n, k):
    """Exact int64 Q4_K block dots S[m][n][b] = (sd, sm): sd = sum_i sc_i * (sum over sub-block i of q * x), sm =
    sum_i m_i * (sum over sub-block i of x), with q the 4-bit values, x the q8_K activations and (sc_i, m_i) the
    6-bit scale and min of the 32-value sub-block i (ggml vec_dot_q4_K_q8_K's integer sums; its mins term uses the
    q8_K bsums, whose pairs are these sub-block sums)."""
    nb = k // 256
    v = weight_values("q4_k", wq, n, k).reshape(n, nb, 8, 32).astype(np.int64)
    q = np.asarray(xq, np.int8).reshape(-1, nb, 8, 32).astype(np.int64)
    meta = np.ascontiguousarray(ws, dtype=np.int16).view(np.uint8).reshape(n, nb, 16)
    sc, mn = q4_k_scales(meta[:, :, 4:])
    dots = np.einsum("nbil,mbil->mnbi", v, q)
    sd = np.einsum("mnbi,nbi->mnb", dots, sc.astype(np.int64))
    sm = np.einsum("mbi,nbi->mnb", q.sum(-1), mn.astype(np.int64))
    return np.stack([sd, sm], axis=-1)


def block_dots(fmt, wq, xq, n, k, ws=None):
    """Exact int64 block dots S[m][n][b] = sum_i w(n, b*blk + i) * q(m, b*blk + i) (verify.py:94-100); q4_k (whose
    sums need the scale plane ws): S[m][n][b] = (sd, sm) of q4_k_block_dots."""
    if fmt == "q4_k":
        return q4_k_block_dots(wq, ws, xq, n, k)
    blk = FORMATS[fmt]["block"]
    v = weight_values(fmt, wq, n, k).reshape(n, k // blk, blk).astype(np.int64)
    q = np.asarray(xq, np.int8).reshape(-1, k // blk, blk).astype(np.int64)
    return np.einsum("nbi,mbi->mnb", v, q)


def reference_dot(fmt, ws, xd, s):
    """f64 reference outputs [M][N], summed block by block in order (verify.py:103-120).

    q4_0 adds f16(dw) * f16(dx) * s, tq2_0 adds f32(dx) * f16(dw) * s, left to right, in Python-float (f64)
    arithmetic.  Both products are exact in f64 (11+11+22 and 24+11+16 significant bits), so only the running
    sum rounds, and the result depends on the block order alone.  q8_0 and iq4_nl weights take q4_0's form (ggml's
    vec_dot_q8_0_q8_0 and vec_dot_iq4_nl_q8_0 scale the int block dot by f16(dw) * f16(dx)); their block dots stay
    below 2**22 in magnitude, so the products are exact there too."""
    dx = np.asarray(xd, np.float32).astype(np.float64)  # [M][nb]
    s = np.asarray(s, dtype=np.int64)
    if fmt == "q4_k":
        # y = sum_b f16(d) * dx * sd - f16(dmin) * dx * sm (ggml vec_dot_q4_K_q8_K), each term in f64: the products
        # are not all exact there (sd reaches 2**24), which the 1e-5 tolerance of the comparisons covers
        meta = np.ascontiguousarray(ws, dtype=np.int16).reshape(ws.shape[0], -1, 8)
        d = f16_bits_to_f32(meta[:, :, 0]).astype(np.float64)
        dmin = f16_bits_to_f32(meta[:, :, 1]).astype(np.float64)
        m, n, nb, _ = s.shape
        total = np.zeros((m, n), dtype=np.float64)
        for b in range(nb):
            total = total + ((d[None, :, b] * dx[:, None, b]) * s[:, :, b, 0]
                             - (dmin[None, :, b] * dx[:, None, b]) * s[:, :, b, 1])  # fmt: skip
        return total
    dw = f16_bits_to_f32(ws).astype(np.float64)  # [N][nb]
    m, n, nb = s.shape
    total = np.zeros((m, n), dtype=np.float64)
    for b in range(nb):
        if fmt != "tq2_0":
            term = (dw[None, :, b] * dx[:, None, b]) * s[:, :, b]
        else:
            term = (dx[:, None, b] * dw[None, :, b]) * s[:, :, b]
        total = total + term
    return total


def gemv(fmt, wq, ws, xq, xd, n, k):
    """(Y f64 reference [M][N], S int64 [M][N][blocks] ([M][N][blocks][2] for q4_k)) for split planes and q8
    activations."""
    s = block_dots(fmt, wq, xq, n, k, ws)
    return reference_dot(fmt, ws, xd, s), s


def relerr(y, r):
    """Norm-wise relative error max|y - r| / max|r| (0 when both are all zero).

    KURN's own `kurn.gpu.ref.relerr` is in the absent `kurn` package: its formula is parity unpinned.  The norm-wise
    form stays meaningful for outputs that cancel to near zero, where an element-wise ratio would not."""
    y = np.asarray(y, dtype=np.float64).reshape(-1)
    r = np.asarray(r, dtype=np.float64).reshape(-1)
    if y.size == 0:
        return 0.0
    den = float(np.max(np.abs(r)))
    num = float(np.max(np.abs(y - r)))
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


def relerr2(y, r):
    """Norm-wise relative error in the 2-norm, ||y - r||_2 / ||r||_2 (0 when both are all zero): the other norm-wise
    form KURN's relerr may take.  The f32 outputs of the reference's own checks, in its kernels' summation order
    (kernels.py:93, :141, :94), give 5e-8 .. 2e-7 under either form and up to 7e-3 element-wise on extreme data
    (README.md:107-108 publishes 5e-8 .. 2e-7 with 0 failures under the 1e-5 rule), which rules the element-wise form
    out; tests/test_relerr_form.py holds that check."""
    y = np.asarray(y, dtype=np.float64).reshape(-1)
    r = np.asarray(r, dtype=np.float64).reshape(-1)
    if y.size == 0:
        return 0.0
    den = float(np.linalg.norm(r))
    num = float(np.linalg.norm(y - r))
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / den


# ---------------------------------------------------------------------------------------------------------------------
# per-output error bound of an f32 evaluation (the gate every device output passes)

F32_UNIT = 2.0**-24          # unit roundoff of f32 round-to-nearest
F64_UNIT = 2.0**-53
F32_HALF_MIN = 2.0**-150     # half the smallest f32 subnormal: a product's absolute rounding error below 2**-126


def _gamma(n, u):
    """Higham's gamma_n = n u / (1 - n u)."""
    nu = n * u
    return nu / (1.0 - nu)


def output_terms(fmt, ws, xd, s):
    """The exact terms of every output, f64 [M][N][T], and each term's factor magnitudes for the underflow slack.

    Output y[m][n] of the decode GEMV is sum_t term[m][n][t] (kernels.py:93, :141): one term per block,
    s * d_w * d_x; q4_k has two per block, sd * d * d_x and -sm * dmin * d_x (ggml vec_dot_q4_K_q8_K).  The terms
    are exact in f64 (an integer of at most 19 significant bits times an 11-bit f16 scale and an 11-bit q8_0 or a
    24-bit q8_K scale) except q4_k's, whose sd reaches 25 bits and rounds once.  Returns (terms, factor_sum) with
    factor_sum[m][n][t] = |int| + |d_w| + |d_x|."""
    dx = np.asarray(xd, np.float32).astype(np.float64)  # [M][nb]
    s = np.asarray(s, dtype=np.int64)
    if fmt == "q4_k":
        meta = np.ascontiguousarray(ws, dtype=np.int16).reshape(ws.shape[0], -1, 8)
        d = f16_bits_to_f32(meta[:, :, 0]).astype(np.float64)
        dmin = f16_bits_to_f32(meta[:, :, 1]).astype(np.float64)
        sd = s[..., 0].astype(np.float64)
        sm = s[..., 1].astype(np.float64)
        t1 = d[None] * dx[:, None, :] * sd
        t2 = -(dmin[None] * dx[:, None, :] * sm)
        f1 = np.abs(sd) + np.abs(d)[None] + np.abs(dx)[:, None, :]
        f2 = np.abs(sm) + np.abs(dmin)[None] + np.abs(dx)[:, None, :]
        return np.concatenate([t1, t2], axis=-1), np.concatenate([f1, f2], axis=-1)
    dw = f16_bits_to_f32(ws).astype(np.float64)  # [N][nb]
    sf = s.astype(np.float64)
    terms = dw[None] * dx[:, None, :] * sf
    return terms, np.abs(sf) + np.abs(dw)[None] + np.abs(dx)[:, None, :]


def output_error_bound(fmt, ws, xd, s):
    """Bound on |y - r| per output [M][N], for any f32 evaluation y of the GEMV against the f64 reference r.

    The device forms each term as a chain of two f32 multiplications of the exact integer dot (|s| < 2**24, so
    f32(s) is exact) and the two scales, or folds the last multiplication into a fused multiply-add, and adds the
    terms in an order of its own (per-lane running sums, then DPP / LDS trees).  With u = 2**-24 and every f32
    operation fl(x) = x (1 + d) + e, |d| <= u, |e| <= 2**-150 (e only for results below 2**-126; sums that land
    there are exact):
      * a term's product chain: |p - t| <= (2u + u^2) |t| + 2**-150 (1 + |the factor applied last|);
      * any summation tree over n terms: |fl(sum p) - sum p| <= gamma_{n-1} sum |p| (Higham, Accuracy and
        Stability of Numerical Algorithms, 2nd ed., eq. 4.4, which holds for every order);
    so |y - sum t| <= gamma_{n+2} sum |t| + 2 sum_t 2**-150 (1 + |s| + |d_w| + |d_x|).  The reference sums the same
    exact terms in f64 (q4_k's products round there once more): |r - sum t| <= gamma^{f64}_{n+2} sum |t|.
    n is the number of terms (blocks; q4_k two per block)."""
    terms, factors = output_terms(fmt, ws, xd, s)
    n = terms.shape[-1]
    mag = np.abs(terms).sum(axis=-1)
    slack = 2.0 * F32_HALF_MIN * (terms.shape[-1] + factors.sum(axis=-1))
    return (_gamma(n + 2, F32_UNIT) + _gamma(n + 2, F64_UNIT)) * mag + slack


def output_check(fmt, y, ws, xd, s, r):
    """(ok, worst): every output of y within output_error_bound of the f64 reference r; worst = max |y - r| / bound
    over the outputs (0 when all match exactly), inf when an output is not finite or misses a zero bound."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64).reshape(y.shape)
    bound = output_error_bound(fmt, ws, xd, s).reshape(y.shape)
    if y.size == 0:
        return True, 0.0
    if not np.all(np.isfinite(y)):
        return False, float("inf")
    err = np.abs(y - r)
    if np.any((bound == 0.0) & (err > 0.0)):
        return False, float("inf")
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0.0, err / np.where(bound > 0.0, bound, 1.0), 0.0)
    worst = float(ratio.max())
    return worst <= 1.0, worst


# ---------------------------------------------------------------------------------------------------------------------
# weight builders used by the synthetic problems


def quantize_q4_0_weights(w):
    """f32 [n][k] -> ggml q4_0 blocks (bytes), ggml quantize_row_q4_0_ref.

    Per block of 32: max = the signed value of largest |x| (first on ties); d = max / -8; id = 1/d (0 if d == 0);
    q = min(15, trunc(x * id + 8.5)); byte j = q[j] | q[j+16] << 4; f16 d first."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    wb = w.reshape(n, k // 32, 32)
    ax = np.abs(wb)
    first = np.argmax(ax == ax.max(axis=2)[:, :, None], axis=2)
    mx = np.take_along_axis(wb, first[:, :, None], axis=2)[:, :, 0]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    nz = d != 0
    idv = np.where(nz, np.float32(1.0) / np.where(nz, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (wb * idv[:, :, None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(np.trunc(v), np.float32(15.0)).astype(np.int32)
    q = np.clip(q, 0, 15).astype(np.uint8)
    qs = (q[:, :, :16] | (q[:, :, 16:] << 4)).astype(np.uint8)
    out = np.empty((n, k // 32, 18), dtype=np.uint8)
    with np.errstate(over="ignore"):
        out[:, :, :2] = d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    out[:, :, 2:] = qs
    return out.tobytes()


def pack_q4_0(nibbles, d_bits):
    """nibbles uint8 [n][k] in 0..15 (value = nibble - 8) and f16 bit patterns [n][k/32] -> ggml q4_0 blocks."""
    nib = np.asarray(nibbles, np.uint8)
    n, k = nib.shape
    nb = nib.reshape(n, k // 32, 32)
    out = np.empty((n, k // 32, 18), dtype=np.uint8)
    out[:, :, :2] = np.ascontiguousarray(d_bits, dtype=np.uint16).view(np.uint8).reshape(n, k // 32, 2)
    out[:, :, 2:] = (nb[:, :, :16] & 15) | ((nb[:, :, 16:] & 15) << 4)
    return out.tobytes()


def pack_tq2_0(crumbs, d_bits):
    """crumbs uint8 [n][k] in 0..3 (value = crumb - 1) and f16 bit patterns [n][k/256] -> ggml tq2_0 blocks."""
    c = np.asarray(crumbs, np.uint8)
    n, k = c.shape
    cb = c.reshape(n, k // 256, 2, 4, 32)  # value h*128 + j*32 + i
    qs = np.zeros((n, k // 256, 2, 32), dtype=np.uint8)
    for j in range(4):
        qs |= (cb[:, :, :, j, :] & 3) << (2 * j)
    out = np.empty((n, k // 256, 66), dtype=np.uint8)
    out[:, :, :64] = qs.reshape(n, k // 256, 64)
    out[:, :, 64:] = np.ascontiguousarray(d_bits, dtype=np.uint16).view(np.uint8).reshape(n, k // 256, 2)
    return out.tobytes()


def pack_q8_0(q, d_bits):
    """int8 values [n][k] and f16 bit patterns [n][k/32] -> ggml q8_0 blocks (f16 d, then 32 int8)."""
    q = np.asarray(q, np.int8)
    n, k = q.shape
    out = np.empty((n, k // 32, 34), dtype=np.uint8)
    out[:, :, :2] = np.ascontiguousarray(d_bits, dtype=np.uint16).view(np.uint8).reshape(n, k // 32, 2)
    out[:, :, 2:] = q.view(np.uint8).reshape(n, k // 32, 32)
    return out.tobytes()


def pack_q4_k(nibbles, d_bits, dmin_bits, sc12):
    """nibbles uint8 [n][k] in 0..15, f16 bit patterns of d and dmin [n][k/256] and packed scale bytes
    [n][k/256][12] -> ggml q4_K blocks (d, dmin, scales, then value 64j + l / 64j + 32 + l in the low / high nibble
    of byte 32j + l)."""
    nib = np.asarray(nibbles, np.uint8)
    n, k = nib.shape
    nb = k // 256
    g = nib.reshape(n, nb, 4, 2, 32)
    out = np.empty((n, nb, 144), dtype=np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(d_bits, dtype=np.uint16).view(np.uint8).reshape(n, nb, 2)
    out[:, :, 2:4] = np.ascontiguousarray(dmin_bits, dtype=np.uint16).view(np.uint8).reshape(n, nb, 2)
    out[:, :, 4:16] = np.asarray(sc12, np.uint8).reshape(n, nb, 12)
    out[:, :, 16:] = ((g[:, :, :, 0] & 15) | ((g[:, :, :, 1] & 15) << 4)).reshape(n, nb, 128)
    return out.tobytes()


F16_MAX_BITS = 0x7BFF  # 65504
F16_MIN_SUBNORMAL_BITS = 0x0001  # 2**-24


def weights(fmt, rng, n, k, extreme=False):
    """Seeded ggml weight blocks for an n x k matrix.

    random  q4_0: W ~ N(0, 0.02) quantized by ggml's q4_0 rule; tq2_0: trits from {-1, 0, +1} with p 0.3/0.4/0.3,
            d ~ U(0.01, 0.05) rounded to f16; q8_0: W ~ N(0, 0.02) quantized by ggml's q8_0 rule; iq4_nl: uniform
            table indices, d ~ U(0.0005, 0.002).
    extreme per block: f16 d at 65504, at the smallest subnormal 2**-24 or random; values all at the minimum
            (nibble 0 / crumb 0), all at the maximum (nibble 15 / crumb 2), random, or (tq2_0) crumb 3."""
    nb = k // FORMATS[fmt]["block"]
    if fmt == "q8_0":
        if not extreme:  # ggml quantize_row_q8_0_ref of W ~ N(0, 0.02): the activation quantizer's rule
            q, d = quant_q8_0(rng.normal(0.0, 0.02, size=(n, k)).astype(np.float32))
            return pack_q8_0(q, d.astype(np.float16).view(np.uint16))
        q = rng.integers(-128, 128, size=(n, nb, 32)).astype(np.int8)
        kind = rng.integers(0, 4, size=(n, nb))
        q[kind == 1] = -128
        q[kind == 2] = 127
        q[kind == 3] = -127
        d = np.asarray(rng.uniform(-0.05, 0.05, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
        sk = rng.integers(0, 4, size=(n, nb))
        d = np.where(sk == 1, F16_MAX_BITS, np.where(sk == 2, F16_MIN_SUBNORMAL_BITS, d)).astype(np.uint16)
        return pack_q8_0(q.reshape(n, k), d)
    if fmt == "iq4_nl":  # any nibbles are valid table indices; d ~ U(0.0005, 0.002) (values up to 127 * d)
        nib = rng.integers(0, 16, size=(n, nb, 32), dtype=np.uint8)
        d = np.asarray(rng.uniform(0.0005, 0.002, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
        if extreme:
            kind = rng.integers(0, 3, size=(n, nb))
            nib[kind == 1] = 0
            nib[kind == 2] = 15
            sk = rng.integers(0, 4, size=(n, nb))
            d = np.where(sk == 1, F16_MAX_BITS, np.where(sk == 2, F16_MIN_SUBNORMAL_BITS, d)).astype(np.uint16)
        return pack_q4_0(nib.reshape(n, k), d)  # same bytes as Q4_0: index i low nibble, index i+16 high nibble
    if fmt == "q4_k":  # any 12 scale bytes are valid 6-bit scales and mins; d, dmin ~ U(0.0002, 0.001)
        nib = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        sc12 = rng.integers(0, 256, size=(n, nb, 12), dtype=np.uint8)
        d = np.asarray(rng.uniform(0.0002, 0.001, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
        dm = np.asarray(rng.uniform(0.0002, 0.001, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
        if extreme:
            nb4 = nib.reshape(n, nb, 256)
            kind = rng.integers(0, 3, size=(n, nb))
            nb4[kind == 1] = 0
            nb4[kind == 2] = 15
            sk = rng.integers(0, 4, size=(n, nb))
            sc12[sk == 1] = 0xFF  # every scale and min 63
            sc12[sk == 2] = 0
            dk = rng.integers(0, 4, size=(n, nb))
            d = np.where(dk == 1, F16_MAX_BITS, np.where(dk == 2, F16_MIN_SUBNORMAL_BITS, d)).astype(np.uint16)
            mk = rng.integers(0, 4, size=(n, nb))
            dm = np.where(mk == 1, F16_MAX_BITS, np.where(mk == 2, F16_MIN_SUBNORMAL_BITS, dm)).astype(np.uint16)
        return pack_q4_k(nib, d, dm, sc12)
    if fmt == "q4_0" and not extreme:
        return quantize_q4_0_weights(rng.normal(0.0, 0.02, size=(n, k)).astype(np.float32))
    if fmt == "q4_0":
        nib = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
        kind = rng.integers(0, 3, size=(n, nb))
        nibb = nib.reshape(n, nb, 32)
        nibb[kind == 1] = 0
        nibb[kind == 2] = 15
        d = np.asarray(rng.uniform(-0.05, 0.05, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
        sk = rng.integers(0, 4, size=(n, nb))
        d = np.where(sk == 1, F16_MAX_BITS, np.where(sk == 2, F16_MIN_SUBNORMAL_BITS, d)).astype(np.uint16)
        return pack_q4_0(nibb.reshape(n, k), d)
    crumbs = (rng.choice(3, size=(n, k), p=[0.3, 0.4, 0.3])).astype(np.uint8)  # crumb = trit + 1
    d = np.asarray(rng.uniform(0.01, 0.05, size=(n, nb)), np.float32).astype(np.float16).view(np.uint16)
    if extreme:
        cb = crumbs.reshape(n, nb, 256)
        kind = rng.integers(0, 4, size=(n, nb))
        cb[kind == 1] = 0
        cb[kind == 2] = 2
        three = (kind == 3)[:, :, None] & (rng.random(size=(n, nb, 256)) < 0.05)
        cb[three] = 3
        crumbs = cb.reshape(n, k)
        sk = rng.integers(0, 4, size=(n, nb))
        d = np.where(sk == 1, F16_MAX_BITS, np.where(sk == 2, F16_MIN_SUBNORMAL_BITS, d)).astype(np.uint16)
    return pack_tq2_0(crumbs, d)


def activations(rng, k, m, block=32, extreme=False, outliers=0.0):
    """Seeded f32 activations [m][k] ~ N(0, 1).

    outliers: that fraction of entries scaled x20.  extreme per block: all zero, one +-1e4 spike in N(0, 1) noise,
    or random."""
    x = rng.normal(0.0, 1.0, size=(m, k)).astype(np.float32)
    if outliers:
        sel = rng.random(size=(m, k)) < outliers
        x[sel] *= np.float32(20.0)
    if extreme:
        nb = k // block
        xb = x.reshape(m, nb, block)
        kind = rng.integers(0, 3, size=(m, nb))
        xb[kind == 1] = 0.0
        pos = rng.integers(0, block, size=(m, nb))
        sign = np.where(rng.random(size=(m, nb)) < 0.5, -1.0, 1.0).astype(np.float32)
        mi, bi = np.nonzero(kind == 2)
        xb[mi, bi, pos[mi, bi]] = sign[mi, bi] * np.float32(1e4)
        x = xb.reshape(m, k)
    return x


def problem(fmt, n, k, m, seed, extreme=False):
    """(W ggml block bytes, x f32 [m][k]) for one GEMV problem, seeded."""
    rng = np.random.default_rng(seed)
    W = weights(fmt, rng, n, k, extreme)
    x = activations(rng, k, m, block=ACT_BLOCK[FORMATS[fmt]["act"]], extreme=extreme)
    return W, x


def quantize(fmt, x):
    """The activation quantizer for a weight format: q4_0 -> (xq, xd, None); tq2_0 -> (xq, xd, bsums)."""
    if FORMATS[fmt]["act"] == "q8_0":
        xq, xd = quant_q8_0(x)
        return xq, xd, None
    return quant_q8_K(x)
