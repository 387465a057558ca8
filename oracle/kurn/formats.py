"""kurn.formats, restated for the calls COMP's verification makes -- TEST INFRASTRUCTURE ONLY.

split_blocks  src/komp/verify.py:59,65,85,107   (block bytes of a buffer, per format)
_vals_q4_0    src/komp/verify.py:59             (the 32 values of one q4_0 block)
reference_dot src/komp/verify.py:90 and :103-120 (f64 dot of one weight row with one activation column, in block order)
"""

import struct

import numpy as np

from oracle import oracle as O

BLOCK_BYTES = {"q4_0": 18, "tq2_0": 66, "q8_0": 34, "q8_K": 292}


def split_blocks(fmt, data):
    """bytes -> list of per-block byte strings."""
    nb = BLOCK_BYTES[fmt]
    data = bytes(data)
    if len(data) % nb:
        raise ValueError(f"{fmt}: {len(data)} bytes is not a whole number of {nb}-byte blocks")
    return [data[i : i + nb] for i in range(0, len(data), nb)]


def _vals_q4_0(block):
    """The 32 int values of one q4_0 block: value i = (byte 2+i & 15) - 8, value 16+i = (byte 2+i >> 4) - 8."""
    return [int(v) for v in O.q4_0_values(np.frombuffer(bytes(block), np.uint8)[2:18])]


def _vals_tq2_0(block):
    return [int(v) for v in O.tq2_0_values(np.frombuffer(bytes(block), np.uint8)[:64])]


def _dot_block(fmt, w, x):
    if fmt == "q4_0":
        wv = _vals_q4_0(w)
        xv = struct.unpack_from("<32b", x, 2)
        return struct.unpack_from("<e", w, 0)[0] * struct.unpack_from("<e", x, 0)[0] * sum(a * b for a, b in zip(wv, xv))
    wv = _vals_tq2_0(w)
    xv = struct.unpack_from("<256b", x, 4)
    return struct.unpack_from("<f", x, 0)[0] * struct.unpack_from("<e", w, 64)[0] * sum(a * b for a, b in zip(wv, xv))


def reference_dot(fmt, wbl, xbl):
    """Sum over blocks, in order, of the block's scales times its exact integer dot, in Python floats (f64).

    q4_0: f16 d_w * f16 d_x * s; tq2_0: f32 d_x * f16 d_w * s -- the operation order COMP's rebuild follows
    (src/komp/verify.py:115-118), which it states is bit-identical to this function's."""
    if len(wbl) != len(xbl):
        raise ValueError("weight and activation block counts differ")
    total = 0.0
    for w, x in zip(wbl, xbl):
        total += _dot_block(fmt, w, x)
    return total
