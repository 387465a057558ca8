"""kurn.gpu.ref, restated for the calls COMP's verification makes -- TEST INFRASTRUCTURE ONLY.

Call sites: src/komp/verify.py:74,79,84,126,130,133,135 and tests/test_komp.py:72.  The generators take the
random.Random the reference passes and draw a numpy seed from it; the streams are this repository's own.
"""

import numpy as np

from oracle import oracle as O

from .. import formats


def _np_rng(rng):
    return np.random.default_rng(rng.getrandbits(64))


def weight_blocks(fmt, rng, nblocks, extreme=False):
    """ggml blocks of one row of `nblocks` blocks (bytes)."""
    return O.weights(fmt, _np_rng(rng), 1, nblocks * O.FORMATS[fmt]["block"], extreme)


def weights(fmt, rng, n, k, extreme=False):
    """ggml blocks of an n x k matrix (bytes)."""
    return O.weights(fmt, _np_rng(rng), n, k, extreme)


def activations(rng, k, m, block=32, extreme=False):
    """f32 activations [m][k] (numpy)."""
    return O.activations(_np_rng(rng), k, m, block=block, extreme=extreme)


def quant_q8_0(x):
    """ggml q8_0 blocks (bytes) of one activation row, ggml quantize_row_q8_0_ref."""
    xq, xd = O.quant_q8_0(np.asarray(x, np.float32).reshape(1, -1))
    return O.q8_0_blocks(xq, xd)


def quant_q8_K(x):
    """ggml q8_K blocks (bytes) of one activation row, ggml quantize_row_q8_K_ref (with bsums)."""
    xq, xd, xb = O.quant_q8_K(np.asarray(x, np.float32).reshape(1, -1))
    return O.q8_K_blocks(xq, xd, xb)


def problem(fmt, n, k, m, seed, extreme=False):
    """(W ggml blocks, x f32 [m][k]) for one GEMV problem."""
    return O.problem(fmt, n, k, m, seed, extreme)


def act_blocks(fmt, x):
    """ggml activation blocks (bytes) of every column of x, by the reference quantizer of the format."""
    x = np.asarray(x, np.float32)
    xq, xd, xb = O.quantize(fmt, x)
    return O.act_blocks(fmt, xq, xd, xb)


def reference(fmt, W, xb, n, k, m):
    """formats.reference_dot for every output, column-major ([i * n + r]), from weight and activation block bytes."""
    f = O.FORMATS[fmt]
    nb = k // f["block"]
    wbl = formats.split_blocks(fmt, W)
    xbl = formats.split_blocks(f["act"], xb)
    return [formats.reference_dot(fmt, wbl[r * nb : (r + 1) * nb], xbl[i * nb : (i + 1) * nb]) for i in range(m)
            for r in range(n)]  # fmt: skip


def relerr(y, r):
    """Norm-wise relative error (the formula of KURN's own relerr is not available: parity unpinned)."""
    return O.relerr(y, r)
