"""Verification of the gfx950 decode kernels against KURN's exact references ("komp verify" semantics).

Restates src/komp/verify.py:1-170 on hardware.  Checks, per problem (random and extreme data; row, column and K-step
tails):
  dp4a    v_dot4c_i32_i8 and the emulated dp4a == the dp4a.s32.s32 definition, on edge and random words
  quant   activation blocks from the HIP quantizers == ggml's reference quantizers (kurn.gpu.ref), byte for byte
  decode  the Q4_0 and TQ2_0 decode kernels == KURN's reference values (kurn.formats), every value
  idots   the GEMV's int32 block dots == the exact integer dots of KURN's reference values, bit for bit; and
          kurn.formats.reference_dot rebuilt from them (same float operations, same order) is bit-identical
  output  f32 Y vs the exact reference: relative error <= TOL (KURN's rule; the f32 accumulation order differs)

The reference runs in the Triton interpreter, with dp4a through its fallback (mode 1); here every mode runs on the GPU:
0 bytes, 1 emulated dp4a, 2 v_dot4c_i32_i8.

KURN's references come from the `kurn` package, imported lazily as in the reference (src/komp/verify.py:23-24).
"""

from __future__ import annotations

import random
import struct

import numpy as np
import torch

from . import host

TOL = 1e-5
MODE_NAMES = {0: "bytes", 1: "dp4a-emulated", 2: "dp4a-sdot4"}


class ReferencesMissing(RuntimeError):
    """KURN's exact references (kurn.formats, kurn.gpu.ref) are not importable."""


def _kurn():
    try:
        from kurn import formats
        from kurn.gpu import ref
    except ImportError as e:
        raise ReferencesMissing(f"komp verify needs KURN's references (kurn.formats, kurn.gpu.ref): {e}") from e
    return formats, ref


def _need_device():
    if not torch.cuda.is_available():
        raise RuntimeError("komp verify runs the HIP kernels: no HIP device is visible")


def dp4a_ref(a, b, c):
    """dp4a.s32.s32: c + sum of the products of the four signed bytes of a and b (int32 wraparound)."""
    sb = lambda v, i: ((v >> (8 * i)) & 0xFF) - (256 if (v >> (8 * i)) & 0x80 else 0)  # noqa: E731
    r = c + sum(sb(a, i) * sb(b, i) for i in range(4))
    return (r + 2**31) % 2**32 - 2**31


def check_dp4a(seed=0, n=1024, modes=(1, 2)):
    """Edge and random words through the dp4a probe kernel, in each mode, vs dp4a_ref (src/komp/verify.py:44-54)."""
    _need_device()
    rng = random.Random(seed)
    edge = [0, -1, 0x7F7F7F7F, -0x7F7F7F80, 0x01010101, 0x0F0F0F0F, 0x03030303, 2**31 - 1, -(2**31), 0x80000000 - 2**32]
    vals = lambda: [rng.choice(edge) if rng.random() < 0.3 else rng.randrange(-(2**31), 2**31) for _ in range(n)]  # noqa: E731
    a, b = vals(), vals()
    c = [rng.randrange(-(2**20), 2**20) for _ in range(n)]
    want = [dp4a_ref(x, y, z) for x, y, z in zip(a, b, c)]
    dev = lambda v: torch.tensor(v, dtype=torch.int32, device="cuda")  # noqa: E731
    ok = True
    for mode in modes:
        out = host.dp4a_probe(dev(a), dev(b), dev(c), mode)
        ok = ok and out.cpu().tolist() == want
    return ok


def q4_0_values(W, n, k):
    """KURN's reference values (kurn.formats._vals_q4_0) -> int32 [n][k]."""
    formats, _ = _kurn()
    return np.array([formats._vals_q4_0(b) for b in formats.split_blocks("q4_0", W)], dtype=np.int32).reshape(n, k)


def tq2_0_values(W, nblk):
    """Values q - 1 of every tq2_0 block, in KURN's reference order -> int32 [nblk][256] (src/komp/verify.py:62-67)."""
    formats, _ = _kurn()
    out = np.empty((nblk, 256), dtype=np.int32)
    for b, w in enumerate(formats.split_blocks("tq2_0", W)):
        out[b] = [((w[(v // 128) * 32 + v % 32] >> (2 * ((v % 128) // 32))) & 3) - 1 for v in range(256)]
    return out


def check_decode(seed=0, extreme=False):
    """Decode kernels vs KURN's values; a TQ2_0 dot built from the decoded values == reference_dot exactly
    (src/komp/verify.py:70-91)."""
    _need_device()
    formats, ref = _kurn()
    rng = random.Random(seed)
    res = {}
    W = ref.weight_blocks("q4_0", rng, 37, extreme)
    wq, _ = host.split_q4_0(W, 37, 32)
    out = host.q4_0_decode(torch.from_numpy(wq).cuda())
    res["q4_0"] = bool(np.array_equal(out.cpu().numpy(), q4_0_values(W, 37, 32)))
    W = ref.weight_blocks("tq2_0", rng, 5, extreme)
    out = host.tq2_0_decode(torch.from_numpy(host.tq2_0_qplane(W, 5)).cuda()).cpu()
    ok = bool(np.array_equal(out.numpy(), tq2_0_values(W, 5)))
    xb = ref.quant_q8_K(ref.activations(random.Random(seed + 1), 256 * 5, 1, block=256)[0])
    wbl, xbl = formats.split_blocks("tq2_0", W), formats.split_blocks("q8_K", xb)
    total = 0.0
    for b in range(5):
        s = int(sum(int(a) * q for a, q in zip(out[b].tolist(), struct.unpack_from("<256b", xbl[b], 4))))
        total += struct.unpack_from("<f", xbl[b], 0)[0] * struct.unpack_from("<e", wbl[b], 64)[0] * s
    res["tq2_0"] = ok and total == formats.reference_dot("tq2_0", wbl, xbl)
    return res


def exact_idots(fmt, W, xq, n, k):
    """Exact int64 block dots [M][N][blocks] of KURN's reference weight values with the int8 activations."""
    blk = host.FORMATS[fmt]["block"]
    vals = q4_0_values(W, n, k) if fmt == "q4_0" else tq2_0_values(W, n * k // 256).reshape(n, k)
    v = vals.reshape(n, k // blk, blk).astype(np.int64)
    q = np.asarray(xq).reshape(-1, k // blk, blk).astype(np.int64)
    return np.einsum("nbi,mbi->mnb", v, q)


def rebuild_reference(fmt, W, xb, s, n, k, m):
    """kurn.formats.reference_dot for every output with each block's integer dot taken from `s`: the same float
    operations in the same order (src/komp/verify.py:103-120), so equal integer dots give a bit-identical result."""
    formats, _ = _kurn()
    f = host.FORMATS[fmt]
    wbl, xbl = formats.split_blocks(fmt, W), formats.split_blocks(f["act"], xb)
    nb = k // f["block"]
    out = []
    for i in range(m):
        for r in range(n):
            total = 0.0
            for b in range(nb):
                w, x, sv = wbl[r * nb + b], xbl[i * nb + b], int(s[i, r, b])
                if fmt == "q4_0":
                    total += struct.unpack_from("<e", w, 0)[0] * struct.unpack_from("<e", x, 0)[0] * sv
                else:
                    total += struct.unpack_from("<f", x, 0)[0] * struct.unpack_from("<e", w, 64)[0] * sv
            out.append(total)
    return out


def check_gemv(fmt, n, k, m, seed=0, extreme=False, block_n=32, nb=4, mode=0, num_warps=4):
    """One problem through the HIP quantizer + GEMV.  Returns a dict of results (src/komp/verify.py:123-137)."""
    _need_device()
    _, ref = _kurn()
    W, x = ref.problem(fmt, n, k, m, seed, extreme)
    wq, ws = host.split(fmt, W, n, k)
    xq, xd = host.quantize(fmt, torch.tensor(np.asarray(x), dtype=torch.float32, device="cuda"))
    xq_h, xd_h = xq.cpu().numpy(), xd.cpu().numpy()
    xb = host.act_blocks(fmt, xq_h, xd_h)
    quant_ok = xb == ref.act_blocks(fmt, x)
    y, s = host.gemv(fmt, torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(), xq, xd, n, k, block_n, nb, mode,
                     num_warps, store_s=True)  # fmt: skip
    s = s.cpu().numpy()
    idots_ok = bool(np.array_equal(s.astype(np.int64), exact_idots(fmt, W, xq_h, n, k)))
    rf = ref.reference(fmt, W, xb, n, k, m)
    rebuilt_ok = rebuild_reference(fmt, W, xb, s, n, k, m) == list(rf)
    err = ref.relerr(y.cpu().numpy().reshape(-1).tolist(), rf)
    return {"fmt": fmt, "n": n, "k": k, "m": m, "quant": quant_ok, "idots": idots_ok, "rebuilt": rebuilt_ok, "relerr": err,
            "ok": quant_ok and idots_ok and rebuilt_ok and err <= TOL}  # fmt: skip


# shapes: row tails (n not a multiple of block_n), K steps not a multiple of nb blocks, several columns
PROBLEMS = {"q4_0": ((64, 512, 1), (37, 416, 3), (5, 96, 2)), "tq2_0": ((64, 1024, 1), (37, 768, 3), (5, 1280, 2))}
CONFIGS = {"q4_0": ((32, 4, 4), (16, 2, 2), (64, 8, 4)), "tq2_0": ((32, 2, 4), (16, 1, 2), (64, 4, 4))}


def line(r, block_n, nb, nw, mode):
    return (f"{'ok  ' if r['ok'] else 'FAIL'} {r['fmt']:5} gemv {MODE_NAMES[mode]:13} block_n={block_n} nb={nb} warps={nw} "
            f"n={r['n']} k={r['k']} m={r['m']} quant={'exact' if r['quant'] else 'MISMATCH'} "
            f"idots={'exact' if r['idots'] else 'MISMATCH'} reference_dot={'bit-identical' if r['rebuilt'] else 'DIFFERS'} "
            f"relerr={r['relerr']:.1e}")  # fmt: skip


def run_all(log=print, formats_=("q4_0", "tq2_0"), modes=(0, 1, 2)):
    """The full check set: dp4a, decode (random and extreme), every GEMV problem x config x mode x data kind.
    1 + 4 + 2 x 3 x 3 x 3 x 2 = 113 checks with the default three modes.  Returns the failure count."""
    fails = 0
    ok = check_dp4a(seed=3)
    fails += not ok
    log(f"{'ok  ' if ok else 'FAIL'} dp4a v_dot4c_i32_i8 and emulated == dp4a.s32.s32 semantics (1024 edge/random words)")
    for extreme in (False, True):
        for f, ok in check_decode(seed=7, extreme=extreme).items():
            fails += not ok
            log(f"{'ok  ' if ok else 'FAIL'} decode {f:5} {'extreme' if extreme else 'random '} (values == KURN reference)")
    for fmt in formats_:
        for mode in modes:
            for block_n, nb, nw in CONFIGS[fmt]:
                for n, k, m in PROBLEMS[fmt]:
                    for seed, extreme in ((1, False), (2, True)):
                        r = check_gemv(fmt, n, k, m, seed, extreme, block_n, nb, mode, nw)
                        fails += not r["ok"]
                        log(line(r, block_n, nb, nw, mode) + (" extreme" if extreme else ""))
    log(f"{fails} failures")
    return fails
