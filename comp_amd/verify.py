"""`komp verify` for the gfx950 build: the HIP decode kernels against KURN's exact references.

The check set and the report are the reference's (src/komp/verify.py:3-9, 141-170); the way they are computed is this
module's own.  Every check launches the HIP kernels through comp_amd.host and compares them with what KURN provides
(`kurn.gpu.ref` problems, activation blocks and f64 references; `kurn.formats` block splitting, Q4_0 values and
reference_dot).  The integer references are computed here, vectorised over whole blocks, from numpy views of the
ggml block bytes:

  dp4a    the probe kernel in each device mode == the signed-byte dot with int32 wraparound, on edge and random words
  quant   the ggml activation blocks of the HIP quantizer == KURN's reference quantizer blocks, byte for byte
  decode  the Q4_0 / TQ2_0 decode probes == KURN's values (Q4_0) and the TQ2_0 layout's values; a dot through the
          decoded TQ2_0 values, scaled as KURN scales it, == kurn.formats.reference_dot exactly
  idots   the GEMV's int32 block dots == the exact int64 dots of those values with the quantized activations
  rebuilt the f64 sum over blocks of scale products times the GEMV's block dots, one block at a time for a whole
          column of outputs (the per-output operations and order of KURN's reference_dot), == KURN's reference
          bit for bit
  output  Y against KURN's reference: relerr <= TOL, and every output within the f32 error bound of its exact terms
          (an f32 sum of n products can be off by gamma_{n+2} times the sum of their magnitudes; see _output_bound)

Modes: 0 bytes, 1 emulated dp4a, 2 v_dot4c_i32_i8, all on the GPU.  KURN is imported lazily, as the reference does.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch

from . import host

TOL = 1e-5
MODE_NAMES = {0: "bytes", 1: "dp4a-emulated", 2: "dp4a-sdot4"}
# the reference's problem list (row tails, K steps that are not a multiple of nb blocks, several columns) and knob
# sets (block_n, nb, num_warps), src/komp/verify.py:141-142
PROBLEMS = {"q4_0": ((64, 512, 1), (37, 416, 3), (5, 96, 2)), "tq2_0": ((64, 1024, 1), (37, 768, 3), (5, 1280, 2))}
CONFIGS = {"q4_0": ((32, 4, 4), (16, 2, 2), (64, 8, 4)), "tq2_0": ((32, 2, 4), (16, 1, 2), (64, 4, 4))}
DP4A_EDGE_WORDS = (0, -1, 0x7F7F7F7F, -0x7F7F7F80, 0x01010101, 0x0F0F0F0F, 0x03030303, 2**31 - 1, -(2**31),
                   0x80000000 - 2**32)  # fmt: skip  (src/komp/verify.py:47)


class ReferencesMissing(RuntimeError):
    """KURN's exact references (kurn.formats, kurn.gpu.ref) are not importable."""


def _kurn():
    try:
        from kurn import formats
        from kurn.gpu import ref
    except ImportError as e:
        raise ReferencesMissing(f"komp verify needs KURN's references (kurn.formats, kurn.gpu.ref): {e}") from e
    return formats, ref


def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("komp verify runs the HIP kernels: no HIP device is visible")
    return torch.device("cuda", torch.cuda.current_device())


# ---- ggml block bytes as numpy views ---------------------------------------------------------------------------------
# (block bytes, offset and dtype of the scale, offset and count of the quant bytes)
_LAYOUT = {"q4_0": (18, 0, "<f2", 2, 16), "tq2_0": (66, 64, "<f2", 0, 64), "q8_0": (34, 0, "<f2", 2, 32),
           "q8_K": (292, 0, "<f4", 4, 256)}  # fmt: skip


def _blocks(kind, data):
    """(scales f64 [blocks], quant bytes u8 [blocks][q]) of a buffer of ggml blocks of one kind."""
    size, soff, sdt, qoff, qn = _LAYOUT[kind]
    raw = np.frombuffer(bytes(data), np.uint8).reshape(-1, size)
    scale = raw[:, soff : soff + np.dtype(sdt).itemsize].copy().view(sdt)[:, 0].astype(np.float64)
    return scale, raw[:, qoff : qoff + qn]


# TQ2_0 value v of a block sits in byte (v // 128) * 32 + v % 32 at bits 2 * ((v % 128) // 32) (patch:18-19)
_TQ2_BYTE = np.array([(v // 128) * 32 + v % 32 for v in range(256)])
_TQ2_SHIFT = np.array([2 * ((v % 128) // 32) for v in range(256)], dtype=np.uint8)


def weight_values(fmt, W):
    """int32 [blocks][block] values of every weight block: Q4_0 from KURN (kurn.formats._vals_q4_0, the values
    the reference checks against), TQ2_0 from its layout, crumb - 1 (crumb 3 decodes to +2)."""
    formats, _ = _kurn()
    if fmt == "q4_0":
        return np.asarray(list(map(formats._vals_q4_0, formats.split_blocks("q4_0", W))), dtype=np.int32)
    _, qs = _blocks("tq2_0", W)
    return ((qs[:, _TQ2_BYTE] >> _TQ2_SHIFT) & 3).astype(np.int32) - 1


def exact_idots(fmt, W, xq, n, k):
    """Exact int64 block dots [M][N][blocks] of the weight values with the int8 activations xq [M][K]."""
    blk = host.FORMATS[fmt]["block"]
    v = weight_values(fmt, W).reshape(n, k // blk, blk).astype(np.int64)
    q = np.asarray(xq, np.int64).reshape(-1, k // blk, blk)
    return np.einsum("nbv,mbv->mnb", v, q)


def _scales(fmt, W, xb, n, m):
    """(d_w [n][blocks], d_x [m][blocks]) in f64 (exact) from the weight and activation block bytes."""
    dw, _ = _blocks(fmt, W)
    dx, _ = _blocks(host.FORMATS[fmt]["act"], xb)
    return dw.reshape(n, -1), dx.reshape(m, -1)


def rebuild_reference(fmt, W, xb, s, n, k, m):
    """KURN's reference_dot of every output ([i * n + r], as kurn.gpu.ref.reference lists them) with each block's
    integer dot taken from s [M][N][blocks].  Each output is (scale product) * s summed over blocks in order, in f64
    (src/komp/verify.py:103-120), here a whole column of outputs per block; equal block dots give a bit-identical
    result."""
    dw, dx = _scales(fmt, W, xb, n, m)
    s = np.asarray(s, dtype=np.int64).reshape(m, n, -1)
    total = np.zeros((m, n), dtype=np.float64)
    for b in range(s.shape[2]):
        total = total + (dw[None, :, b] * dx[:, None, b]) * s[:, :, b].astype(np.float64)
    return total.reshape(-1).tolist()


def _output_bound(fmt, W, xb, s, n, m):
    """Per-output bound [M][N] on |Y - reference| for any f32 evaluation of Y = sum_b (d_w d_x s)_b: each term is
    two f32 products of exact values (relative error 2u + u^2, u = 2^-24, plus 2^-150 absolute below 2^-126, times
    the factor applied last), any summation tree of n terms adds gamma_{n-1} (Higham, eq. 4.4), and the f64 reference
    sums the same exact terms: gamma_{n+2}(u) + gamma_{n+2}(2^-53) times sum |t|, plus the underflow slack."""
    dw, dx = _scales(fmt, W, xb, n, m)
    s = np.asarray(s, dtype=np.int64).reshape(m, n, -1).astype(np.float64)
    nb = s.shape[2]
    t = np.abs(dw[None] * dx[:, None, :] * s)
    g = lambda nn, u: nn * u / (1.0 - nn * u)  # noqa: E731
    slack = 2.0**-149 * (nb + (np.abs(s) + np.abs(dw)[None] + np.abs(dx)[:, None, :]).sum(-1))
    return (g(nb + 2, 2.0**-24) + g(nb + 2, 2.0**-53)) * t.sum(-1) + slack


def dp4a_expected(a, b, c):
    """c + sum of the four signed-byte products of a and b, wrapped to int32 (PTX dp4a.s32.s32, patch:66-81)."""
    a8 = np.asarray(a, np.int64).astype(np.uint32).view(np.int8).reshape(-1, 4).astype(np.int64)
    b8 = np.asarray(b, np.int64).astype(np.uint32).view(np.int8).reshape(-1, 4).astype(np.int64)
    r = np.asarray(c, np.int64) + (a8 * b8).sum(axis=1)
    return ((r + 2**31) % 2**32 - 2**31).astype(np.int32)


def check_dp4a(seed=0, n=1024, modes=(1, 2)):
    """Edge and random words (30% edge) through the dp4a probe in each device mode."""
    dev = _device()
    rng = np.random.default_rng(seed)

    def words():
        w = rng.integers(-(2**31), 2**31, size=n)
        edge = rng.random(n) < 0.3
        w[edge] = rng.choice(np.asarray(DP4A_EDGE_WORDS, np.int64), size=int(edge.sum()))
        return w.astype(np.int32)

    a, b = words(), words()
    c = rng.integers(-(2**20), 2**20, size=n).astype(np.int32)
    want = dp4a_expected(a, b, c)
    t = [torch.from_numpy(v).to(dev) for v in (a, b, c)]
    return all(np.array_equal(host.dp4a_probe(*t, mode).cpu().numpy(), want) for mode in modes)


def check_decode(seed=0, extreme=False):
    """{"q4_0": ok, "tq2_0": ok}: the decode probes on 37 Q4_0 and 5 TQ2_0 KURN blocks; for TQ2_0 also the dot
    through the decoded values with a q8_K activation row, scaled as KURN scales it, == formats.reference_dot."""
    import random

    dev = _device()
    formats, ref = _kurn()
    rng = random.Random(seed)
    W = ref.weight_blocks("q4_0", rng, 37, extreme)
    got = host.q4_0_decode(torch.from_numpy(host.split_q4_0(W, 37, 32)[0]).to(dev)).cpu().numpy()
    res = {"q4_0": bool(np.array_equal(got, weight_values("q4_0", W)))}
    W = ref.weight_blocks("tq2_0", rng, 5, extreme)
    got = host.tq2_0_decode(torch.from_numpy(host.tq2_0_qplane(W, 5)).to(dev)).cpu().numpy()
    xb = ref.quant_q8_K(ref.activations(random.Random(seed + 1), 256 * 5, 1, block=256)[0])
    dw, _ = _blocks("tq2_0", W)
    dx, q = _blocks("q8_K", xb)
    s = (got.astype(np.int64) * q.view(np.int8).astype(np.int64)).sum(axis=1)
    total = 0.0
    for b in range(5):
        total = total + (float(dx[b]) * float(dw[b])) * float(s[b])
    res["tq2_0"] = bool(np.array_equal(got, weight_values("tq2_0", W))) and total == formats.reference_dot(
        "tq2_0", formats.split_blocks("tq2_0", W), formats.split_blocks("q8_K", xb))
    return res


def check_gemv(fmt, n, k, m, seed=0, extreme=False, block_n=32, nb=4, mode=0, num_warps=4):
    """One KURN problem through the HIP quantizer and GEMV with the given knobs and mode.  Returns the check results
    and the report fields (fmt, n, k, m, quant, idots, rebuilt, relerr, bound, ok)."""
    dev = _device()
    _, ref = _kurn()
    W, x = ref.problem(fmt, n, k, m, seed, extreme)
    wq, ws = host.split(fmt, W, n, k)
    xq, xd = host.quantize(fmt, torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev))
    y, s = host.gemv(fmt, torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev), xq, xd, n, k, block_n, nb, mode,
                     num_warps, store_s=True)  # fmt: skip
    xq_h = xq.cpu().numpy()
    xb = host.act_blocks(fmt, xq_h, xd.cpu().numpy())
    s = s.cpu().numpy().astype(np.int64)
    y = y.cpu().numpy().astype(np.float64)
    reference = ref.reference(fmt, W, xb, n, k, m)
    r = {"fmt": fmt, "n": n, "k": k, "m": m}
    r["quant"] = xb == ref.act_blocks(fmt, x)
    r["idots"] = bool(np.array_equal(s, exact_idots(fmt, W, xq_h, n, k)))
    r["rebuilt"] = rebuild_reference(fmt, W, xb, s, n, k, m) == list(reference)
    r["relerr"] = ref.relerr(y.reshape(-1).tolist(), reference)
    err = np.abs(y - np.asarray(reference, np.float64).reshape(m, n))
    r["bound"] = bool(np.all(np.isfinite(y)) and np.all(err <= _output_bound(fmt, W, xb, s, n, m)))
    r["ok"] = r["quant"] and r["idots"] and r["rebuilt"] and r["relerr"] <= TOL and r["bound"]
    return r


def line(r, block_n, nb, nw, mode):
    """The report line of one GEMV check (the reference's grammar, src/komp/verify.py:145-149); an output past its
    f32 error bound adds ` outputs=PAST-BOUND`."""
    exact = lambda v: "exact" if v else "MISMATCH"  # noqa: E731
    head = "ok  " if r["ok"] else "FAIL"
    out = (f"{head} {r['fmt']:5} gemv {MODE_NAMES[mode]:13} block_n={block_n} nb={nb} warps={nw} n={r['n']} k={r['k']} "
           f"m={r['m']} quant={exact(r['quant'])} idots={exact(r['idots'])} "
           f"reference_dot={'bit-identical' if r['rebuilt'] else 'DIFFERS'} relerr={r['relerr']:.1e}")  # fmt: skip
    return out if r.get("bound", True) else out + " outputs=PAST-BOUND"


def _gemv_jobs(formats_, modes):
    """Every (fmt, mode, knobs, problem, data kind) of the GEMV checks, in report order."""
    for fmt, mode in itertools.product(formats_, modes):
        yield from ((fmt, mode, cfg, prob, kind) for cfg, prob, kind in
                    itertools.product(CONFIGS[fmt], PROBLEMS[fmt], ((1, False), (2, True))))  # fmt: skip


def run_all(log=print, formats_=("q4_0", "tq2_0"), modes=(0, 1, 2)):
    """dp4a, decode (random and extreme) and every GEMV problem x knob set x mode x data kind: 1 + 4 + 2 x 3 x 3 x 3
    x 2 = 113 checks with the three modes.  Logs one line per check and the failure count, which it returns."""
    results = []
    ok = check_dp4a(seed=3)
    results.append(ok)
    log(f"{'ok  ' if ok else 'FAIL'} dp4a v_dot4c_i32_i8 and emulated == dp4a.s32.s32 semantics (1024 edge/random words)")
    for extreme in (False, True):
        for fmt, ok in check_decode(seed=7, extreme=extreme).items():
            results.append(ok)
            log(f"{'ok  ' if ok else 'FAIL'} decode {fmt:5} {'extreme' if extreme else 'random '} (values == KURN reference)")
    for fmt, mode, (block_n, nb, nw), (n, k, m), (seed, extreme) in _gemv_jobs(formats_, modes):
        r = check_gemv(fmt, n, k, m, seed, extreme, block_n, nb, mode, nw)
        results.append(r["ok"])
        log(line(r, block_n, nb, nw, mode) + (" extreme" if extreme else ""))
    fails = results.count(False)
    log(f"{fails} failures")
    return fails
