"""The fused quantize-and-GEMV launch equals quantize() followed by gemv() with the same knobs bit for bit (Y, S and
the q8 planes), for every mode, edge data, tails and 1..4 columns; block_n=None plans the fused launch with
auto_config(..., fused=True)."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


CASES = [("q4_0", 37, 416, 3), ("q4_0", 4097, 4192, 1), ("q4_0", 64, 512, 4), ("tq2_0", 37, 768, 3),
         ("tq2_0", 6913, 2816, 2), ("tq2_0", 5, 1280, 1), ("q8_0", 37, 416, 3), ("q8_0", 4097, 4192, 1),
         ("iq4_nl", 37, 416, 3), ("iq4_nl", 4097, 4192, 1), ("iq4_nl", 64, 512, 4), ("q4_k", 37, 768, 3),
         ("q4_k", 4097, 4352, 1), ("q4_k", 64, 1024, 4),
         ("tq2_0", 2048, 2816, 3), ("tq2_0", 1000, 4096, 3),  # 3 columns over few rows: 9 and 12 waves of one row
         ("q4_0", 300, 4096, 1), ("q8_0", 127, 4096, 1), ("iq4_nl", 127, 4096, 1), ("q4_k", 127, 4096, 1)]  # fmt: skip
# (the last four: one f32 column over few rows a CU, staged in one pass by 16 or 4 waves)


@pytest.mark.parametrize("fmt,n,k,m", CASES)
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("extreme", [False, True])
@pytest.mark.parametrize("knobs", [(32, 4, 4), None])
def test_fused_equals_two_launches(fmt, n, k, m, mode, extreme, knobs):
    W, x = O.problem(fmt, n, k, m, 40 + extreme, extreme)
    wq, ws = host.split(fmt, W, n, k)
    wq, ws, xg = dev(wq), dev(ws), dev(x)
    bn, nb, nw = knobs if knobs else (None, 0, 0)
    y1, s1, q = host.gemv_f32(fmt, wq, ws, xg, n, k, bn, nb, mode, nw, store_s=True, return_q=True)
    qq = host.quantize(fmt, xg, bsums=(O.FORMATS[fmt]["act"] == "q8_K"))
    y2, s2 = host.gemv(fmt, wq, ws, qq[0], qq[1], n, k, bn, nb, mode, nw, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2)
    # with block_n=None each launch plans for itself: Y is bit-identical when both planned alike (the f32 sums then
    # run in the same order), and within the oracle tolerance below otherwise
    # (from host.GEMM_MIN_M columns on, the unfused dp4a launch with block_n=None runs the matrix-core GEMM instead,
    # and three TQ2_0 columns the matrix-core GEMV)
    if knobs or (host.auto_plan(fmt, m, n, k, True, mode) == host.auto_plan(fmt, m, n, k, False, mode)
                 and not host.uses_gemm(fmt, m, n, k, False, mode) and not host.uses_mfma(fmt, m, n, k, False, mode)):
        assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    for a, b in zip(q, qq):
        assert torch.equal(a.view(torch.uint8) if a.dtype != torch.int16 else a, b.view(torch.uint8) if b.dtype != torch.int16 else b)
    rq, rd, rb = O.quantize(fmt, x)
    assert np.array_equal(q[0].cpu().numpy(), rq)
    wq_h, ws_h = host.split(fmt, W, n, k)
    r, rs = O.gemv(fmt, wq_h, ws_h, rq, rd, n, k)
    assert np.array_equal(s1.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok(fmt, y1.cpu().numpy(), ws_h, rd, rs, r) and outputs_ok(fmt, y2.cpu().numpy(), ws_h, rd, rs, r)


def test_fused_without_q_outputs():
    fmt, n, k, m = "tq2_0", 2560, 6912, 1
    W, x = O.problem(fmt, n, k, m, 7)
    wq, ws = host.split(fmt, W, n, k)
    y, s = host.gemv_f32(fmt, dev(wq), dev(ws), dev(x), n, k)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert s is None and outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
