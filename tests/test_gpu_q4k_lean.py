"""Q4_K lean GEMV kernels (gemv_q4k.h, dp4a mode) through the C ABI: S exact and Y within the output gate against the
oracle, and S and Y bit for bit the general kernel's for the same knobs (its bytes mode, which the lean kernels do not
take, computes the same exact block dots and the same f32 operations in the same order).  The plans cover the
single-pass, single-step form and the loop form (several K steps, two passes), 1-3 columns, fused and unfused, row
tails and slots past a row's end."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

# (n, k, m, block_n, nb, num_warps): lanes per row = 64 / min(block_n / num_warps, 16)
CASES = [
    (4096, 4096, 1, 16, 4, 4),   # 16 lanes a row, nb 4: the 16 blocks in one K step
    (300, 4096, 3, 16, 4, 4),    # three columns, a partial last workgroup
    (77, 14336, 2, 8, 4, 8),     # 64 lanes, nb 4: 56 blocks in one step of 64 (8 slots past the row's end)
    (77, 14336, 1, 32, 2, 4),    # 8 lanes, nb 2: 4 blocks a step, 14 steps
    (129, 2560, 3, 64, 1, 2),    # 32 rows a wave: 4 lanes, two passes, 10 steps of one block
    (45, 2304, 2, 128, 4, 8),    # 16 rows a wave: 4 lanes, nb 4, 3 steps (the last one partial)
]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("fused", [False, True])
def test_q4k_lean_matches_oracle_and_general_kernel(case, fused):
    n, k, m, bn, nb, nw = CASES[case]
    print(f"q4k lean n={n} k={k} m={m} knobs={bn},{nb},{nw} fused={fused}", flush=True)
    W, x = O.problem("q4_k", n, k, m, 70 + case)
    wq, ws = host.split("q4_k", W, n, k)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    if fused:
        y2, s2 = host.gemv_f32("q4_k", wq_d, ws_d, x_d, n, k, bn, nb, 2, nw, store_s=True)
        y0, s0 = host.gemv_f32("q4_k", wq_d, ws_d, x_d, n, k, bn, nb, 0, nw, store_s=True)
    else:
        xq, xd, *_ = host.quantize("q4_k", x_d)
        y2, s2 = host.gemv("q4_k", wq_d, ws_d, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
        y0, s0 = host.gemv("q4_k", wq_d, ws_d, xq, xd, n, k, bn, nb, 0, nw, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s2, s0)
    assert torch.equal(y2.view(torch.int32), y0.view(torch.int32))
    rq, rd, _ = O.quantize("q4_k", x)
    r, rs = O.gemv("q4_k", wq, ws, rq, rd, n, k)
    assert np.array_equal(s2.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("q4_k", y2.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("extreme", [False, True])
def test_q4k_lean_fused_writes_the_quantizer_planes(extreme):
    # return_q: one workgroup writes the q8_K planes and bsums it staged, byte for byte the quantizer's
    n, k, m = 300, 4352, 2
    W, x = O.problem("q4_k", n, k, m, 81, extreme)
    wq, ws = host.split("q4_k", W, n, k)
    y, s, (xq, xd, xb) = host.gemv_f32("q4_k", dev(wq), dev(ws), dev(x), n, k, store_s=True, return_q=True)
    torch.cuda.synchronize()
    rq, rd, rb = O.quantize("q4_k", x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(xb.cpu().numpy(), rb)
    r, rs = O.gemv("q4_k", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("q4_k", y.cpu().numpy(), ws, rd, rs, r)
