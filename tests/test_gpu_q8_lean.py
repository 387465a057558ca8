"""Q8_0 lean GEMV kernels (gemv_q8.h, dp4a mode) through the C ABI: S exact and Y within the output gate against the
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
    (4096, 4096, 1, 8, 4, 8),    # 64 lanes a row, nb 4: the 128 blocks in one K step
    (300, 4096, 3, 16, 4, 4),    # three columns, 16 lanes: 32 blocks a step, 4 steps; a partial last workgroup
    (77, 14336, 1, 8, 8, 8),     # nb 8: 256 blocks a step, 2 steps (64 slots past the row's end in the second)
    (129, 2560, 2, 64, 2, 2),    # 32 rows a wave: 4 lanes, two passes, 4 blocks a step
    (45, 2304, 3, 128, 4, 8),    # 16 rows a wave: 4 lanes, nb 4, 9 steps
    (5, 96, 2, 32, 1, 4),        # 3 blocks in one partial step
]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("fused", [False, True])
def test_q8_lean_matches_oracle_and_general_kernel(case, fused):
    n, k, m, bn, nb, nw = CASES[case]
    print(f"q8 lean n={n} k={k} m={m} knobs={bn},{nb},{nw} fused={fused}", flush=True)
    W, x = O.problem("q8_0", n, k, m, 70 + case)
    wq, ws = host.split("q8_0", W, n, k)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    if fused:
        y2, s2 = host.gemv_f32("q8_0", wq_d, ws_d, x_d, n, k, bn, nb, 2, nw, store_s=True)
        y0, s0 = host.gemv_f32("q8_0", wq_d, ws_d, x_d, n, k, bn, nb, 0, nw, store_s=True)
    else:
        xq, xd, *_ = host.quantize("q8_0", x_d)
        y2, s2 = host.gemv("q8_0", wq_d, ws_d, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
        y0, s0 = host.gemv("q8_0", wq_d, ws_d, xq, xd, n, k, bn, nb, 0, nw, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s2, s0)
    assert torch.equal(y2.view(torch.int32), y0.view(torch.int32))
    rq, rd, _ = O.quantize("q8_0", x)
    r, rs = O.gemv("q8_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s2.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("q8_0", y2.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("extreme", [False, True])
def test_q8_lean_fused_writes_the_quantizer_planes(extreme):
    # return_q: one workgroup writes the q8_0 planes it staged, byte for byte the quantizer's
    n, k, m = 300, 4192, 2
    W, x = O.problem("q8_0", n, k, m, 81, extreme)
    wq, ws = host.split("q8_0", W, n, k)
    y, s, (xq, xd) = host.gemv_f32("q8_0", dev(wq), dev(ws), dev(x), n, k, store_s=True, return_q=True)
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize("q8_0", x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    r, rs = O.gemv("q8_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("q8_0", y.cpu().numpy(), ws, rd, rs, r)
