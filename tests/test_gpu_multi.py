"""Several weight matrices sharing one input in one launch (komp_*_gemv_multi): with the same knobs every output equals
the single-matrix launch bit for bit; with the library's plan every output is within the f32 error bound of the f64
reference."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def problems(fmt, ns, k, m, seed):
    """Per matrix: (W bytes, split planes on the device); one shared activation x [m][k]."""
    rng = np.random.default_rng(seed)
    x = O.activations(rng, k, m, block=O.ACT_BLOCK[O.FORMATS[fmt]["act"]], extreme=False, outliers=0.01)
    mats = []
    for i, n in enumerate(ns):
        W = O.weights(fmt, np.random.default_rng(seed + 1 + i), n, k, False)
        wq, ws = host.split(fmt, W, n, k)
        mats.append((wq, ws, n))
    return mats, x


CASES = [("q4_0", (4096, 1024, 1024), 4096), ("tq2_0", (6912, 6912), 2560), ("q4_0", (37, 5, 100, 64), 416),
         ("tq2_0", (13, 300, 1), 1280), ("q4_0", (64, 0, 33), 512), ("q8_0", (4096, 1024, 1024), 4096),
         ("iq4_nl", (37, 5, 100, 64), 416), ("q8_0", (13, 300, 1), 1280), ("q4_k", (37, 5, 100, 64), 768),
         ("q4_k", (6912, 6912), 2560)]  # fmt: skip


@pytest.mark.parametrize("fmt,ns,k", CASES)
@pytest.mark.parametrize("m", [1, 3])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("knobs", [None, (32, 4, 4), (16, 2, 2)])
def test_multi_matches_single_launches(fmt, ns, k, m, fused, knobs):
    mats, x = problems(fmt, ns, k, m, 7 + m)
    dmats = [(dev(wq), dev(ws), n) for wq, ws, n in mats]
    xg = dev(x)
    bn, nb, nw = knobs if knobs else (None, 0, 0)
    if fused:
        ys = host.gemv_multi(fmt, dmats, k, x=xg, block_n=bn, nb=nb, num_warps=nw)
        singles = [host.gemv_f32(fmt, wq, ws, xg, n, k, bn, nb, 2, nw)[0] for wq, ws, n in dmats]
    else:
        xq, xd = host.quantize(fmt, xg)
        ys = host.gemv_multi(fmt, dmats, k, xq=xq, xd=xd, block_n=bn, nb=nb, num_warps=nw)
        singles = [host.gemv(fmt, wq, ws, xq, xd, n, k, bn, nb, 2, nw)[0] for wq, ws, n in dmats]
    torch.cuda.synchronize()
    rq, rd, *_ = O.quantize(fmt, x)
    for (wq, ws, n), y, y1 in zip(mats, ys, singles):
        assert tuple(y.shape) == (m, n)
        if knobs is not None:
            assert torch.equal(y.view(torch.int32), y1.view(torch.int32))
        if n:
            r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
            assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)


def test_multi_four_columns_and_graph_capture():
    # M = 4 runs as two launches of 3 and 1 columns; the multi launch also replays from a captured graph
    fmt, ns, k = "tq2_0", (2560, 512), 6912
    mats, x = problems(fmt, ns, k, 4, 3)
    dmats = [(dev(wq), dev(ws), n) for wq, ws, n in mats]
    xg = dev(x)
    ys = [torch.empty((4, n), dtype=torch.float32, device="cuda") for _, _, n in dmats]
    host.gemv_multi_into(fmt, dmats, ys, k, x=xg)
    torch.cuda.synchronize()
    eager = [y.clone() for y in ys]
    rq, rd, *_ = O.quantize(fmt, x)
    for (wq, ws, n), y in zip(mats, eager):
        r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
        assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        host.gemv_multi_into(fmt, dmats, ys, k, x=xg)
    for _ in range(3):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y, e in zip(ys, eager):
            assert torch.equal(y, e)
