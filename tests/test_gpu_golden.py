"""The HIP kernels against the committed golden vectors, through the C ABI."""

import numpy as np
import pytest
import torch

from comp_amd import host
from tests.checks import outputs_ok
from tests.golden import fixtures as G

pytestmark = pytest.mark.gpu
V = G.load()


def test_quantizers_golden():
    x = np.stack([G.f32(b) for b in V["q8_0"]["x_bits"]]).reshape(1, -1)
    xq, xd = host.quantize("q4_0", torch.from_numpy(x).cuda())
    assert np.array_equal(xq.cpu().numpy().reshape(-1, 32).astype(int), np.asarray(V["q8_0"]["q"]))
    assert np.array_equal(xd.cpu().numpy().reshape(-1).view(np.uint32), np.asarray(V["q8_0"]["d_bits"], np.uint32))
    x = np.stack([G.f32(b) for b in V["q8_K"]["x_bits"]]).reshape(1, -1)
    xq, xd, xb = host.quantize("tq2_0", torch.from_numpy(x).cuda(), bsums=True)
    assert np.array_equal(xq.cpu().numpy().reshape(-1, 256).astype(int), np.asarray(V["q8_K"]["q"]))
    assert np.array_equal(xd.cpu().numpy().reshape(-1).view(np.uint32), np.asarray(V["q8_K"]["d_bits"], np.uint32))
    assert np.array_equal(xb.cpu().numpy().reshape(-1, 16).astype(int), np.asarray(V["q8_K"]["bsums"]))


def test_dp4a_golden():
    t = np.asarray(V["dp4a"], np.int64)
    a, b, c = (torch.from_numpy(t[:, i].astype(np.int32)).cuda() for i in range(3))
    for mode in (1, 2):
        assert np.array_equal(host.dp4a_probe(a, b, c, mode).cpu().numpy().astype(np.int64), t[:, 3])


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("knobs", [(8, 1, 1), (32, 4, 4), (128, 16, 8), None])
def test_gemv_golden(mode, knobs):
    for c in V["gemv"]:
        fmt, n, k, m, W, xq, xd, S, Y = G.gemv_case(c)
        wq, ws = host.split(fmt, W, n, k)
        bn, nb, nw = knobs if knobs else (None, 0, 0)
        y, s = host.gemv(fmt, torch.from_numpy(wq).cuda(), torch.from_numpy(ws).cuda(), torch.from_numpy(xq).cuda(),
                         torch.from_numpy(xd).cuda(), n, k, bn, nb, mode, nw, store_s=True)  # fmt: skip
        assert np.array_equal(s.cpu().numpy().astype(np.int64), S)
        assert outputs_ok(fmt, y.cpu().numpy(), ws, xd, S, Y)
