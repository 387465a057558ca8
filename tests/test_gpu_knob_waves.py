"""Knob launches whose programs run one workgroup a wave (unfused single Q4_0 / IQ4_NL columns on the lean kernel,
programs x waves <= the device's CUs): Y and S bit for bit those of the same knobs over a matrix tall enough to keep
every program one workgroup (the same first rows), S exact and Y within the gate against the oracle."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("fmt,mode,knobs", [("q4_0", 2, (64, 4, 4)), ("q4_0", 0, (64, 4, 4)), ("q4_0", 2, (128, 4, 8)),
                                            ("q4_0", 2, (64, 2, 2)), ("iq4_nl", 2, (64, 8, 4))])  # fmt: skip
@pytest.mark.parametrize("extreme", [False, True])
def test_waves_apart_equal_whole_programs(fmt, mode, knobs, extreme):
    n, tall, k = 4096, 16384, 4096
    bn, nb, nw = knobs
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert (n // bn) * nw <= cus < (tall // bn) * nw  # one workgroup a wave here, whole programs over the tall matrix
    print(f"knob waves apart {fmt} mode={mode} knobs={knobs} extreme={extreme}", flush=True)
    W, x = O.problem(fmt, tall, k, 1, 60 + bn + nb + nw + extreme, extreme)
    wq_t, ws_t = host.split(fmt, W, tall, k)
    row_bytes = k // host.FORMATS[fmt]["block"] * host.FORMATS[fmt]["nbytes"]  # W holds the rows' blocks packed
    wq, ws = host.split(fmt, W[: n * row_bytes], n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    y, s = host.gemv(fmt, dev(wq), dev(ws), xq, xd, n, k, bn, nb, mode, nw, store_s=True)
    y_t, s_t = host.gemv(fmt, dev(wq_t), dev(ws_t), xq, xd, tall, k, bn, nb, mode, nw, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), y_t[:, :n].contiguous().view(torch.int32))
    assert torch.equal(s, s_t[:, :n])
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
