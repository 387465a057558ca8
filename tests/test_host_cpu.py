"""Host-side logic that runs without a GPU: split layouts, ggml block packing, and loud failure for CPU tensors
(there is no CPU path behind the operator API)."""

import numpy as np
import pytest
import torch

from comp_amd import _abi, host
from oracle import oracle as O


@pytest.mark.parametrize("fmt,k", [("q4_0", 160), ("tq2_0", 768)])
def test_split_matches_oracle_and_joins_back(fmt, k):
    W = O.weights(fmt, np.random.default_rng(1), 7, k, extreme=True)
    wq, ws = host.split(fmt, W, 7, k)
    owq, ows = O.split(fmt, W, 7, k)
    assert np.array_equal(wq, owq) and np.array_equal(ws, ows) and wq.dtype == np.uint8 and ws.dtype == np.int16
    assert O.join(fmt, wq, ws) == W


def test_tq2_0_qplane_and_split_q4_0():
    W = O.weights("tq2_0", np.random.default_rng(2), 1, 1280)
    assert np.array_equal(host.tq2_0_qplane(W, 5), O.split("tq2_0", W, 1, 1280)[0].reshape(5, 64))
    W = O.weights("q4_0", np.random.default_rng(3), 3, 96)
    assert all(np.array_equal(a, b) for a, b in zip(host.split_q4_0(W, 3, 96), O.split("q4_0", W, 3, 96)))


def test_act_blocks_match_oracle():
    x = O.activations(np.random.default_rng(4), 512, 2, block=256, extreme=True)
    xq, xd, xb = O.quant_q8_K(x)
    assert host.act_blocks("tq2_0", xq, xd) == O.act_blocks("tq2_0", xq, xd, xb)
    assert host.act_blocks("tq2_0", torch.from_numpy(xq), torch.from_numpy(xd), torch.from_numpy(xb)) == \
        O.act_blocks("tq2_0", xq, xd, xb)
    xq, xd = O.quant_q8_0(x)
    assert host.act_blocks("q4_0", xq, xd) == O.act_blocks("q4_0", xq, xd)


def test_formats_and_modes_match_reference():
    assert host.FORMATS == O.FORMATS
    assert host.MODES == {"bytes": 0, "dp4a": 2}


def test_cpu_tensors_fail_loudly():
    x = torch.zeros((1, 64))
    with pytest.raises(_abi.KompArgumentError, match="HIP device"):
        host.quantize("q4_0", x)
    wq = torch.zeros((4, 32), dtype=torch.uint8)
    ws = torch.zeros((4, 2), dtype=torch.int16)
    xq = torch.zeros((1, 64), dtype=torch.int8)
    xd = torch.zeros((1, 2))
    with pytest.raises(_abi.KompArgumentError, match="HIP device"):
        host.gemv("q4_0", wq, ws, xq, xd, 4, 64)
    with pytest.raises(_abi.KompArgumentError, match="HIP device"):
        host.gemv("iq4_nl", wq, ws, xq, xd, 4, 64)
    with pytest.raises(KeyError):
        host.gemv("q5_k", wq, ws, xq, xd, 4, 64)
    with pytest.raises(_abi.KompArgumentError, match="HIP device"):
        host.gemv_multi("q4_0", [(wq, ws, 4), (wq, ws, 4)], 64, xq=xq, xd=xd)
    with pytest.raises(_abi.KompArgumentError, match="either"):
        host.gemv_multi("q4_0", [(wq, ws, 4)], 64, xq=xq, xd=xd, x=x)
    with pytest.raises(_abi.KompArgumentError, match="1..4"):
        host.gemv_multi("q4_0", [(wq, ws, 4)] * 5, 64, xq=xq, xd=xd)
