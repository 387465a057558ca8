"""Weight ingestion on the device (komp_{q4_0,tq2_0,q8_0,iq4_nl,q4_k}_split) vs the oracle's split of the same ggml block
bytes: WQ and WS bit-identical, row padding left untouched, and a GEMV over the device-split planes equal to one over
the host-split planes.  Everything goes through the C ABI."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

# block values, block bytes, quant bytes
NBYTES = {"q4_0": (32, 18, 16), "tq2_0": (256, 66, 64), "q8_0": (32, 34, 32), "iq4_nl": (32, 18, 16),
          "q4_k": (256, 144, 128)}
SHAPES = [(1, 1), (5, 3), (37, 13), (64, 128), (300, 27), (1023, 7)]  # (rows, blocks per row)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
@pytest.mark.parametrize("shape", range(len(SHAPES)))
def test_split_matches_oracle(fmt, shape):
    n, nb = SHAPES[shape]
    blk, nbytes, qbytes = NBYTES[fmt]
    k = nb * blk
    rng = np.random.default_rng(700 + shape)
    W = rng.integers(0, 256, n * nb * nbytes, dtype=np.uint8)  # any bytes: the split moves them
    rq, rs = O.split(fmt, W.tobytes(), n, k)
    print(f"split {fmt} n={n} k={k}", flush=True)
    wq, ws = host.split_device(fmt, dev(W), n, k)
    torch.cuda.synchronize()
    assert np.array_equal(wq.cpu().numpy(), rq) and np.array_equal(ws.cpu().numpy(), rs)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_split_padded_rows_and_offset_input(fmt):
    n, nb = 29, 11
    blk, nbytes, qbytes = NBYTES[fmt]
    k = nb * blk
    rng = np.random.default_rng(77)
    W = rng.integers(0, 256, n * nb * nbytes, dtype=np.uint8)
    rq, rs = O.split(fmt, W.tobytes(), n, k)
    base = torch.zeros(W.size + 8, dtype=torch.uint8, device="cuda")  # the input starts 4 bytes into its allocation
    base[4 : 4 + W.size] = dev(W)
    w_in = base[4 : 4 + W.size]
    sw = (nb * qbytes + 15) // 16 * 16 + 48
    wq = torch.full((n, sw), 0xA5, dtype=torch.uint8, device="cuda")
    ws = torch.zeros((n, nb * O.FORMATS[fmt]["sbytes"] // 2), dtype=torch.int16, device="cuda")
    host.split_into(fmt, w_in, wq, ws, n, k)
    torch.cuda.synchronize()
    got = wq.cpu().numpy()
    assert np.array_equal(got[:, : nb * qbytes], rq) and np.array_equal(ws.cpu().numpy(), rs)
    assert (got[:, nb * qbytes :] == 0xA5).all()  # padding untouched


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemv_over_device_split(fmt):
    n, k, m = (96, 1024, 3) if fmt != "tq2_0" else (96, 1536, 3)
    W, x = O.problem(fmt, n, k, m, 81)
    wq_h, ws_h = host.split(fmt, W, n, k)
    wq_d, ws_d = host.split_device(fmt, dev(np.frombuffer(W, dtype=np.uint8)), n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    y1, s1 = host.gemv(fmt, dev(wq_h), dev(ws_h), xq, xd, n, k, 32, 2, 2, 4, store_s=True)
    y2, s2 = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, 32, 2, 2, 4, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq_h, ws_h, rq, rd, n, k)
    assert np.array_equal(s2.cpu().numpy().astype(np.int64), rs) and outputs_ok(fmt, y2.cpu().numpy(), ws_h, rd, rs, r)
