"""The single-column TQ2_0 dp4a kernel (gemv_tq2.hip) vs the oracle, over every lanes-per-row / chunks-per-lane
instantiation it is built for: S exact, Y within 1e-5 of the f64 reference_dot, Y independent of whether S is stored,
and the fused launch bit-identical to quantizer + GEMV.  Shapes leave a partial last workgroup, a partial last K step
and (with 128 rows over 4 waves) two passes per wave; padded weight rows and a multi-matrix launch too.  Everything
goes through the C ABI."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5
# knob sets (block_n, num_warps) -> lanes per row 64, 32, 16, 8, 4 and 4 with two passes per wave
LAYOUTS = [(8, 8), (16, 8), (32, 8), (64, 8), (128, 8), (128, 4)]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("nb", [1, 2, 4, 8])
@pytest.mark.parametrize("extreme", [False, True])
def test_every_instantiation_matches_oracle(layout, nb, extreme):
    bn, nw = layout
    n, k = 300, 2816  # 11 blocks: a partial last K step for every lanes-per-row / nb pair
    W, x = O.problem("tq2_0", n, k, 1, 70 + nb + bn, extreme)
    wq, ws = host.split("tq2_0", W, n, k)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    print(f"tq2_0 n={n} k={k} block_n={bn} nb={nb} num_warps={nw} extreme={extreme}", flush=True)
    y_s, s = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k, bn, nb, 2, nw, store_s=True)
    y = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k, bn, nb, 2, nw)[0]
    xq, xd, *_ = host.quantize("tq2_0", x_d)
    y2, s2 = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize("tq2_0", x)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs) and torch.equal(s, s2)
    assert torch.equal(y.view(torch.int32), y_s.view(torch.int32))
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    assert O.relerr(y.cpu().numpy(), r) <= TOL


@pytest.mark.parametrize("n,k", [(6912, 2560), (2560, 6912), (5, 256), (16400, 8192), (257, 512)])
def test_auto_plans_padded_rows(n, k):
    W, x = O.problem("tq2_0", n, k, 1, 90)
    wq, ws = host.split("tq2_0", W, n, k)
    wq_pad = dev(np.pad(wq, ((0, 0), (0, 64))))[:, : wq.shape[1]]  # a row stride 64 bytes past the row
    y, s = host.gemv_f32("tq2_0", wq_pad, dev(ws), dev(x), n, k, store_s=True)
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize("tq2_0", x)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert O.relerr(y.cpu().numpy(), r) <= TOL


def test_multi_matrix_launch():
    k = 2560
    ns = (6912, 300, 6912)
    rng = np.random.default_rng(91)
    x = O.activations(rng, k, 1, block=256)
    rq, rd, _ = O.quantize("tq2_0", x)
    mats, refs = [], []
    for n in ns:
        wq, ws = host.split("tq2_0", O.weights("tq2_0", rng, n, k), n, k)
        mats.append((dev(wq), dev(ws), n))
        refs.append(O.gemv("tq2_0", wq, ws, rq, rd, n, k)[0])
    ys = host.gemv_multi("tq2_0", mats, k, x=dev(x))
    torch.cuda.synchronize()
    for y, r in zip(ys, refs):
        assert O.relerr(y.cpu().numpy(), r) <= TOL
