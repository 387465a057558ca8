"""The lean kernels (gemv_tq2.h: 1-3 TQ2_0 columns in dp4a and bytes modes; gemv_q4.h: 1-3 Q4_0 / IQ4_NL columns in
dp4a mode, Q4_0 in bytes mode too) vs the oracle, over every lanes-per-row / chunks-per-lane / column-count
instantiation they are built for: S exact, every output of Y within the f32 error bound of the f64 reference_dot, Y
independent of whether S is stored, and the fused launch bit-identical to quantizer + GEMV.  The Q4_0 / IQ4_NL
kernels keep the general kernel's accumulation order (whole block dots scaled in f32, lane sums in the same tree), so
their Y is also bit-identical to the emulated-dp4a mode (which runs the general kernel); the TQ2_0 kernel scales each
block in the lane that owns its chunk slot, another order of the same terms, so there both Y are checked against the
bound and S against each other.  Bytes mode (every crumb or nibble and activation unpacked to a 16-bit integer first)
gives the dp4a form's S and Y bit for bit.  Shapes leave a partial last workgroup, a partial last K step and (with 128
rows over 4 waves) two passes per wave; padded weight rows and multi-matrix launches too.  Everything goes through the
C ABI."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

# knob sets (block_n, num_warps) -> lanes per row 64, 32, 16, 8, 4 and 4 with two passes per wave
LAYOUTS = [(8, 8), (16, 8), (32, 8), (64, 8), (128, 8), (128, 4)]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


FORMATS = ["tq2_0", "q4_0", "iq4_nl"]
BYTES_LEAN = ("tq2_0", "q4_0")  # the formats whose lean kernel has a bytes form
K_TAIL = {"tq2_0": 2816, "q4_0": 2400, "iq4_nl": 2400}  # 11 / 75 blocks: a partial last K step for every layout, nb


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("nb", [1, 2, 4, 8])
@pytest.mark.parametrize("extreme", [False, True])
@pytest.mark.parametrize("m", [1, 2, 3])
def test_every_instantiation_matches_oracle(fmt, layout, nb, extreme, m):
    bn, nw = layout
    n, k = 300, K_TAIL[fmt]
    W, x = O.problem(fmt, n, k, m, 70 + nb + bn + 7 * m, extreme)
    wq, ws = host.split(fmt, W, n, k)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    print(f"{fmt} n={n} k={k} m={m} block_n={bn} nb={nb} num_warps={nw} extreme={extreme}", flush=True)
    y_s, s = host.gemv_f32(fmt, wq_d, ws_d, x_d, n, k, bn, nb, 2, nw, store_s=True)
    y = host.gemv_f32(fmt, wq_d, ws_d, x_d, n, k, bn, nb, 2, nw)[0]
    xq, xd, *_ = host.quantize(fmt, x_d)
    y2, s2 = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
    y_emu, s_emu = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, bn, nb, 1, nw, store_s=True)  # the general kernel
    if fmt in BYTES_LEAN:  # bytes mode: the lean kernel's bytes form, the same block dots in the same order
        y_b, s_b = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, bn, nb, 0, nw, store_s=True)
        y_bf = host.gemv_f32(fmt, wq_d, ws_d, x_d, n, k, bn, nb, 0, nw)[0]
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs) and torch.equal(s, s2) and torch.equal(s, s_emu)
    assert torch.equal(y.view(torch.int32), y_s.view(torch.int32))
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))
    if fmt == "tq2_0":
        assert outputs_ok(fmt, y_emu.cpu().numpy(), ws, rd, rs, r)
    else:
        assert torch.equal(y.view(torch.int32), y_emu.view(torch.int32))
    if fmt in BYTES_LEAN:
        assert torch.equal(s_b, s) and torch.equal(y_b.view(torch.int32), y2.view(torch.int32))
        assert torch.equal(y_bf.view(torch.int32), y.view(torch.int32))
    assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)


SHAPES = {"tq2_0": [(6912, 2560), (2560, 6912), (5, 256), (16400, 8192), (257, 512)],
          "q4_0": [(4096, 4096), (14336, 4096), (4096, 14336), (5, 32), (16400, 4192)]}
SHAPES["iq4_nl"] = SHAPES["q4_0"]


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("shape", range(5))
@pytest.mark.parametrize("fused", [False, True])
def test_auto_plans_padded_rows(fmt, shape, fused):
    n, k = SHAPES[fmt][shape]
    W, x = O.problem(fmt, n, k, 1, 90 + shape)
    wq, ws = host.split(fmt, W, n, k)
    wq_pad = dev(np.pad(wq, ((0, 0), (0, 64))))[:, : wq.shape[1]]  # a row stride 64 bytes past the row
    ys = []
    for mode in (2, 0) if fmt in BYTES_LEAN else (2,):  # dp4a and bytes, bit-identical
        if fused:
            y, s = host.gemv_f32(fmt, wq_pad, dev(ws), dev(x), n, k, mode=mode, store_s=True)
        else:
            xq, xd, *_ = host.quantize(fmt, dev(x))
            y, s = host.gemv(fmt, wq_pad, dev(ws), xq, xd, n, k, block_n=None, mode=mode, store_s=True)
        ys.append((y, s))
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    y, s = ys[0]
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
    for y2, s2 in ys[1:]:
        assert torch.equal(s2, s) and torch.equal(y2.view(torch.int32), y.view(torch.int32))


@pytest.mark.parametrize("fmt", FORMATS)
def test_multi_matrix_launch(fmt):
    k = 2560
    ns = (6912, 300, 6912)
    rng = np.random.default_rng(91)
    x = O.activations(rng, k, 1, block=O.ACT_BLOCK[O.FORMATS[fmt]["act"]])
    rq, rd, _ = O.quantize(fmt, x)
    mats, refs = [], []
    for n in ns:
        wq, ws = host.split(fmt, O.weights(fmt, rng, n, k), n, k)
        mats.append((dev(wq), dev(ws), n))
        refs.append((ws, *O.gemv(fmt, wq, ws, rq, rd, n, k)))
    ys = host.gemv_multi(fmt, mats, k, x=dev(x))
    torch.cuda.synchronize()
    for y, (ws, r, rs) in zip(ys, refs):
        assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
