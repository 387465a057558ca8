"""The TQ2_0 matrix-core GEMV (gemv_tq2_mfma.hip: three columns, q8_K or f32 in, dp4a mode, block_n=None) through the C ABI: S exact and Y within the output gate against the oracle, S bit for bit the lean dp4a
kernel's (explicit knobs), at the BitNet-2B shapes, ragged row counts (full and partial last workgroups of 9-16 rows),
rows of 1-56 blocks (one wave a workgroup up to
16 waves of 1-4 blocks), one and two row tiles a workgroup, and the extreme data (crumb 3 against +-127
activations)."""

import numpy as np
import pytest
import torch

from comp_amd import _abi, host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

CASES = [  # workgroups as planned on the 256 CUs of an MI355X
    (6912, 2560, 3),   # BitNet-2B W1: 432 workgroups of 16 rows and 10 waves, one block a wave
    (2560, 6912, 3),   # BitNet-2B W2: 256 workgroups of 10 rows; 14 waves of 2 blocks, the last one 1
    (2600, 2560, 3),   # 237 workgroups of 11 rows, the last of 4
    (2100, 14336, 3),  # 56 blocks: 16 waves of 3-4 blocks; 234 workgroups of 9 rows, the last of 3
    (2053, 256, 3),    # one block: one wave, no partial sums to add; the last workgroup of 1 row
    (2090, 512, 3),    # two blocks, two waves; the last workgroup of 2 rows
    (3000, 4096, 3),   # 16 blocks, 16 waves; 250 workgroups of 12 rows
    (16389, 512, 3),   # 1025 row tiles: two tiles a workgroup (the last one past the matrix), one wave of 2 blocks
    (16400, 2304, 3),  # two tiles a workgroup, 5 waves of 1-2 blocks
    (16390, 4096, 3),  # two tiles a workgroup, 8 waves of 2 blocks
]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("extreme", [False, True])
def test_mfma_gemv_matches_oracle_and_lean_kernel(case, extreme):
    n, k, m = CASES[case]
    print(f"tq2 mfma n={n} k={k} m={m} extreme={extreme}", flush=True)
    assert host.uses_mfma("tq2_0", m, n, k)
    W, x = O.problem("tq2_0", n, k, m, 90 + case, extreme)
    wq, ws = host.split("tq2_0", W, n, k)
    wq_d, ws_d = dev(wq), dev(ws)
    xq, xd = host.quantize("tq2_0", dev(x))
    y, s = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, 0, 2, 0, store_s=True)
    y_plain, _ = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, 0, 2, 0)
    y_lean, s_lean = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, 64, 1, 2, 4, store_s=True)
    # fused (f32 in; from 4 row tiles a CU on): the same plan, each wave quantizing its own blocks; S and Y bit for bit
    # the unfused launch's
    fused = host.uses_mfma("tq2_0", m, n, k, fused=True)
    assert fused == (n >= 16384)
    y_f, s_f = host.gemv_f32("tq2_0", wq_d, ws_d, dev(x), n, k, None, 0, 2, 0, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s, s_lean) and torch.equal(s_f, s)
    assert torch.equal(y.view(torch.int32), y_plain.view(torch.int32))  # S stores do not change Y
    if fused:
        assert torch.equal(y_f.view(torch.int32), y.view(torch.int32))
    rq, rd, _ = O.quantize("tq2_0", x)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("tq2_0", y.cpu().numpy(), ws, rd, rs, r)
    assert outputs_ok("tq2_0", y_lean.cpu().numpy(), ws, rd, rs, r)


def test_mfma_gemv_routing():
    # three dp4a columns with block_n=None, q8 in (f32 in from 4 row tiles a CU on); one and two columns, the other
    # modes and explicit knobs keep the GEMV kernels, 4+ columns the GEMM
    assert host.uses_mfma("tq2_0", 3, 6912, 2560) and host.uses_mfma("tq2_0", 3, 32768, 8192)
    assert not host.uses_mfma("tq2_0", 2, 32768, 8192) and not host.uses_mfma("tq2_0", 2, 6912, 2560)
    assert not host.uses_mfma("tq2_0", 1, 32768, 8192) and not host.uses_mfma("tq2_0", 4, 6912, 2560)
    assert host.uses_mfma("tq2_0", 3, 32768, 8192, fused=True) and not host.uses_mfma("tq2_0", 3, 6912, 2560, fused=True)
    assert not host.uses_mfma("tq2_0", 3, 6912, 2560, mode=0) and not host.uses_mfma("q4_0", 3, 4096, 4096)
    assert not host.uses_mfma("tq2_0", 3, 4096, 65536)  # rows of 256 blocks: past its 4 blocks a wave
    # up to 8 rows a CU (2048 on 256 CUs) the lean kernel is faster; past it the rows spread evenly, at most 16 a
    # workgroup
    assert not host.uses_mfma("tq2_0", 3, 2048, 2560) and not host.uses_mfma("tq2_0", 3, 127, 2816)
    assert host.mfma_plan("tq2_0", 3, 2560, 6912) == (10, 14) and host.mfma_plan("tq2_0", 3, 6912, 2560) == (16, 10)
    assert host.mfma_plan("tq2_0", 3, 32768, 8192) == (32, 8)


@pytest.mark.parametrize("pad", [16, 64])
def test_mfma_gemv_padded_row_stride(pad):
    # a weight plane with padded rows (the row stride is the tensor's): Y and S bit for bit the packed plane's, on the
    # matrix cores; a stride that is not a multiple of 16 is refused by the entry point (and by the plan query)
    n, k, m = 2560, 6912, 3
    row = k // 4
    sw = row + pad
    print(f"tq2 mfma padded rows sw={sw}", flush=True)
    W, x = O.problem("tq2_0", n, k, m, 77 + pad)
    wq, ws = host.split("tq2_0", W, n, k)
    wq_d, ws_d = dev(wq), dev(ws)
    wide = torch.full((n, sw), 0xA5, dtype=torch.uint8, device="cuda")  # pad bytes never read
    wide[:, :row] = wq_d
    xq, xd = host.quantize("tq2_0", dev(x))
    assert host.uses_mfma("tq2_0", m, n, k, sw=sw) and not host.uses_mfma("tq2_0", m, n, k, sw=row + 8)
    y, s = host.gemv("tq2_0", wide, ws_d, xq, xd, n, k, None, 0, 2, 0, store_s=True)
    y0, s0 = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, 0, 2, 0, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s, s0) and torch.equal(y.view(torch.int32), y0.view(torch.int32))
    rq, rd, _ = O.quantize("tq2_0", x)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("tq2_0", y.cpu().numpy(), ws, rd, rs, r)
    odd = torch.zeros((n, row + 8), dtype=torch.uint8, device="cuda")
    with pytest.raises(_abi.KompArgumentError, match="multiple of 16"):
        host.gemv("tq2_0", odd, ws_d, xq, xd, n, k, None, 0, 2, 0)


def test_mfma_gemv_stamped_instantiation():
    # with the tuning harness's stamps on, the launch runs the stamped instantiation: the same Y and S, and one record
    # per wave whose phases are in order
    n, k, m = 6912, 2560, 3
    W, x = O.problem("tq2_0", n, k, m, 99)
    wq, ws = host.split("tq2_0", W, n, k)
    wq_d, ws_d = dev(wq), dev(ws)
    xq, xd = host.quantize("tq2_0", dev(x))
    y0, s0 = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, 0, 2, 0, store_s=True)
    buf = torch.zeros(1 << 20, dtype=torch.int32, device="cuda")
    _abi.stamps_begin(buf)
    try:
        y1, s1 = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, 0, 2, 0, store_s=True)
    finally:
        used, khz = _abi.stamps_end()
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(s0, s1)
    rows, waves = _abi.gemv_mfma_plan(1, False, 2, m, n, k, k // 4)
    recs = _abi.parse_stamps(buf[:used].cpu().numpy().view(np.uint32), khz)
    assert len(recs) == 1 and recs[0]["n"] == n and recs[0]["k"] == k
    assert recs[0]["waves"] == (n + rows - 1) // rows * waves
    r = recs[0]
    assert (r["entry"] <= r["staged"]).all() and (r["staged"] <= r["dots"]).all() and (r["dots"] <= r["stored"]).all()


@pytest.mark.parametrize("extreme", [False, True])
def test_mfma_gemv_fused_writes_the_quantizer_planes(extreme):
    # return_q: workgroup 0's waves write the q8_K planes and bsums of their blocks, byte for byte the quantizer's
    n, k, m = 16400, 2304, 3
    W, x = O.problem("tq2_0", n, k, m, 98, extreme)
    wq, ws = host.split("tq2_0", W, n, k)
    assert host.uses_mfma("tq2_0", m, n, k, fused=True)
    y, s, (xq, xd, xb) = host.gemv_f32("tq2_0", dev(wq), dev(ws), dev(x), n, k, store_s=True, return_q=True)
    torch.cuda.synchronize()
    rq, rd, rb = O.quantize("tq2_0", x)
    assert np.array_equal(xq.cpu().numpy(), rq)
    assert np.array_equal(xd.cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(xb.cpu().numpy(), rb)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok("tq2_0", y.cpu().numpy(), ws, rd, rs, r)
