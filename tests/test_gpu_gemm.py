"""Matrix-core GEMM (komp_{q4_0,tq2_0,q8_0,iq4_nl,q4_k}_gemm) vs the oracle: int32 block dots S exact, every output of Y
within the f32 error bound of the f64 reference_dot, on the same seeded problems.  Shapes cover the kernel's tails: rows not a
multiple of 16, column counts around the 16-column tiles and the 64-column workgroups, Q4_0 block counts that are not
a multiple of the 4-block K step, scale planes that take the 2-byte staging path, padded weight rows, and the
two-row-tile workgroups of tall matrices.  Everything goes through the C ABI."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

# (n, k, m)
SHAPES = {
    "q4_0": [(16, 128, 1), (16, 128, 2), (64, 512, 4), (37, 416, 5), (5, 96, 17), (33, 1024, 31), (100, 4096, 33),
             (48, 2048, 64), (40, 640, 65), (300, 768, 130)],
    "tq2_0": [(16, 256, 1), (16, 256, 3), (64, 1024, 4), (37, 768, 5), (5, 1280, 17), (33, 2560, 31),
              (100, 2560, 33), (40, 6912, 64), (48, 256, 65), (300, 512, 130)],
}
SHAPES["q8_0"] = SHAPES["iq4_nl"] = SHAPES["q4_0"]
SHAPES["q4_k"] = SHAPES["tq2_0"]  # 256-value blocks
BLK32 = ("q4_0", "q8_0", "iq4_nl")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def check(fmt, n, k, m, seed, extreme=False, ws_offset=0, pad=0):
    W, x = O.problem(fmt, n, k, m, seed, extreme)
    wq, ws = host.split(fmt, W, n, k)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    wq_d = dev(np.pad(wq, ((0, 0), (0, pad))))[:, : wq.shape[1] + pad]
    if ws_offset:  # a scale plane that starts 2 bytes into its allocation (not 16-byte aligned)
        base = torch.zeros(ws.size + ws_offset, dtype=torch.int16, device="cuda")
        base[ws_offset:] = dev(ws.reshape(-1))
        ws_d = base[ws_offset:].view(n, -1)
    else:
        ws_d = dev(ws)
    print(f"gemm {fmt} n={n} k={k} m={m} seed={seed} extreme={extreme} ws_offset={ws_offset} pad={pad}", flush=True)
    xq_d, xd_d = dev(rq), dev(rd)
    y, s = host.gemm(fmt, wq_d, ws_d, xq_d, xd_d, n, k, store_s=True)
    # the kernel without S (its own instantiation: blocks past K and slots past a wave's last step add exact zeros
    # where the S kernel branches) gives the same Y bit for bit
    y_plain, _ = host.gemm(fmt, wq_d, ws_d, xq_d, xd_d, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs)
    assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)
    assert torch.equal(y_plain, y)
    return y


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
@pytest.mark.parametrize("shape", range(10))
@pytest.mark.parametrize("extreme", [False, True])
def test_gemm_matches_oracle(fmt, shape, extreme):
    n, k, m = SHAPES[fmt][shape]
    check(fmt, n, k, m, 300 + shape, extreme)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemm_unaligned_scales_and_padded_rows(fmt):
    k = 416 if fmt in BLK32 else 768
    odd = (1, 3) if fmt != "q4_k" else (8, 24)  # q4_k's 16-byte scale entries need a 16-byte aligned plane
    check(fmt, 45, k, 20, 11, ws_offset=odd[0], pad=48)
    check(fmt, 64, 2 * k if fmt in BLK32 else 1024, 8, 12, ws_offset=odd[1])


# one shape per plan family on a 256-CU device: (n, k, m, rows per workgroup, columns per workgroup)
FAMILIES = [
    (4000, 512, 20, 16, 32),    # ~1 row tile per CU: K split over 8 waves
    (6144, 512, 20, 32, 32),    # 1.5 per CU, 2 column tiles: 4 x 2 waves
    (9600 + 7, 512, 12, 64, 16),  # 2..8 per CU, 1 column tile: 4 x 2 waves, 2 row tiles each
    (9600, 256, 20, 64, 32),    # 2..4 per CU, 2 column tiles: 4 x 2 waves, 2 row tiles each (Q8_0: 2 x 4 waves)
    (20000 + 3, 256, 40, 64, 48),  # 4..8 per CU, 3 column tiles: 2 x 2 waves, 2 row tiles each (Q8_0: 2 x 4)
    (33600, 256, 4, 128, 16),   # > 8 per CU: 8 waves, each its own rows
    (33600 - 5, 256, 12, 256, 16),  # ... 2 row tiles each
    (16400, 256, 70, 128, 48),  # ... 3 column tiles, 2 column groups
    (4096, 512, 64, 64, 16),    # 4 column tiles over 1 row tile per CU: 4 column groups of 1 tile (4 x 2 waves)
    (6912, 256, 64, 64, 32),    # ... over 1.7 per CU: 2 column groups of 2 tiles (2 x 2 waves; Q8_0: 2 x 4)
]


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
@pytest.mark.parametrize("fam", range(len(FAMILIES)))
def test_gemm_plan_families(fmt, fam):
    n, k, m, rows, cols = FAMILIES[fam]
    if fmt in ("tq2_0", "q4_k"):
        k = 512 if k == 256 else 1024
    if fmt == "q8_0" and rows == 256:
        rows = 128  # Q8_0 waves take one row tile each (two would need more than 256 VGPRs)
    plan = host.gemm_plan(fmt, m, n, k)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256 and fmt != "q4_k":  # q4_k: its own families
        assert (plan["rows"], plan["cols"]) == (rows, cols), plan
    check(fmt, n, k, m, 60 + fam)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemv_auto_routes_batches_to_gemm(fmt):
    n, k, m = (96, 1024, 12) if fmt in BLK32 else (96, 1536, 12)
    W, x = O.problem(fmt, n, k, m, 31)
    wq, ws = host.split(fmt, W, n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    lo = host.GEMM_MIN_M[fmt]
    assert host.uses_gemm(fmt, m, n, k) and host.uses_gemm(fmt, lo, n, k) and not host.uses_gemm(fmt, lo - 1, n, k)
    assert not host.uses_gemm(fmt, m, n, k, mode=1) and not host.uses_gemm(fmt, m, n, k, fused=True)
    assert host.knob_equivalent(fmt, m, n, k) is None
    y_auto, s_auto = host.gemv(fmt, dev(wq), dev(ws), xq, xd, n, k, block_n=None, mode=2, store_s=True)
    y_gemm, s_gemm = host.gemm(fmt, dev(wq), dev(ws), xq, xd, n, k, store_s=True)
    y_gemv, s_gemv = host.gemv(fmt, dev(wq), dev(ws), xq, xd, n, k, 32, 2, 2, 4, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(y_auto, y_gemm) and torch.equal(s_auto, s_gemm)
    assert torch.equal(s_gemm, s_gemv)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert outputs_ok(fmt, y_gemm.cpu().numpy(), ws, rd, rs, r) and outputs_ok(fmt, y_gemv.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemm_multi_matrix_batches(fmt):
    k = 512
    ns = (40, 24, 64)
    m = 9
    rng = np.random.default_rng(41)
    mats, refs = [], []
    x = O.activations(rng, k, m, block=O.ACT_BLOCK[O.FORMATS[fmt]["act"]])
    rq, rd, _ = O.quantize(fmt, x)
    for n in ns:
        W = O.weights(fmt, rng, n, k)
        wq, ws = host.split(fmt, W, n, k)
        mats.append((dev(wq), dev(ws), n))
        refs.append((ws, *O.gemv(fmt, wq, ws, rq, rd, n, k)))
    ys = host.gemv_multi(fmt, mats, k, xq=dev(rq), xd=dev(rd))
    torch.cuda.synchronize()
    for y, (ws, r, rs) in zip(ys, refs):
        assert outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemm_empty_k_writes_zeros(fmt):
    n, m = 20, 5
    wq = torch.zeros((n, 16), dtype=torch.uint8, device="cuda")  # a row stride of 16 bytes, no quant bytes used
    ws = torch.zeros((n, 0), dtype=torch.int16, device="cuda")
    xq = torch.zeros((m, 0), dtype=torch.int8, device="cuda")
    xd = torch.zeros((m, 0), dtype=torch.float32, device="cuda")
    y = torch.full((m, n), 7.0, device="cuda")
    host.gemm_into(fmt, wq, ws, xq, xd, y, n, 0)
    torch.cuda.synchronize()
    assert torch.count_nonzero(y).item() == 0


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
def test_gemm_graph_replays(fmt):
    n, k, m = (200, 1024, 24) if fmt in BLK32 else (200, 1280, 24)
    W, x = O.problem(fmt, n, k, m, 51)
    wq, ws = host.split(fmt, W, n, k)
    wq, ws = dev(wq), dev(ws)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    y_eager, _ = host.gemm(fmt, wq, ws, xq, xd, n, k)
    y = torch.empty_like(y_eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        host.gemm_into(fmt, wq, ws, xq, xd, y, n, k)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        host.gemm_into(fmt, wq, ws, xq, xd, y, n, k)
    for _ in range(3):
        y.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager)


@pytest.mark.parametrize("m", [4, 16, 33])
def test_q4_k_gemm_plans_and_long_rows(m):
    # every Q4_K plan family (one row tile per wave, 1-2 column tiles) and a row long enough that the unpacked scale
    # slab pushes the plan down the family list
    for n, k in ((4000, 512), (9600, 512), (33600, 256), (700, 14336)):
        plan = host.gemm_plan("q4_k", m, n, k)
        assert plan is not None and plan["cols"] <= 64 and plan["rows"] <= 128, plan
        check("q4_k", n, k, m, 90 + m)
