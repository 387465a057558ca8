"""HIP kernels vs the oracle on the same seeded inputs: quantizer bytes exact, int32 block dots exact, every f32 output
within the f32 error bound of the f64 reference_dot (oracle.output_error_bound).  Everything goes through the C ABI
(comp_amd.host -> libkomp_hip.so)."""

import numpy as np
import pytest
import torch

from comp_amd import host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu

# src/komp/verify.py:141-142
PROBLEMS = {"q4_0": ((64, 512, 1), (37, 416, 3), (5, 96, 2)), "tq2_0": ((64, 1024, 1), (37, 768, 3), (5, 1280, 2))}
CONFIGS = {"q4_0": ((32, 4, 4), (16, 2, 2), (64, 8, 4)), "tq2_0": ((32, 2, 4), (16, 1, 2), (64, 4, 4))}
for _f in ("q8_0", "iq4_nl"):  # the ggml formats beyond the reference's two take Q4_0's problems and knob sets
    PROBLEMS[_f], CONFIGS[_f] = PROBLEMS["q4_0"], CONFIGS["q4_0"]
PROBLEMS["q4_k"] = PROBLEMS["tq2_0"]  # 256-value blocks
CONFIGS["q4_k"] = ((32, 4, 4), (16, 2, 2), (128, 8, 8))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_quant(fmt, x):
    xq, xd, *xb = host.quantize(fmt, dev(x), bsums=(fmt == "tq2_0"))
    torch.cuda.synchronize()
    return xq.cpu().numpy(), xd.cpu().numpy(), (xb[0].cpu().numpy() if xb else None)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0"])
@pytest.mark.parametrize("extreme", [False, True])
@pytest.mark.parametrize("m,k", [(1, 256), (3, 2560), (2, 4096 + 256)])
def test_quantizer_bytes_exact(fmt, extreme, m, k):
    rng = np.random.default_rng(100 + m + k + extreme)
    x = O.activations(rng, k, m, block=32 if fmt == "q4_0" else 256, extreme=extreme, outliers=0.01)
    xq, xd, xb = run_quant(fmt, x)
    rq, rd, rb = O.quantize(fmt, x)
    assert np.array_equal(xq, rq)
    assert np.array_equal(xd.view(np.uint32), rd.view(np.uint32))
    if fmt == "tq2_0":
        assert np.array_equal(xb, rb)
    assert host.act_blocks(fmt, xq, xd, xb) == O.act_blocks(fmt, rq, rd)


def test_q8_0_f16_scale_edges():
    # d = amax / 127 rounds to f16 subnormals, to f16 overflow (inf) and exactly to 1
    k = 32 * 6
    x = np.zeros((1, k), np.float32)
    x[0, 0:32] = np.linspace(-127, 127, 32, dtype=np.float32)  # amax 127 -> d 1, q == x
    x[0, 32:64] = 3e-6  # d in the f16 subnormal range
    x[0, 64:96] = np.float32(1e38)  # f16(d) overflows to inf
    x[0, 96:100] = np.float32(1e-36)  # d = amax / 127 is an f32 subnormal with a finite 1 / d
    x[0, 100] = np.float32(-1e-40)  # subnormal input in the same block
    x[0, 128:160] = np.arange(32, dtype=np.float32) - np.float32(15.5)  # ties at k + 0.5 (d = 16.5 / 127)
    x[0, 160:192] = 0.0
    xq, xd, _ = run_quant("q4_0", x)
    rq, rd = O.quant_q8_0(x)
    assert np.array_equal(xq, rq)
    assert np.array_equal(xd.view(np.uint32), rd.view(np.uint32))
    assert np.isinf(xd[0, 2]) and xd[0, 5] == 0.0


def tie_blocks():
    """q8_K blocks whose largest |x| occurs with both signs: the first index decides mx (and the sign of every q)."""
    k = 256 * 8
    x = np.clip(np.random.default_rng(5).normal(size=(1, k)), -4.5, 4.5).astype(np.float32)  # below every planted |x|
    x[0, 10], x[0, 20] = 7.0, -7.0  # first positive, different lanes of the 16-lane row
    x[0, 256 + 3], x[0, 256 + 200] = -5.0, 5.0  # first negative, different lanes
    x[0, 512 + 5], x[0, 512 + 9] = -6.0, 6.0  # first negative, same lane
    x[0, 768 + 5], x[0, 768 + 9], x[0, 768 + 250] = 6.5, -6.5, -6.5  # first positive, same lane, three occurrences
    x[0, 1024:1280] = 0.0  # all-zero block
    x[0, 1280 + 254], x[0, 1280 + 255] = 5.5, -5.5  # tie inside the last lane
    x[0, 1536:1792] = -0.0  # negative zeros only: d = 0, q = 0
    x[0, 1792 + 100] = -1e4  # single spike, no tie
    return x


def test_q8_K_first_index_and_ties():
    x = tie_blocks()
    xq, xd, xb = run_quant("tq2_0", x)
    rq, rd, rb = O.quant_q8_K(x)
    assert np.array_equal(xq, rq) and np.array_equal(xd.view(np.uint32), rd.view(np.uint32)) and np.array_equal(xb, rb)
    assert xq[0, 10] == -127 and xq[0, 20] == 127 and xq[0, 256 + 3] == -127 and xq[0, 512 + 5] == -127
    assert xq[0, 768 + 5] == -127 and xq[0, 1280 + 254] == -127 and xd[0, 4] == 0.0 and xd[0, 6] == 0.0


def test_q8_K_random_ties_standalone_and_fused():
    # 64 blocks, each with its largest |x| planted at two random positions with opposite signs in random order
    rng = np.random.default_rng(17)
    nblk = 64
    x = rng.normal(size=(nblk, 256)).astype(np.float32)
    for b in range(nblk):
        i, j = rng.choice(256, size=2, replace=False)
        a = np.float32(abs(rng.normal()) + 8.0)
        x[b, i], x[b, j] = (a, -a) if rng.random() < 0.5 else (-a, a)
    x = x.reshape(1, -1)
    xq, xd, xb = run_quant("tq2_0", x)
    rq, rd, rb = O.quant_q8_K(x)
    assert np.array_equal(xq, rq) and np.array_equal(xd.view(np.uint32), rd.view(np.uint32)) and np.array_equal(xb, rb)
    n, k = 40, x.shape[1]
    W, _ = O.problem("tq2_0", n, k, 1, 3)
    wq, ws = host.split("tq2_0", W, n, k)
    _, _, q = host.gemv_f32("tq2_0", dev(wq), dev(ws), dev(x), n, k, return_q=True)
    torch.cuda.synchronize()
    assert np.array_equal(q[0].cpu().numpy(), rq) and np.array_equal(q[1].cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(q[2].cpu().numpy(), rb)


def test_q8_K_tie_blocks_fused():
    x = tie_blocks()
    n, k = 24, x.shape[1]
    W, _ = O.problem("tq2_0", n, k, 1, 4)
    wq, ws = host.split("tq2_0", W, n, k)
    y, s, q = host.gemv_f32("tq2_0", dev(wq), dev(ws), dev(x), n, k, store_s=True, return_q=True)
    torch.cuda.synchronize()
    rq, rd, rb = O.quant_q8_K(x)
    assert np.array_equal(q[0].cpu().numpy(), rq) and np.array_equal(q[1].cpu().numpy().view(np.uint32), rd.view(np.uint32))
    assert np.array_equal(q[2].cpu().numpy(), rb)
    r, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs) and outputs_ok("tq2_0", y.cpu().numpy(), ws, rd, rs, r)


def run_gemv(fmt, n, k, m, seed, extreme, block_n, nb, mode, num_warps):
    W, x = O.problem(fmt, n, k, m, seed, extreme)
    wq, ws = host.split(fmt, W, n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    y, s = host.gemv(fmt, dev(wq), dev(ws), xq, xd, n, k, block_n, nb, mode, num_warps, store_s=True)
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    return y.cpu().numpy(), s.cpu().numpy(), r, rs, xq.cpu().numpy(), rq, ws, rd


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("cfg", [0, 1, 2])
@pytest.mark.parametrize("prob", [0, 1, 2])
@pytest.mark.parametrize("extreme", [False, True])
def test_gemv_verify_problems(fmt, mode, cfg, prob, extreme):
    n, k, m = PROBLEMS[fmt][prob]
    block_n, nb, nw = CONFIGS[fmt][cfg]
    y, s, r, rs, xq, rq, ws, rd = run_gemv(fmt, n, k, m, 1 + extreme, extreme, block_n, nb, mode, nw)
    assert np.array_equal(xq, rq)
    assert np.array_equal(s.astype(np.int64), rs)
    assert outputs_ok(fmt, y, ws, rd, rs, r)


@pytest.mark.parametrize("fmt", ["q4_0", "tq2_0", "q8_0", "iq4_nl", "q4_k"])
@pytest.mark.parametrize("block_n", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("nb", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("nw", [1, 2, 4, 8])
def test_gemv_every_legal_knob(fmt, block_n, nb, nw):
    n, k, m = (77, 96 * 32, 3) if O.FORMATS[fmt]["block"] == 32 else (77, 13 * 256, 3)
    if fmt == "q4_k" and nb > 8:  # q4_k: a lane slot is a 32-byte group; nb 16 is out of range
        with pytest.raises(host._abi.KompArgumentError, match="nb <= 8"):
            run_gemv(fmt, n, k, m, 11, False, block_n, nb, 2, nw)
        return
    y, s, r, rs, _, _, ws, rd = run_gemv(fmt, n, k, m, 11, False, block_n, nb, 2, nw)
    assert np.array_equal(s.astype(np.int64), rs)
    assert outputs_ok(fmt, y, ws, rd, rs, r)


@pytest.mark.parametrize("fmt,n,k", [("q4_0", 16384, 8192), ("q4_0", 16400, 4192), ("tq2_0", 16384, 2816),
                                     ("q4_0", 20000, 1024), ("q8_0", 16400, 4192), ("iq4_nl", 16384, 8192),
                                     ("q8_0", 20000, 1024), ("q4_k", 16400, 4352), ("tq2_0", 16400, 8192)])  # fmt: skip
def test_gemv_auto_plan_throughput_shapes(fmt, n, k):
    # N >= 16384 (16400 and 20000 leave a partial last workgroup); q4_0 reads whole rows in one K step, two passes,
    # except the single-column q4_0 / iq4_nl rows of up to 256 blocks (one pass) and tq2_0
    single = fmt == "tq2_0" or (fmt in ("q4_0", "iq4_nl") and k // 32 <= 256)
    assert host.auto_plan(fmt, 1, n, k)["passes"] == (1 if single else 2)
    y, s, r, rs, _, _, ws, rd = run_gemv(fmt, n, k, 1, 23, False, None, None, 2, None)
    assert np.array_equal(s.astype(np.int64), rs)
    assert outputs_ok(fmt, y, ws, rd, rs, r)


@pytest.mark.parametrize("fmt,n,k", [("q4_0", 4096, 4096), ("q4_0", 4097, 4192), ("q4_0", 127, 4192),
                                     ("q4_0", 16383, 4096), ("q4_0", 300, 96), ("tq2_0", 6912, 2560),
                                     ("tq2_0", 2560, 6912), ("tq2_0", 6913, 2816), ("tq2_0", 16383, 256),
                                     ("tq2_0", 513, 1280), ("q8_0", 4096, 4096), ("q8_0", 4097, 4192),
                                     ("q8_0", 300, 96), ("iq4_nl", 4096, 4096), ("iq4_nl", 127, 4192),
                                     ("iq4_nl", 16383, 4096), ("q4_k", 4096, 4096), ("q4_k", 4097, 4352),
                                     ("q4_k", 6912, 2560), ("q4_k", 300, 256), ("q4_k", 2560, 6912)])  # fmt: skip
@pytest.mark.parametrize("m", [1, 3])
def test_gemv_auto_config_shapes(fmt, n, k, m):
    y, s, r, rs, _, _, ws, rd = run_gemv(fmt, n, k, m, 21, False, None, None, 2, None)
    assert np.array_equal(s.astype(np.int64), rs)
    assert outputs_ok(fmt, y, ws, rd, rs, r)


def test_dp4a_probe_both_modes():
    rng = np.random.default_rng(3)
    edge = np.array([0, -1, 0x7F7F7F7F, -0x7F7F7F80, 0x01010101, 0x0F0F0F0F, 0x03030303, 2**31 - 1, -(2**31),
                     0x80000000 - 2**32], dtype=np.int64)  # fmt: skip  (src/komp/verify.py:47)
    n = 1024
    def vals():
        v = rng.integers(-(2**31), 2**31, size=n)
        pick = rng.random(n) < 0.3
        v[pick] = rng.choice(edge, size=int(pick.sum()))
        return v.astype(np.int32)
    a, b = vals(), vals()
    c = rng.integers(-(2**20), 2**20, size=n).astype(np.int32)
    want = O.dp4a(a, b, c)
    for mode in (1, 2):
        got = host.dp4a_probe(dev(a), dev(b), dev(c), mode).cpu().numpy()
        assert np.array_equal(got, want), mode


def test_decode_probes():
    rng = np.random.default_rng(7)
    wq = rng.integers(0, 256, size=(37, 16), dtype=np.uint8)
    got = host.q4_0_decode(dev(wq)).cpu().numpy()
    assert np.array_equal(got, O.q4_0_values(wq))
    tq = rng.integers(0, 256, size=(5, 64), dtype=np.uint8)
    got = host.tq2_0_decode(dev(tq)).cpu().numpy()
    assert np.array_equal(got, O.tq2_0_values(tq))


@pytest.mark.parametrize("fmt,n,k,knobs", [("q4_0", 300, 4096, (16, 4, 4)), ("q4_0", 4096, 4096, None),
                                           ("tq2_0", 300, 8192, (32, 2, 8)), ("tq2_0", 2560, 8192, None),
                                           ("q8_0", 300, 4096, (16, 4, 4)), ("iq4_nl", 4096, 4096, None)])  # fmt: skip
def test_scale_slab_and_per_tile_scales_agree(fmt, n, k, knobs):
    # a 16-byte aligned WS is staged in LDS per workgroup; a WS view at a 2-byte offset takes the per-tile scale loads
    W, x = O.problem(fmt, n, k, 1, 31)
    wq, ws = host.split(fmt, W, n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    bn, nb, nw = knobs if knobs else (None, 0, 0)
    wq_d, ws_d = dev(wq), dev(ws)
    big = torch.zeros(ws.size + 8, dtype=torch.int16, device="cuda")
    ws_odd = big[1 : 1 + ws.size].view(ws.shape)
    ws_odd.copy_(ws_d)
    assert ws_d.data_ptr() % 16 == 0 and ws_odd.data_ptr() % 16 == 2
    y1, s1 = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
    y2, s2 = host.gemv(fmt, wq_d, ws_odd, xq, xd, n, k, bn, nb, 2, nw, store_s=True)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2) and torch.equal(y1.view(torch.int32), y2.view(torch.int32))
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert np.array_equal(s1.cpu().numpy().astype(np.int64), rs) and outputs_ok(fmt, y1.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("fmt,n,k,fused", [("tq2_0", 6912, 2560, True), ("tq2_0", 6913, 2816, False),
                                           ("q4_0", 4097, 4096, True), ("tq2_0", 4097, 2048, False),
                                           ("tq2_0", 300, 1280, False), ("q4_0", 6144, 4096, True),
                                           ("q4_0", 4096, 14336, True), ("tq2_0", 2560, 6912, True),
                                           ("q8_0", 4097, 4096, True), ("iq4_nl", 6144, 4096, True),
                                           ("q4_k", 4096, 4096, True), ("q4_k", 4096, 14336, True)])  # fmt: skip
def test_one_workgroup_per_cu_plans(fmt, n, k, fused):
    # small single-column GEMVs plan one workgroup of ceil(N / CUs) rows per CU; the first five shapes give the waves
    # more row slots than rows (clipped per wave), q4_0 4097x4096 and tq2_0 4097x2048 with the scale slab in LDS
    p = host.auto_plan(fmt, 1, n, k, fused)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if (fmt, n) == ("tq2_0", 300):
        # one TQ2_0 column over fewer rows a CU than one wave stages for: as many waves as one staging pass takes (5
        # blocks x 16 threads: 2), each with its full rows
        assert (p["waves"], p["block_n"], p["passes"]) == (2, 2 * (64 // p["lanes_per_row"]), 1)
    else:
        assert p["block_n"] == -(-n // cus) and p["passes"] == 1
    W, x = O.problem(fmt, n, k, 1, 29)
    wq, ws = host.split(fmt, W, n, k)
    if fused:
        y, s = host.gemv_f32(fmt, dev(wq), dev(ws), dev(x), n, k, store_s=True)
    else:
        xq, xd, *_ = host.quantize(fmt, dev(x))
        y, s = host.gemv(fmt, dev(wq), dev(ws), xq, xd, n, k, None, 0, 2, 0, store_s=True)
    torch.cuda.synchronize()
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    assert np.array_equal(s.cpu().numpy().astype(np.int64), rs) and outputs_ok(fmt, y.cpu().numpy(), ws, rd, rs, r)


@pytest.mark.parametrize("knobs", [(64, 4, 8), (16, 4, 2), None])
def test_q4_k_scale_slab_and_global_scales(knobs):
    # q4_k's 16-byte scale entries: (64, 4, 8) needs 8 x 8 rows x 32 blocks x 16 B = 32 KB of slab, past the 16 KB
    # limit, so its lanes load their entries from global memory; (16, 4, 2) stages an 8 KB slab in LDS
    n, k = 300, 8192
    bn, nb, nw = knobs or (None, None, None)
    y, s, r, rs, _, _, ws, rd = run_gemv("q4_k", n, k, 2, 41, False, bn, nb, 2, nw)
    assert np.array_equal(s.astype(np.int64), rs)
    assert outputs_ok("q4_k", y, ws, rd, rs, r)


def test_q4_k_extreme_scales_every_mode():
    # every scale and min at 63 or 0, d / dmin at 65504 or the smallest subnormal, nibbles all 0 or 15
    for mode in (0, 1, 2):
        y, s, r, rs, _, _, ws, rd = run_gemv("q4_k", 45, 2304, 3, 43, True, 16, 4, mode, 2)
        assert np.array_equal(s.astype(np.int64), rs)
        assert outputs_ok("q4_k", y, ws, rd, rs, r)


@pytest.mark.parametrize("nbytes", [16, 4096, 32768 + 48, 4599808, 33030144 + 16])
def test_stream_read_probe_reads_every_byte(nbytes):
    # the streaming-read probe bench.py measures GEMVs against: every dword is folded into exactly one wave's word
    rng = np.random.default_rng(nbytes)
    data = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    out = host.stream_read(dev(data.view(np.int32)))
    torch.cuda.synchronize()
    words = out.cpu().numpy().view(np.uint32)
    assert words.size == host.stream_read_words(nbytes)
    assert np.bitwise_xor.reduce(words) == np.bitwise_xor.reduce(data)
    # workgroup g, wave w, lane l reads 16-byte pieces 2048 g + 512 u + 64 w + l (u < 4)
    grid = words.size // 8
    pieces = np.zeros(grid * 2048 * 4, dtype=np.uint32)
    pieces[: data.size] = data
    per_wave = np.bitwise_xor.reduce(pieces.reshape(grid, 4, 8, 64 * 4), axis=(1, 3)).reshape(-1)
    assert np.array_equal(words, per_wave)


@pytest.mark.parametrize("fmt,n,k", [("tq2_0", 127, 65536), ("tq2_0", 1000, 32768), ("q4_0", 127, 32768),
                                     ("q8_0", 127, 32768), ("iq4_nl", 127, 32768), ("q4_k", 127, 32768)])  # fmt: skip
def test_few_rows_long_columns(fmt, n, k):
    # one column over few rows a CU with rows of 128-256 blocks: the plans that stage in one pass of up to 16 waves
    # (several K steps a row), q8 and f32 in, dp4a and (Q4_0, TQ2_0) bytes mode, against the oracle
    print(f"few rows long columns {fmt} {n}x{k}", flush=True)
    W, x = O.problem(fmt, n, k, 1, 77)
    wq, ws = host.split(fmt, W, n, k)
    wq_d, ws_d = dev(wq), dev(ws)
    rq, rd, _ = O.quantize(fmt, x)
    r, rs = O.gemv(fmt, wq, ws, rq, rd, n, k)
    xq, xd, *_ = host.quantize(fmt, dev(x))
    for mode in (2, 0) if fmt in ("q4_0", "tq2_0") else (2,):
        y, s = host.gemv(fmt, wq_d, ws_d, xq, xd, n, k, None, 0, mode, 0, store_s=True)
        yf, sf = host.gemv_f32(fmt, wq_d, ws_d, dev(x), n, k, None, 0, mode, 0, store_s=True)
        torch.cuda.synchronize()
        for yy, ss in ((y, s), (yf, sf)):
            assert np.array_equal(ss.cpu().numpy().astype(np.int64), rs)
            assert outputs_ok(fmt, yy.cpu().numpy(), ws, rd, rs, r)
