"""The C-ABI library without a GPU: it loads, exports exactly what include/komp_abi.h declares, and rejects bad
arguments before touching the device."""

import ctypes
import os
import re
import subprocess

import pytest

from comp_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "komp_abi.h")


def declared():
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int|const char\*)\s+(komp_\w+)\(", text, re.M))


def test_header_and_binding_agree():
    assert declared() == set(_abi.SIGNATURES)
    kinds = re.search(r"#define KOMP_TIMING_KINDS (\d+)", open(HEADER).read())
    assert int(kinds.group(1)) == len(_abi.TIMING_KINDS)


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    for name in declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (komp_\w+)", out))
    assert exported == declared()


def test_abi_version():
    assert _abi.lib().komp_abi_version() == 1


def _gemv(name="komp_q4_0_gemv", M=1, N=4, K=64, SW=32, bn=32, nb=4, mode=2, nw=4, ptr=16):
    p = ctypes.c_void_p(ptr)
    return getattr(_abi.lib(), name)(p, p, p, p, p, None, M, N, K, SW, bn, nb, mode, nw, None)


@pytest.mark.parametrize("kw,needle", [
    (dict(K=33), "multiple of the 32"), (dict(SW=24), "SW"), (dict(SW=16), "SW"), (dict(mode=3), "mode"),
    (dict(bn=33), "block_n"), (dict(nb=3), "nb"), (dict(nw=16), "num_warps"), (dict(M=-1), "negative"),
    (dict(ptr=8), "16-byte aligned"), (dict(name="komp_tq2_0_gemv", K=128, SW=32), "multiple of the 256"),
    (dict(K=2 ** 31 + 32, SW=2 ** 30 + 16), "2^31"), (dict(K=64 * 3000, SW=96000), "LDS"),
])  # fmt: skip
def test_gemv_rejects_bad_arguments(kw, needle):
    st = _gemv(**kw)
    assert st == _abi.KOMP_EINVAL
    assert needle in _abi.last_error()


def test_q4_k_rejects_bad_arguments():
    lib = _abi.lib()
    p16, p8 = ctypes.c_void_p(16), ctypes.c_void_p(8)
    q4k = dict(name="komp_q4_k_gemv", K=256, SW=128)
    assert _gemv(**q4k, nb=16) == _abi.KOMP_EINVAL and "nb <= 8" in _abi.last_error()  # 32-byte lane slots
    assert _gemv(name="komp_q4_k_gemv", K=288, SW=144) == _abi.KOMP_EINVAL
    assert "multiple of the 256" in _abi.last_error()
    st = lib.komp_q4_k_gemv(p16, p8, p16, p16, p16, None, 1, 4, 256, 128, 32, 4, 2, 4, None)  # WS 8-byte aligned
    assert st == _abi.KOMP_EINVAL and "16-byte aligned" in _abi.last_error()
    st = lib.komp_q4_k_split(p16, p16, p8, 4, 256, 128, None)
    assert st == _abi.KOMP_EINVAL and "WS 16-byte aligned" in _abi.last_error()
    rows, cols, waves = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.komp_gemm_plan(4, 64, 4096, 4096, 2048, ctypes.byref(rows), ctypes.byref(cols), ctypes.byref(waves)) == 0
    assert cols.value == 64 and rows.value <= 128  # q4_k: one row tile per wave
    st = lib.komp_q4_k_gemm(p16, p8, p16, p16, p16, None, 4, 4, 256, 128, None)
    assert st == _abi.KOMP_EINVAL and "16-byte aligned" in _abi.last_error()


def test_empty_shapes_are_no_ops():
    assert _gemv(M=0) == 0 and _gemv(N=0) == 0
    lib = _abi.lib()
    assert lib.komp_quant_q8_0(None, None, None, 0, 64, 4, None) == 0
    assert lib.komp_quant_q8_K(None, None, None, None, 3, 0, None) == 0
    assert lib.komp_dp4a_probe(None, None, None, None, 0, 2, None) == 0
    assert lib.komp_stream_read(None, 0, None, None) == 0


def _multi(count=2, n=(4, 4), K=64, sw=(32, 32), wq_ptr=16, x=False, xq=True, mode=2, arrays=True):
    lib = _abi.lib()
    P = ctypes.c_void_p * 4
    I64 = ctypes.c_int64 * 4
    p = ctypes.c_void_p(16)
    wq = P(*([wq_ptr] * 4)) if arrays else None
    ws = P(*([16] * 4))
    y = P(*([16] * 4))
    ns = I64(*(list(n) + [4] * (4 - len(n))))
    sws = I64(*(list(sw) + [32] * (4 - len(sw))))
    return lib.komp_q4_0_gemv_multi(count, wq, ws, y, ns, sws, p if xq else None, p if xq else None, p if x else None,
                                    1, K, 0, 0, mode, 0, None)  # fmt: skip


@pytest.mark.parametrize("kw,needle", [
    (dict(count=0), "count"), (dict(count=5), "count"), (dict(x=True), "either"), (dict(xq=False), "either"),
    (dict(arrays=False), "arrays"), (dict(n=(4, -1)), "N="), (dict(sw=(32, 24)), "SW"), (dict(K=48), "multiple"),
    (dict(wq_ptr=8), "16-byte aligned"), (dict(mode=5), "mode"),
])  # fmt: skip
def test_gemv_multi_rejects_bad_arguments(kw, needle):
    assert _multi(**kw) == _abi.KOMP_EINVAL
    assert needle in _abi.last_error()


def test_gemv_multi_empty_is_a_no_op():
    assert _multi(n=(0, 0)) == 0


def test_quantizers_reject_bad_arguments():
    lib = _abi.lib()
    p = ctypes.c_void_p(16)
    assert lib.komp_quant_q8_0(p, p, p, 1, 48, 4, None) == _abi.KOMP_EINVAL and "multiple of 32" in _abi.last_error()
    assert lib.komp_quant_q8_0(p, p, p, 1, 64, 0, None) == _abi.KOMP_EINVAL and "bb" in _abi.last_error()
    assert lib.komp_quant_q8_K(p, p, p, None, 1, 300, None) == _abi.KOMP_EINVAL
    assert lib.komp_quant_q8_K(ctypes.c_void_p(8), p, p, None, 1, 256, None) == _abi.KOMP_EINVAL
    assert lib.komp_dp4a_probe(p, p, p, p, 4, 0, None) == _abi.KOMP_EINVAL
    assert lib.komp_stream_read(p, 24, p, None) == _abi.KOMP_EINVAL and "multiple of 16" in _abi.last_error()
    assert lib.komp_stream_read(ctypes.c_void_p(8), 32, p, None) == _abi.KOMP_EINVAL
    assert lib.komp_stream_read(None, 32, p, None) == _abi.KOMP_EINVAL


def test_python_errors_carry_the_message():
    with pytest.raises(_abi.KompArgumentError, match="mode=7"):
        _abi.check(_gemv(mode=7), "komp_q4_0_gemv")


@pytest.mark.parametrize("fmt,n,k", [(0, 4096, 4096), (0, 128256, 4096), (0, 4097, 4192), (1, 6912, 2560),
                                     (1, 2560, 6912), (1, 32768, 8192), (0, 1, 32), (1, 3, 256), (0, 28672, 8192),
                                     (0, 28672, 14336), (0, 4096, 14336), (0, 20000, 1024)])  # fmt: skip
@pytest.mark.parametrize("fused", [False, True])
def test_auto_plan(fmt, n, k, fused):
    # without a device the library plans for 256 CUs (MI355X)
    bn, nb, nw, lanes, passes = _abi.auto_plan(fmt, 1, n, k, fused)
    assert _abi.auto_config(fmt, 1, n, k, fused) == (bn, nb, nw)
    assert nb in (1, 2, 4, 8, 16) and lanes in (4, 8, 16, 32, 64) and passes >= 1
    assert nw * (64 // lanes) * passes >= bn  # the waves' row slots cover the workgroup's rows
    blocks_per_step = nb * (lanes if fmt == 0 else lanes // 4)
    nblk = k // (32 if fmt == 0 else 256)
    if n < 16384 and (fused or fmt == 1):  # one workgroup per CU, one row group per wave, one K step up to nb 8
        assert bn == -(-n // 256) and 1 <= nw <= 16 and passes == 1 and nw == -(-bn // (64 // lanes))
        assert blocks_per_step >= nblk or nb == 8
    elif n < 16384:  # unfused q4_0: an explicit knob set whose mapping gives the same lanes per row and passes
        rpw = bn // nw
        assert bn in (8, 16, 32, 64, 128) and nw in (1, 2, 4, 8) and bn % nw == 0
        assert lanes == 64 // min(rpw, 16) and passes == rpw // min(rpw, 16)
        assert blocks_per_step >= nblk or nb == 4  # one K step unless the q4_0 nb cap applies
    elif fmt == 0 and not fused and nblk <= 256:  # one q4_0 column, rows of up to 256 blocks: one K step of nb 4
        assert nb == 4 and passes == 1 and lanes == max(16, 1 << (-(-nblk // 4) - 1).bit_length())
        rpw = 64 // lanes  # 8 rows a workgroup, at least 4 waves
        assert blocks_per_step >= nblk and (bn, nw) == (max(4, 8 // rpw) * rpw, max(4, 8 // rpw))
    elif fmt == 0 and nblk <= 128:  # fused q4_0 rows of up to 128 blocks: 16 lanes per row, 8 waves
        assert (bn, nb, nw, lanes, passes) == (32, 2, 8, 16, 1)
    elif fmt == 0:  # throughput regime, q4_0: whole rows in one K step, two passes per wave
        assert passes == 2 and nw == 4 and bn == nw * (64 // lanes) * 2 and (blocks_per_step >= nblk or lanes == 64)
    else:  # throughput regime, tq2_0: nb 4, one K step (a lane quad per block), 8 waves
        assert (nb, nw, passes) == (4, 8, 1) and lanes == max(16, nblk) and bn == 8 * (64 // lanes)


@pytest.mark.parametrize("mode,m", [(0, 1), (1, 1), (2, 2), (2, 3)])
def test_auto_plan_other_modes_and_columns_use_knob_sets(mode, m):
    for fmt, n, k in ((0, 4096, 4096), (1, 6912, 2560), (1, 2560, 6912)):
        if (mode == 2 and (fmt == 1 or m > 1)) or (mode == 0 and fmt == 1):
            continue  # one workgroup per CU: TQ2_0 at 1-3 columns (dp4a and bytes), Q4_0 at 2-3 (the tests below)
        for fused in (False, True):
            if fused and mode == 0 and fmt == 0:
                continue  # one fused Q4_0 column in bytes mode: one workgroup per CU, as in dp4a mode
            bn, nb, nw, lanes, passes = _abi.auto_plan(fmt, m, n, k, fused, mode)
            assert bn in (8, 16, 32, 64, 128) and nw in (1, 2, 4, 8) and lanes == 64 // min(bn // nw, 16)


@pytest.mark.parametrize("m,w1,w2", [(1, (27, 4, 7, 16, 1), (10, 2, 10, 64, 1)),
                                     (2, (27, 4, 7, 16, 1), (10, 2, 10, 64, 1)),
                                     # 3 x 10 blocks x 16 = 480 staging threads: 8 waves of 4 rows, one staging pass
                                     (3, (32, 4, 8, 16, 1), (10, 2, 10, 64, 1))])
def test_auto_plan_bitnet_shapes(m, w1, w2):
    # the BitNet-2B shapes, 1-3 columns: one workgroup per CU (256 CUs), fused and unfused alike, dp4a and bytes
    for mode in (2, 0):
        assert _abi.auto_plan(1, m, 6912, 2560, True, mode) == _abi.auto_plan(1, m, 6912, 2560, False, mode) == w1
        assert _abi.auto_plan(1, m, 2560, 6912, True, mode) == _abi.auto_plan(1, m, 2560, 6912, False, mode) == w2


@pytest.mark.parametrize("n,k,plan", [(4096, 4096, (16, 2, 16, 64, 1)), (6144, 4096, (24, 4, 12, 32, 1)),
                                      (4096, 14336, (16, 4, 16, 64, 1))])  # nb 4 at most for 2-3 columns
def test_auto_plan_q4_0_columns_llama_shapes(n, k, plan):
    for m in (2, 3):
        assert _abi.auto_plan(0, m, n, k, True) == _abi.auto_plan(0, m, n, k, False) == plan
    assert _abi.auto_plan(0, 1, n, k, False)[2] == 8  # one unfused column keeps the 8-wave plan


def test_mfma_plan_needs_aligned_rows():
    # the three-column TQ2_0 matrix-core GEMV: 16-byte aligned row strides of at least the packed row, more than 8
    # rows a CU (256 CUs when no device is visible)
    assert _abi.gemv_mfma_plan(1, False, 2, 3, 6912, 2560, 640) is not None
    assert _abi.gemv_mfma_plan(1, False, 2, 3, 6912, 2560, 704) is not None
    assert _abi.gemv_mfma_plan(1, False, 2, 3, 6912, 2560, 648) is None
    assert _abi.gemv_mfma_plan(1, False, 2, 3, 6912, 2560, 624) is None
    assert _abi.gemv_mfma_plan(1, False, 2, 2, 6912, 2560, 640) is None


def test_auto_plan_tq2_one_column_stages_in_one_pass():
    # one TQ2_0 column over few rows a CU: as many waves as one staging pass of 16 threads a block takes, each with
    # its full rows; fused, q8 in and bytes mode alike; the BitNet-2B plans already have the waves
    for fused in (False, True):
        for mode in (2, 0):
            assert _abi.auto_plan(1, 1, 127, 2816, fused, mode) == (12, 4, 3, 16, 1)  # 11 blocks: 176 threads
            assert _abi.auto_plan(1, 1, 127, 6912, fused, mode) == (7, 2, 7, 64, 1)  # 27 blocks: 432 threads
            assert _abi.auto_plan(1, 1, 6912, 2560, fused, mode) == (27, 4, 7, 16, 1)


def test_auto_plan_fused_one_column_stages_in_one_pass():
    # one f32 column over few rows a CU: 8 staging threads a block of q8_0 activations, 16 of q8_K ones, as many
    # waves as one pass takes (at most 16), each with its full rows; the Llama-3-8B plans keep theirs
    assert _abi.auto_plan(0, 1, 300, 4096, True) == (16, 2, 16, 64, 1)  # 128 blocks x 8 threads
    assert _abi.auto_plan(2, 1, 127, 4096, True) == (16, 4, 16, 64, 1)
    assert _abi.auto_plan(4, 1, 127, 4096, True) == (8, 2, 4, 32, 1)  # q4_k: 16 blocks x 16 threads
    assert _abi.auto_plan(0, 1, 4097, 4096, True) == (17, 4, 9, 32, 1)
    assert _abi.auto_plan(0, 1, 6144, 4096, True) == (24, 4, 12, 32, 1)


def test_auto_plan_q4_0_columns_one_k_step():
    # 131 blocks a row (K 4192): the one-CU plan's 32 lanes x nb 4 would take two K steps, 64 lanes one; with q8 in,
    # 2-3 columns take the one-column plan's shape, fused launches keep the wider plan
    for n in (4097, 6913):
        for m in (2, 3):
            assert _abi.auto_plan(0, m, n, 4192, False) == (8, 4, 8, 64, 1)
            assert _abi.auto_plan(0, m, n, 4192, True)[3] == 32


def test_auto_plan_tq2_columns_few_rows_use_knob_sets():
    # 2-3 columns need at least 7 waves of the one-workgroup-per-CU plan; fewer rows take the 8-wave knob-set plans,
    # except three dp4a columns whose q8_K staging (16 threads per block and column) needs more than 8 waves: one
    # row a wave, as many waves as one staging pass takes (3 x 11 blocks x 16 = 528 threads: 9 waves)
    for n, k in ((127, 2816), (4097, 2816)):
        for fused in (True, False):
            bn, nb, nw, lanes, passes = _abi.auto_plan(1, 2, n, k, fused)
            assert bn in (8, 16, 32, 64, 128) and nw == 8 and lanes == 64 // min(bn // nw, 16)
            assert _abi.auto_plan(1, 3, n, k, fused) == (9, 1, 9, 64, 1)
            bn, nb, nw, lanes, passes = _abi.auto_plan(1, 3, n, k, fused, 0)  # bytes mode: the knob sets
            assert nw == 8 and lanes == 64 // min(bn // nw, 16)
    assert _abi.auto_plan(1, 3, 1000, 4096, False) == (12, 1, 12, 64, 1)
    assert _abi.auto_plan(1, 3, 300, 2560, False)[2] == 8  # 480 staging threads: 8 waves take them in one pass
    assert _abi.auto_plan(1, 3, 127, 6912, False)[2] == 8  # 1296: two passes either way, 8 waves
    assert _abi.auto_plan(1, 3, 6913, 2816, True)[2] == 7  # 28 rows per CU: 7 waves of 4 rows


def test_auto_plan_tq2_columns_fall_back_when_the_lean_kernel_cannot_take_them():
    # a row of 256 blocks at 3 columns needs more than 160 KB of staged activations: the 8-wave knob-set plan, which
    # the general kernel runs
    bn, nb, nw, lanes, passes = _abi.auto_plan(1, 3, 4096, 65536, True)
    assert nw <= 8 and bn in (8, 16, 32, 64, 128) and lanes == 64 // min(bn // nw, 16)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_abi, "_lib", None)
    monkeypatch.setattr(_abi, "LIB_PATH", str(tmp_path / "libkomp_hip.so"))
    with pytest.raises(_abi.KompError, match="not built"):
        _abi.lib()


@pytest.mark.parametrize("fn,blk,row", [("komp_q4_0_split", 32, 16), ("komp_tq2_0_split", 256, 64)])
def test_split_rejects_bad_arguments(fn, blk, row):
    lib = _abi.lib()
    f = getattr(lib, fn)
    p = ctypes.c_void_p(256)
    assert f(p, p, p, 4, 3 * blk + 1, 3 * row, None) == _abi.KOMP_EINVAL and "multiple" in _abi.last_error()
    assert f(p, p, p, 4, 3 * blk, 3 * row - 16, None) == _abi.KOMP_EINVAL and "SW" in _abi.last_error()
    assert f(p, p, p, 4, 3 * blk, 3 * row + 8, None) == _abi.KOMP_EINVAL and "SW" in _abi.last_error()
    assert f(ctypes.c_void_p(258), p, p, 4, 3 * blk, 3 * row, None) == _abi.KOMP_EINVAL and "aligned" in _abi.last_error()
    assert f(p, ctypes.c_void_p(264), p, 4, 3 * blk, 3 * row, None) == _abi.KOMP_EINVAL
    assert f(p, p, ctypes.c_void_p(257), 4, 3 * blk, 3 * row, None) == _abi.KOMP_EINVAL
    assert f(None, p, p, 4, 3 * blk, 3 * row, None) == _abi.KOMP_EINVAL
    assert f(p, p, p, -1, 3 * blk, 3 * row, None) == _abi.KOMP_EINVAL
    assert f(None, None, None, 0, 3 * blk, 0, None) == 0 and f(None, None, None, 5, 0, 16, None) == 0


def test_gemm_rejects_bad_arguments():
    lib = _abi.lib()
    p = ctypes.c_void_p(256)
    assert lib.komp_q4_0_gemm(p, p, p, p, p, None, 4, 8, 100, 64, None) == _abi.KOMP_EINVAL
    assert lib.komp_tq2_0_gemm(p, p, p, p, p, None, 4, 8, 256, 48, None) == _abi.KOMP_EINVAL and "SW" in _abi.last_error()
    assert lib.komp_q4_0_gemm(p, p, p, p, p, None, 4, 8, 1 << 26, 1 << 25, None) == _abi.KOMP_EINVAL
    assert "limits" in _abi.last_error()
    assert lib.komp_q4_0_gemm(p, p, p, p, p, None, 0, 8, 64, 32, None) == 0
    rows, cols, waves = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.komp_gemm_plan(0, 16, 4096, 4096, 2048, ctypes.byref(rows), ctypes.byref(cols), ctypes.byref(waves)) == 0
    assert cols.value == 16 and waves.value == 8 and rows.value % 16 == 0
    for fmt in (2, 3):  # q8_0, iq4_nl
        assert lib.komp_gemm_plan(fmt, 16, 4096, 4096, 4096, None, None, None) == 0
    for fmt in (-1, 5):
        assert lib.komp_gemm_plan(fmt, 16, 4096, 4096, 2048, None, None, None) == _abi.KOMP_EINVAL


def test_stamps_begin_rejects_bad_buffers():
    lib = _abi.lib()
    assert lib.komp_stamps_begin(ctypes.c_void_p(8), 64) == _abi.KOMP_EINVAL and "16-byte" in _abi.last_error()
    assert lib.komp_stamps_begin(None, 64) == _abi.KOMP_EINVAL
    assert lib.komp_stamps_begin(ctypes.c_void_p(16), -1) == _abi.KOMP_EINVAL
    used = ctypes.c_int64(-1)
    assert lib.komp_stamps_end(ctypes.byref(used), None) == _abi.KOMP_OK and used.value == 0


def test_parse_stamps_walks_records_across_a_counter_wrap():
    import numpy as np

    # two launches: 2 waves (counter wrapping past 2^32 inside the launch), then 3 waves; 100 MHz = 10 ns a tick
    a = [_abi.STAMP_MAGIC, 2, 6912, 2560, 0xFFFFFFF0, 0xFFFFFFF8, 2, 20, 0xFFFFFFF4, 0, 5, 30]
    b = [_abi.STAMP_MAGIC, 3, 2560, 6912] + [100, 110, 120, 130] * 2 + [90, 111, 121, 200]
    words = np.array(a + b, dtype=np.uint64).astype(np.uint32)
    recs = _abi.parse_stamps(words, 100_000)
    assert [(r["n"], r["k"], r["waves"]) for r in recs] == [(6912, 2560, 2), (2560, 6912, 3)]
    assert list(recs[0]["entry"]) == [0, 40] and list(recs[0]["stored"]) == [360, 460] and recs[0]["span_ns"] == 460
    assert list(recs[1]["entry"]) == [100, 100, 0] and recs[1]["span_ns"] == 1100
    with pytest.raises(_abi.KompError, match="header"):
        _abi.parse_stamps(np.array([1, 2, 3, 4], dtype=np.uint32), 100_000)


def test_clock_rejects_bad_pointers():
    lib = _abi.lib()
    assert lib.komp_clock(None, None) == _abi.KOMP_EINVAL and "8-byte" in _abi.last_error()
    assert lib.komp_clock(ctypes.c_void_p(12), None) == _abi.KOMP_EINVAL
    assert lib.komp_clock_khz(None) == _abi.KOMP_EINVAL
