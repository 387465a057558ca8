"""The wave stamps of the tuning harness (komp_stamps_begin / komp_stamps_end): the stamped instantiation computes
what the plain kernel does, bit for bit, and writes one well-formed record per launch; launches it does not cover, and
launches past the buffer's room, run unstamped."""

import numpy as np
import pytest
import torch

from comp_amd import _abi, host
from oracle import oracle as O
from tests.checks import outputs_ok

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _problem(n, k, m, seed):
    W, x = O.problem("tq2_0", n, k, m, seed)
    wq, ws = host.split("tq2_0", W, n, k)
    return wq, ws, x


@pytest.mark.parametrize("n,k,m,fused", [(6912, 2560, 1, True), (2560, 6912, 1, True), (6912, 2560, 3, True),
                                         (6912, 2560, 2, False), (300, 1280, 1, False)])  # fmt: skip
def test_stamped_launch_equals_plain_and_records(n, k, m, fused):
    wq, ws, x = _problem(n, k, m, 41)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    plan = host.auto_plan("tq2_0", m, n, k, fused=fused)
    print(f"stamps tq2_0 {n}x{k} m={m} fused={fused} plan={plan}", flush=True)

    def run():
        if fused:
            y, s = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k, store_s=True)
        else:
            xq, xd, *_ = host.quantize("tq2_0", x_d)
            y, s = host.gemv("tq2_0", wq_d, ws_d, xq, xd, n, k, None, None, 2, None, store_s=True)
        return y, s

    y0, s0 = run()
    buf = torch.zeros(1 << 20, dtype=torch.int32, device="cuda")
    _abi.stamps_begin(buf)
    try:
        y1, s1 = run()
    finally:
        used, khz = _abi.stamps_end()
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(s0, s1)
    groups = -(-n // plan["block_n"])
    waves = groups * plan["waves"]
    assert used == (4 + 4 * waves + 3) // 4 * 4 and khz > 0
    recs = _abi.parse_stamps(buf[:used].cpu().numpy().view(np.uint32), khz)
    assert len(recs) == 1 and (recs[0]["n"], recs[0]["k"], recs[0]["waves"]) == (n, k, waves)
    r = recs[0]
    assert np.all(r["entry"] <= r["staged"]) and np.all(r["staged"] <= r["dots"]) and np.all(r["dots"] <= r["stored"])
    assert r["entry"].min() == 0 and 0 < r["span_ns"] < 1e6  # a launch of these sizes takes microseconds
    rq, rd, _ = O.quantize("tq2_0", x)
    ref, rs = O.gemv("tq2_0", wq, ws, rq, rd, n, k)
    assert np.array_equal(s1.cpu().numpy().astype(np.int64), rs) and outputs_ok("tq2_0", y1.cpu().numpy(), ws, rd, rs, ref)


def test_uncovered_and_overflowing_launches_run_unstamped():
    n, k, m = 2560, 6912, 1
    wq, ws, x = _problem(n, k, m, 43)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    y_ref, _ = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k)
    buf = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    _abi.stamps_begin(buf)
    try:
        y_bytes, _ = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k, mode=0)  # bytes mode: no stamped instantiation
    finally:
        used, _ = _abi.stamps_end()
    assert used == 0
    small = torch.zeros(64, dtype=torch.int32, device="cuda")  # no room for one launch's records
    _abi.stamps_begin(small)
    try:
        y_small, _ = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k)
    finally:
        used, _ = _abi.stamps_end()
    torch.cuda.synchronize()
    assert used == 0 and torch.equal(y_small, y_ref) and torch.equal(y_bytes, y_ref)
    assert int(small.abs().sum()) == 0


def test_clock_marks_order_work_in_a_graph():
    """komp_clock marks around the stream's work read increasing counter values, eager and inside a HIP graph, at a
    rate the device reports (the benchmark's headline timing rests on them)."""
    n, k = 6912, 2560
    wq, ws, x = _problem(n, k, 1, 47)
    wq_d, ws_d, x_d = dev(wq), dev(ws), dev(x)
    y = torch.empty((1, n), dtype=torch.float32, device="cuda")
    marks = torch.zeros(3, dtype=torch.int64, device="cuda")
    khz = _abi.clock_khz()
    assert 1_000 <= khz <= 10_000_000
    _abi.clock_into(marks[0:1])
    host.gemv_f32_into("tq2_0", wq_d, ws_d, x_d, y, n, k)
    _abi.clock_into(marks[1:2])
    torch.cuda.synchronize()
    t = marks.cpu().tolist()
    assert t[1] > t[0] and (t[1] - t[0]) / khz < 100.0  # ms
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _abi.clock_into(marks[0:1])
        for _ in range(4):
            host.gemv_f32_into("tq2_0", wq_d, ws_d, x_d, y, n, k)
        _abi.clock_into(marks[1:2])
    for _ in range(3):
        marks.zero_()
        g.replay()
        torch.cuda.synchronize()
        t = marks.cpu().tolist()
        assert t[1] > t[0] > 0 and t[2] == 0
    y_ref, _ = host.gemv_f32("tq2_0", wq_d, ws_d, x_d, n, k)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
