"""The counter half of the tuning harness (comp_amd.counters, `komp counters`): two synthetic rocprofv3 counter passes
of a two-case launch sequence, merged and reduced to the per-weight table."""

import csv
import json

from comp_amd import cli, counters

CASES = [{"fmt": "tq2_0", "n": 256, "k": 2560, "m": 1, "launch": "fused", "calls": 2},
         {"fmt": "q4_0", "n": 128, "k": 4096, "m": 3, "launch": "gemv", "calls": 1}]  # fmt: skip
KERNELS = [("void komp::gemv_tq2::tq2_lean_kernel<16, 4, 1, true, true, false>(int, int)", 16384, 448),
           ("void komp::gemv_tq2::tq2_lean_kernel<16, 4, 1, true, true, false>(int, int)", 16384, 448),
           ("void komp::(anonymous namespace)::quant_q8_0_kernel(float const*)", 1024, 256),
           ("void komp::gemv_q4::q4_lean_kernel<0, 64, 4, 3, false, false>(int, int)", 8192, 512)]  # fmt: skip


def write_pass(path, counters_of):
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name", "Counter_Value"])
        w.writerow([1, "at::native::elementwise_kernel", 4096, 256, "SQ_WAVES", 64])  # not a GEMV: skipped
        for i, (name, grid, wg) in enumerate(KERNELS):
            for cname, value in counters_of(i).items():
                w.writerow([i + 2, name, grid, wg, cname, value])


def test_two_passes_give_the_per_weight_table(tmp_path):
    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    write_pass(a, lambda i: {"SQ_WAVES": 100 + i, "SQ_INSTS_VALU": 1000 * (i + 1), "SQ_INSTS_SALU": 10})
    write_pass(b, lambda i: {"SQ_ACTIVE_INST_VALU": 30, "SQ_ACTIVE_INST_ANY": 60, "SQ_WAIT_ANY": 5,
                             "SQ_WAVE_CYCLES": 20})  # fmt: skip
    rows = counters.table(counters.merge([counters.read_pass(a), counters.read_pass(b)]), CASES)
    assert [r["kernel"] for r in rows] == ["tq2_lean_kernel<16, 4, 1, true, true, false>",
                                           "q4_lean_kernel<0, 64, 4, 3, false, false>"]  # fmt: skip
    t, q = rows
    assert t["dispatches"] == 2 and t["waves"] == 100.5 and t["valu"] == 1500.0
    assert t["valu_per_weight"] == 1500.0 * 64 / (256 * 2560) and t["valu_per_wave"] == 1500.0 / 100.5
    assert t["valu_active"] == 0.5 and t["waiting"] == 0.25 and t["dot4_per_weight"] == 0.25
    assert q["dispatches"] == 1 and q["valu"] == 4000.0 and q["dot4_per_weight"] == 0.75  # the quantizer skipped
    assert q["salu_per_weight"] == 10 * 64 / (128 * 4096)


def test_mismatched_passes_and_cases_are_errors(tmp_path):
    a = tmp_path / "a.csv"
    write_pass(a, lambda i: {"SQ_WAVES": 1})
    d = counters.read_pass(a)
    try:
        counters.table(d, CASES[:1])
    except ValueError as e:
        assert "past the cases" in str(e)
    else:
        raise AssertionError("extra dispatches were not reported")
    try:
        counters.merge([d, d[:2]])
    except ValueError as e:
        assert "different numbers" in str(e)
    else:
        raise AssertionError("passes of different lengths were merged")


def test_cli_prints_the_table(tmp_path, capsys):
    a = tmp_path / "a.csv"
    write_pass(a, lambda i: {"SQ_WAVES": 100, "SQ_INSTS_VALU": 640})
    cases = tmp_path / "cases.json"
    cases.write_text(json.dumps({"counter_calls": CASES}))
    assert cli.main(["counters", str(a), "--cases", str(cases)]) == 0
    out = capsys.readouterr().out
    assert "tq2_0 256x2560, m=1, fused" in out and "| 6.4 |" in out
    assert cli.main(["counters", str(a)]) == 2


def test_bytes_mode_case_names_its_kernel_and_has_no_dot4(tmp_path):
    a = tmp_path / "a.csv"
    name = "void komp::gemv_tq2::tq2_lean_bytes_kernel<16, 4, 1, true, true>(int, int)"
    with open(a, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name", "Counter_Value"])
        w.writerow([1, name, 16384, 448, "SQ_INSTS_VALU", 3200])
    case = {"fmt": "tq2_0", "n": 256, "k": 2560, "m": 1, "launch": "fused", "mode": "bytes", "calls": 1}
    (r,) = counters.table(counters.read_pass(a), [case])
    assert r["kernel"] == "tq2_lean_bytes_kernel<16, 4, 1, true, true>" and r["dot4_per_weight"] == 0.0
    assert "m=1, fused, bytes" in counters.markdown([r])
