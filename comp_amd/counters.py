"""Per-weight instruction mix of GEMV launches from rocprofv3 hardware-counter passes: the counter half of the tuning
harness (`komp gen` and `komp mix` give the static mix of the code, this the instructions the launches issued).

    rocprofv3 --pmc SQ_WAVES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_VMEM_RD SQ_INSTS_LDS ... \\
        -d OUT -o p --output-format csv -- python bench.py --counter-calls 20
    python -m komp counters OUT/p_counter_collection.csv [more passes ...] --cases CASES

CASES is the JSON the counter run prints (its "counter_calls" list: fmt, n, k, m, launch, calls per case, in launch
order) or a file holding it.  The GEMV and GEMM dispatches of every pass are taken in dispatch order, `calls` per case
(the quantizer dispatches of the q8 launches are skipped), the passes zipped dispatch by dispatch, and each counter
averaged over a case's dispatches.  Per weight = instructions x 64 lanes / (N x K): the whole kernel's instructions,
staging, reductions and stores included.  `dot4` is the exact integer work the format defines: 0.25 v_dot4 per weight
and column (4 products an instruction), the floor of the dp4a path; the VALU figure includes it.  A case may name its
mode ("dp4a", the default, or "bytes": no dot instruction, so 0 there); the matrix-core kernels (GEMM, the
three-column TQ2_0 GEMV) issue none either.
"""

from __future__ import annotations

import csv
import json
import os

# kernel families that make one GEMV / GEMM call (the quantizer and the copies of the weight rotation are not counted)
FAMILIES = ("tq2_lean_kernel", "tq2_lean_pre_kernel", "tq2_lean_bytes_kernel", "tq2_lean_bytes_pre_kernel",
            "q4_lean_kernel", "q4_lean_bytes_kernel",
            "q8_lean_kernel", "q4k_lean_kernel", "tq2_mfma_kernel", "gemv_kernel", "gemm_kernel")


def _family(name):
    return next((f for f in FAMILIES if f + "<" in name), None)


def read_pass(path):
    """One counter pass: the GEMV / GEMM dispatches in dispatch order, each {kernel, grid, wg, counters}."""
    by_id = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            name = r["Kernel_Name"]
            fam = _family(name)
            if fam is None or "komp" not in name:
                continue
            d = by_id.setdefault(int(r["Dispatch_Id"]), {"kernel": name[name.index(fam):].split("(")[0],
                                                         "grid": int(r.get("Grid_Size") or r["Grid_Size_X"]),
                                                         "wg": int(r.get("Workgroup_Size") or r["Workgroup_Size_X"]),
                                                         "counters": {}})  # fmt: skip
            d["counters"][r["Counter_Name"]] = d["counters"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [by_id[i] for i in sorted(by_id)]


def merge(passes):
    """Zip several passes of the same launch sequence dispatch by dispatch (their counters joined)."""
    if len({len(p) for p in passes}) > 1:
        raise ValueError(f"the passes hold different numbers of GEMV dispatches: {[len(p) for p in passes]}")
    out = []
    for ds in zip(*passes):
        if len({(d["kernel"], d["grid"]) for d in ds}) > 1:
            raise ValueError(f"the passes launched different kernels at one dispatch: {[d['kernel'] for d in ds]}")
        c = {}
        for d in ds:
            c.update(d["counters"])
        out.append({**ds[0], "counters": c})
    return out


def table(dispatches, cases):
    """Rows of the per-weight table, one per case: the case's `calls` dispatches in order, counters averaged."""
    rows, i = [], 0
    for case in cases:
        ds = dispatches[i : i + case["calls"]]
        i += case["calls"]
        if len(ds) < case["calls"]:
            raise ValueError(f"case {case} has {len(ds)} of its {case['calls']} dispatches")
        keys = sorted({k for d in ds for k in d["counters"]})
        avg = {k: sum(d["counters"].get(k, 0.0) for d in ds) / len(ds) for k in keys}
        weights = case["n"] * case["k"]
        mode = case.get("mode", "dp4a")
        # the matrix-core kernels (GEMM, three-column TQ2_0 GEMV) do their integer dots on MFMA, not v_dot4
        dots = case["launch"] != "gemm" and mode != "bytes" and "mfma_kernel" not in ds[0]["kernel"]
        row = {"fmt": case["fmt"], "n": case["n"], "k": case["k"], "m": case["m"], "launch": case["launch"],
               "mode": mode, "kernel": ds[0]["kernel"], "grid": ds[0]["grid"], "wg": ds[0]["wg"],
               "dispatches": len(ds), "dot4_per_weight": 0.25 * case["m"] if dots else 0.0}  # fmt: skip
        waves = avg.get("SQ_WAVES")
        for name, key in (("valu", "SQ_INSTS_VALU"), ("salu", "SQ_INSTS_SALU"), ("vmem", "SQ_INSTS_VMEM_RD"),
                          ("lds", "SQ_INSTS_LDS"), ("mfma", "SQ_INSTS_MFMA")):  # fmt: skip
            if key in avg:
                row[name] = avg[key]
                row[name + "_per_weight"] = avg[key] * 64 / weights
                if waves:
                    row[name + "_per_wave"] = avg[key] / waves
        if waves:
            row["waves"] = waves
        if avg.get("SQ_ACTIVE_INST_ANY"):
            row["valu_active"] = avg.get("SQ_ACTIVE_INST_VALU", 0.0) / avg["SQ_ACTIVE_INST_ANY"]
        if avg.get("SQ_WAVE_CYCLES") and "SQ_WAIT_ANY" in avg:
            row["waiting"] = avg["SQ_WAIT_ANY"] / avg["SQ_WAVE_CYCLES"]
        rows.append(row)
    if i != len(dispatches):
        raise ValueError(f"{len(dispatches) - i} GEMV dispatches past the cases")
    return rows


def markdown(rows):
    head = ("| launch | kernel | waves | VALU / wave | VALU / weight | dot4 / weight | SALU / weight | VMEM / weight | "
            "LDS / weight | VALU active | waiting |")  # fmt: skip
    out = [head, "|" + "---|" * 11]

    def f(r, k, fmt="{:.2f}"):
        return fmt.format(r[k]) if k in r else "-"

    for r in rows:
        label = f"{r['fmt']} {r['n']}x{r['k']}, m={r['m']}, {r['launch']}" + (", bytes" if r["mode"] == "bytes" else "")
        out.append(f"| {label} | `{r['kernel']}` | {f(r, 'waves', '{:.0f}')} | {f(r, 'valu_per_wave', '{:.1f}')} | "
                   f"{f(r, 'valu_per_weight')} | {r['dot4_per_weight']:.2f} | {f(r, 'salu_per_weight')} | "
                   f"{f(r, 'vmem_per_weight', '{:.3f}')} | {f(r, 'lds_per_weight', '{:.3f}')} | "
                   f"{f(r, 'valu_active', '{:.0%}')} | {f(r, 'waiting', '{:.0%}')} |")  # fmt: skip
    return "\n".join(out)


def load_cases(arg):
    """The counter run's case list: a JSON text or a file holding it (the counter run's output, other lines such as
    the profiler's log around it), either the bare list or the printed object."""
    text = open(arg).read() if os.path.exists(arg) else arg
    for line in text.splitlines():
        if line.startswith('{"counter_calls"'):
            return json.loads(line)["counter_calls"]
    obj = json.loads(text)
    return obj["counter_calls"] if isinstance(obj, dict) else obj
