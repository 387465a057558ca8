"""komp command line on the gfx950 build (src/komp/cli.py).

    python -m comp_amd check  SPEC [k=v ...]   validate a spec (and its tune space)
    python -m comp_amd verify SPEC [k=v ...]   every config of the spec on the GPU vs KURN's exact references
    python -m comp_amd verify --all            the full verification set (dp4a, decode, both GEMVs, every mode)

    python -m comp_amd gen    SPEC [k=v ...] [-o DIR] [--emit hsaco,s]
                                               the spec's GEMV and quantizer as built for gfx950: registers,
                                               spills, approximate math, v_dot4c_i32_i8 in the hot loop, its
                                               instruction mix; -o writes the code object and the kernel's ISA
    python -m comp_amd mix    [--archs gfx950]  hot-loop instruction mixes of the GEMV configs (and the matrix-core
                                               GEMM plans) of this build
    python -m comp_amd counters CSV... --cases CASES
                                               per-weight instruction mix of the launches of a rocprofv3 --pmc run
                                               of `bench.py --counter-calls N` (comp_amd.counters)

`gen` and `mix` read the gfx950 code objects inside this build's own library (comp_amd.isa), where the reference
compiles Triton to PTX/SASS and reads those (src/komp/cli.py:88-158).  `fork` (the Triton fork) has no counterpart and
exits 2.  `kurn check|gen|verify SPEC` reaches this module through spec_command (comp_amd.kurn_ext registers it as
KURN's backend for specs with `target triton`).
"""

from __future__ import annotations

import os
import sys

USAGE = __doc__


def _spec(args):
    from . import spec

    path = next((a for a in args if not a.startswith("-") and "=" not in a), None)
    if path is None:
        raise spec.SpecError("no spec file given")
    base, tune = spec.load(path)
    single, lists = spec.parse_overrides([a for a in args if "=" in a and not a.startswith("-")])
    base.update(single)
    tune.update(lists)
    return spec, base, tune


def cmd_check(args):
    from .spec import SpecError

    try:
        spec, base, tune = _spec(args)
        c = spec.resolve(base)
        n = len(list(spec.configs(base, tune)))
    except (SpecError, OSError) as e:
        print(f"komp check: {e}", file=sys.stderr)
        return 2
    arch = f"{c['arch_requested']} (run as {c['arch']})" if "arch_requested" in c else c["arch"]
    print(f"ok {c['kernel']}: {c['weights']} {c['op']} target {c['target']} {arch} {spec.label(c)}; tune space: "
          f"{n} legal configs")  # fmt: skip
    return 0


def cmd_verify(args):
    from . import verify
    from .spec import SpecError

    try:
        if "--all" in args:
            return 1 if verify.run_all() else 0
        spec, base, tune = _spec(args)
        spec.resolve(base)
        fails = 0
        ok = verify.check_dp4a()
        fails += not ok
        print(f"{'ok  ' if ok else 'FAIL'} dp4a v_dot4c_i32_i8 and emulated == dp4a.s32.s32 semantics")
        for c in spec.configs(base, tune):
            mode = spec.MODE[c["mode"]]
            for seed, extreme in ((1, False), (2, True)):
                res = verify.check_gemv(c["weights"], c["n"], c["k"], c["m"], seed, extreme, c["block_n"], c["nb"], mode,
                                        c["num_warps"])  # fmt: skip
                fails += not res["ok"]
                print(verify.line(res, c["block_n"], c["nb"], c["num_warps"], mode) + (" extreme" if extreme else "")
                      + f"  [{c['arch']}]")  # fmt: skip
        print(f"{fails} failures")
        return 1 if fails else 0
    except (SpecError, OSError, verify.ReferencesMissing) as e:
        print(f"komp verify: {e}", file=sys.stderr)
        return 2
    except RuntimeError as e:
        print(f"komp verify: {e}", file=sys.stderr)
        return 2


# GEMV configs listed by `mix` (block_n, nb, num_warps), the reference's set (src/komp/cli.py:136)
MIX_KOMP = {"q4_0": ((64, 4, 4), (32, 8, 4)), "tq2_0": ((64, 1, 4), (32, 2, 4))}
# the ggml formats beyond the reference's two, at the library's common plan shape
MIX_MORE = {"q8_0": ((64, 4, 4),), "iq4_nl": ((64, 4, 4),), "q4_k": ((64, 2, 4),)}
# weights per 16-byte load of the hot loop (q4_k: a slot's two weight loads come with one 16-byte scale-entry load)
VALUES_PER_LOAD = {"q4_0": 32, "tq2_0": 64, "q8_0": 16, "iq4_nl": 32, "q4_k": 64 / 3}
FMT_NUM = {"q4_0": 0, "tq2_0": 1, "q8_0": 2, "iq4_nl": 3, "q4_k": 4}  # the kernels' format template argument


def _gemv_kernel(fmt, mode, nb, m=1, block_n=None, num_warps=None, k=None, n=None):
    """The kernel instantiation a launch of this config runs, the knobs giving lanes per row = 64 / min(block_n /
    num_warps, 16): in dp4a mode, q4_0 / iq4_nl / tq2_0 with 1-3 columns (nb <= 4, or 8 for one column) run the lean
    kernel <(format,) lanes per row, nb, columns, fused, one pass(, tq2_0: staged through an LDS copy)> (q8_0:
    q8_lean_kernel, q4_k with nb <= 4: q4k_lean_kernel, both <lanes per row, nb, columns, fused, one pass>), and tq2_0 /
    q4_0 in bytes mode its bytes form (tq2_lean_bytes_kernel / q4_lean_bytes_kernel <lanes per row, nb, columns, fused,
    one pass>; tq2_0 when LDS holds the 16-bit activations); everything else the general gemv_kernel <format, mode,
    columns, nb, fused>.  "One pass" is
    the lean kernel's single-pass, single-K-step form, which the launch picks when the rows per wave fit one pass and a
    row's K blocks one step; without k the loop form is named.  The
    LDS-copy form stages two or three tq2_0 columns that need more than one pass of the workgroup's threads, when LDS
    holds them.  One column with nb < 8 whose waves walk 3 tiles or more (passes x K steps; k given) runs the
    pipelined loop form instead (q4_lean_pipe_kernel <format, lanes, nb, fused>, q4_lean_bytes_pipe_kernel <lanes, nb,
    fused>, tq2_lean_pipe_kernel <lanes, nb, fused, bytes>).  One or two tq2_0 dp4a columns in the single-pass form with
    nb x columns <= 4 (or two columns at nb 4 in workgroups of at most 8 waves), launched as at most one workgroup a CU
    (n given: ceil(n / block_n) <= 256, MI355X's CUs), run the form that reads its LDS pieces ahead of the dots
    (tq2_lean_pre_kernel <lanes, nb, columns, fused, copy staging>; one bytes-mode column at nb <= 4 likewise:
    tq2_lean_bytes_pre_kernel <lanes, nb, fused>).  A tq2_0 K step below 256 bytes a row
    (lanes x nb x 16) is widened to it (nb doubled up to 4), as the launch does."""
    cols = min(max(m, 1), 3)
    if fmt == "tq2_0" and block_n and num_warps:  # the launch widens a tq2_0 K step to 256 bytes a row
        while 64 // min(block_n // num_warps, 16) * nb < 16 and nb < 4:
            nb *= 2
    lean_mode = mode == 2 or (mode == 0 and fmt in ("tq2_0", "q4_0"))
    if lean_mode and block_n and num_warps and (nb in (1, 2, 4) or (nb == 8 and cols == 1)):
        rpw = block_n // num_warps
        lanes = 64 // min(rpw, 16)
        one_pass = rpw <= 16 and k is not None
        passes = rpw // min(rpw, 16)
        vals = 256 if fmt == "tq2_0" else 32
        step = (lanes // 4 if fmt == "tq2_0" else lanes) * nb  # blocks a K step covers
        pipe = k is not None and cols == 1 and nb < 8 and passes * -(-(k // vals) // step) >= 3
        if fmt == "tq2_0" and mode == 0:
            one = one_pass and k // 256 <= (lanes // 4) * nb
            bstep = (lanes // 4) * nb
            if k is None or cols * -(-(k // 256) // bstep) * bstep * (2 * 288 + 8) <= 160 * 1024:
                if pipe and not one:
                    return f"gemv_tq2::tq2_lean_pipe_kernel<{lanes}, {nb}, false, true>"
                if (one and cols == 1 and nb <= 4 and (nb <= 2 or num_warps <= 8) and n is not None
                        and -(-n // block_n) <= 256):
                    return f"gemv_tq2::tq2_lean_bytes_pre_kernel<{lanes}, {nb}, false>"
                return f"gemv_tq2::tq2_lean_bytes_kernel<{lanes}, {nb}, {cols}, false, {str(one).lower()}>"
        elif fmt == "tq2_0":
            one = one_pass and k // 256 <= (lanes // 4) * nb
            if pipe and not one:
                return f"gemv_tq2::tq2_lean_pipe_kernel<{lanes}, {nb}, false, false>"
            dma = False
            if k is not None and cols > 1 and cols * (k // 256) * 16 > 64 * num_warps:
                bstep = (lanes // 4) * nb
                staged = cols * -(-(k // 256) // bstep) * bstep * 296
                dma = (staged + 15) // 16 * 16 + cols * k + cols * (k // 256) * 4 <= 160 * 1024
            pre_form = nb * cols <= 4 or (cols == 2 and nb == 4 and num_warps <= 8)
            if one and cols <= 2 and pre_form and n is not None and -(-n // block_n) <= 256:
                return f"gemv_tq2::tq2_lean_pre_kernel<{lanes}, {nb}, {cols}, false, {str(dma).lower()}>"
            return (f"gemv_tq2::tq2_lean_kernel<{lanes}, {nb}, {cols}, false, {str(one).lower()}, "
                    f"{str(dma).lower()}>")
        elif fmt == "q8_0" and mode == 2:
            one = one_pass and k // 32 <= (lanes // 2) * nb
            return f"gemv_q8::q8_lean_kernel<{lanes}, {nb}, {cols}, false, {str(one).lower()}>"
        elif fmt == "q4_k" and mode == 2 and nb <= 4:
            one = one_pass and k // 256 <= (lanes // 4) * nb
            return f"gemv_q4k::q4k_lean_kernel<{lanes}, {nb}, {cols}, false, {str(one).lower()}>"
        elif fmt in ("q4_0", "iq4_nl"):
            one = one_pass and k // 32 <= lanes * nb
            if pipe and not one:
                if mode == 0:
                    return f"gemv_q4::q4_lean_bytes_pipe_kernel<{lanes}, {nb}, false>"
                return f"gemv_q4::q4_lean_pipe_kernel<{FMT_NUM[fmt]}, {lanes}, {nb}, false>"
            if mode == 0:
                return f"gemv_q4::q4_lean_bytes_kernel<{lanes}, {nb}, {cols}, false, {str(one).lower()}>"
            return f"gemv_q4::q4_lean_kernel<{FMT_NUM[fmt]}, {lanes}, {nb}, {cols}, false, {str(one).lower()}>"
    return f"gemv_impl::gemv_kernel<{FMT_NUM[fmt]}, {mode}, {min(max(m, 1), 3)}, {nb}, false>"


def _mix_line(r, name):
    lp = r["loop"]
    return (f"{name:34} hot loop {r['loop_len']:4} insts / {r['values_per_thread']:5.0f} weights per thread: "
            f"{r['insts_per_value']:.2f} insts, {r['int_per_value']:.2f} int, {r['dot4_per_value']:.3f} v_dot4c per "
            f"weight; loads 128-bit {lp.get('ld128', 0)}, 64-bit {lp.get('ld64', 0)}, 32-bit {lp.get('ld32', 0)}, "
            f"16-bit {lp.get('ld16', 0)}, 8-bit {lp.get('ld8', 0)}; LDS {lp.get('lds', 0)}")  # fmt: skip


def _regs(r):
    return (f"vgpr={r['vgpr']} agpr={r['agpr']} sgpr={r['sgpr']} lds={r['lds']} spill={r['vgpr_spill'] + r['sgpr_spill']} "
            f"scratch={r['scratch']} approx-ops={','.join(r['approx']) or 'none'}")  # fmt: skip


def cmd_gen(args):
    from . import isa
    from .spec import SpecError

    try:
        spec, base, tune = _spec(args)
        c = spec.resolve(base)
    except (SpecError, OSError) as e:
        print(f"komp gen: {e}", file=sys.stderr)
        return 2
    if c["arch"] != "gfx950" or "arch_requested" in c:
        print(f"komp gen: arch {c.get('arch_requested', c['arch'])}: this build holds gfx950 code only (set arch "
              f"gfx950, or arch=gfx950 on the command line)", file=sys.stderr)  # fmt: skip
        return 2
    out = args[args.index("-o") + 1] if "-o" in args else None
    emit = (args[args.index("--emit") + 1] if "--emit" in args else "hsaco,s").split(",")
    mode = spec.MODE[c["mode"]]
    fmt = c["weights"]
    quant = "quant_q8_0" if fmt == "q4_0" else "quant_q8_K"
    try:
        r = isa.summary(_gemv_kernel(fmt, mode, c["nb"], c.get("m", 1), c.get("block_n"), c.get("num_warps"),
                                     c.get("k"), c.get("n")), VALUES_PER_LOAD[fmt], keep=out is not None)  # fmt: skip
        q = isa.summary(f"{quant}_kernel", 1, keep=out is not None)
    except (OSError, RuntimeError, KeyError) as e:
        print(f"komp gen: {e}", file=sys.stderr)
        return 2
    fails = 0
    dots = r["loop"].get("dot4", 0)
    bad = r["vgpr_spill"] or r["sgpr_spill"] or r["approx"] or (mode == 2 and not dots)
    fails += bool(bad)
    print(f"{'FAIL' if bad else 'ok  '} {c['kernel']} {c['arch']} {spec.label(c)}: {_regs(r)} "
          f"v_dot4c_i32_i8={r['dot4_total']} in hot loop={dots}")  # fmt: skip
    print("     " + _mix_line(r, f"{fmt} {c['mode']}"))
    print(f"     kernel {r['kernel'].split('(')[0]} (block_n and num_warps are launch parameters on gfx950)")
    qbad = q["vgpr_spill"] or q["sgpr_spill"] or q["approx"]
    fails += bool(qbad)
    print(f"{'FAIL' if qbad else 'ok  '} {quant} {c['arch']}: {_regs(q)}")
    if out:
        os.makedirs(out, exist_ok=True)
        for name, res in ((c["kernel"], r), (quant, q)):
            for e in emit:
                path = os.path.join(out, f"{name}.{c['arch']}.{e}")
                if e == "hsaco":
                    with open(path, "wb") as fh:
                        fh.write(res["code_object"])
                elif e == "s":
                    with open(path, "w") as fh:
                        fh.write(f"; {res['kernel']}\n" + res["asm"])
                else:
                    print(f"komp gen: --emit {e}: one of hsaco, s", file=sys.stderr)
                    return 2
                print(f"     wrote {path}")
    return 1 if fails else 0


def cmd_mix(args):
    from . import isa

    archs = (args[args.index("--archs") + 1] if "--archs" in args else "gfx950").split(",")
    fails = 0
    for arch in archs:
        print(f"== {arch}")
        if arch != "gfx950":
            print(f"{arch}: not built (this build holds gfx950 code only)")
            continue
        for fmt in ("q4_0", "tq2_0"):
            for bn, nb, nw in MIX_KOMP[fmt]:
                for mode in (0, 2):
                    r = isa.summary(_gemv_kernel(fmt, mode, nb, 1, bn, nw), VALUES_PER_LOAD[fmt])
                    spill = r["vgpr_spill"] + r["sgpr_spill"]
                    fails += bool(spill or r["approx"])
                    name = (f"KOMP {fmt} {'dp4a ' if mode else 'bytes'} {bn}/{nb}/{nw}w v{r['vgpr']}"
                            + (" SPILL" if spill else ""))  # fmt: skip
                    print(_mix_line(r, name))
            print(f"KURN-CUDA {fmt}: not available (NVIDIA target; this build holds gfx950 code only)")
        for fmt, cfgs in MIX_MORE.items():
            for bn, nb, nw in cfgs:
                r = isa.summary(_gemv_kernel(fmt, 2, nb, 1, bn, nw), VALUES_PER_LOAD[fmt])
                spill = r["vgpr_spill"] + r["sgpr_spill"]
                fails += bool(spill or r["approx"])
                print(_mix_line(r, f"KOMP {fmt} dp4a  {bn}/{nb}/{nw}w v{r['vgpr']}" + (" SPILL" if spill else "")))
        for prefix, label in (("gemm_impl::gemm_kernel<0, 8, 1, 1, 1, 2, false>", "GEMM q4_0 16 rows x 16 cols"),
                              ("gemm_impl::gemm_kernel<0, 8, 1, 1, 4, 2, false>", "GEMM q4_0 16 rows x 64 cols"),
                              ("gemm_impl::gemm_kernel<1, 8, 1, 1, 1, 2, false>", "GEMM tq2_0 16 rows x 16 cols")):
            r = isa.summary(prefix, 1)
            lp = r["loop"]
            spill = r["vgpr_spill"] + r["sgpr_spill"]
            fails += bool(spill or r["approx"])
            print(f"{label:34} hot loop {r['loop_len']:4} insts: v_mfma {lp.get('mfma', 0)}, VALU {lp.get('valu', 0)}, "
                  f"loads 128-bit {lp.get('ld128', 0)}, 32-bit {lp.get('ld32', 0)}, LDS {lp.get('lds', 0)}; v{r['vgpr']}"
                  + (" SPILL" if spill else ""))  # fmt: skip
    return 1 if fails else 0


def cmd_counters(args):
    from . import counters

    if "--cases" not in args or args.index("--cases") + 1 >= len(args):
        print("komp counters: CSV... --cases CASES (the counter run's counter_calls JSON or a file holding it)",
              file=sys.stderr)  # fmt: skip
        return 2
    i = args.index("--cases")
    paths = [a for a in args[:i] + args[i + 2 :] if not a.startswith("--")]
    try:
        rows = counters.table(counters.merge([counters.read_pass(p) for p in paths]), counters.load_cases(args[i + 1]))
    except (OSError, ValueError, KeyError) as e:
        print(f"komp counters: {e}", file=sys.stderr)
        return 2
    print(counters.markdown(rows))
    return 0


def _unavailable(name):
    def cmd(_args):
        print(f"komp {name}: not available on the gfx950 build (it reports the Triton fork)", file=sys.stderr)
        return 2

    return cmd


COMMANDS = {"check": cmd_check, "verify": cmd_verify, "gen": cmd_gen, "mix": cmd_mix, "counters": cmd_counters,
            "fork": _unavailable("fork")}


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] not in COMMANDS:
        print(USAGE)
        return 0 if argv and argv[0] in ("-h", "--help") else 2
    return COMMANDS[argv[0]](argv[1:])


def spec_command(cmd, argv):
    """Entry for kurn.hooks.TARGET_BACKENDS["triton"] (src/komp/cli.py:195-200)."""
    if cmd not in ("check", "gen", "verify"):
        print(f"kurn {cmd}: not available for target triton on the gfx950 build (komp supports check, gen, verify)",
              file=sys.stderr)  # fmt: skip
        return 2
    return main([cmd, *argv])
