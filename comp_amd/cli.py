"""komp command line on the gfx950 build (src/komp/cli.py).

    python -m comp_amd check  SPEC [k=v ...]   validate a spec (and its tune space)
    python -m comp_amd verify SPEC [k=v ...]   every config of the spec on the GPU vs KURN's exact references
    python -m comp_amd verify --all            the full verification set (dp4a, decode, both GEMVs, every mode)

`gen`, `mix` and `fork` of the reference compile or inspect NVIDIA PTX/SASS and report the Triton fork; they have no
counterpart on this build and exit 2.  `kurn check|verify SPEC` reaches this module through spec_command
(comp_amd.kurn_ext registers it as KURN's backend for specs with `target triton`).
"""

from __future__ import annotations

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
    print(f"ok {c['kernel']}: {c['weights']} {c['op']} target {c['target']} {c['arch']} {spec.label(c)}; tune space: "
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


def _unavailable(name):
    def cmd(_args):
        print(f"komp {name}: not available on the gfx950 build (it compiles or inspects NVIDIA PTX/SASS or reports the "
              f"Triton fork)", file=sys.stderr)  # fmt: skip
        return 2

    return cmd


COMMANDS = {"check": cmd_check, "verify": cmd_verify, "gen": _unavailable("gen"), "mix": _unavailable("mix"),
            "fork": _unavailable("fork")}  # fmt: skip


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] not in COMMANDS:
        print(USAGE)
        return 0 if argv and argv[0] in ("-h", "--help") else 2
    return COMMANDS[argv[0]](argv[1:])


def spec_command(cmd, argv):
    """Entry for kurn.hooks.TARGET_BACKENDS["triton"] (src/komp/cli.py:195-200)."""
    if cmd not in ("check", "verify"):
        print(f"kurn {cmd}: not available for target triton on the gfx950 build (komp supports check, verify)",
              file=sys.stderr)  # fmt: skip
        return 2
    return main([cmd, *argv])
