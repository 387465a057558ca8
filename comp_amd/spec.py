"""KURN-style GEMV specs driving the gfx950 decode kernels (the reference's `target triton` specs, src/komp/spec.py).

    kernel     q4_0_gemv_triton
    op         gemv
    weights    q4_0           # q4_0 | tq2_0
    target     triton         # triton (KURN's routing key for COMP) | hip
    arch       gfx950
    mode       dp4a           # dp4a: packed-word dot products on v_dot4c_i32_i8 | bytes
    block_n    64             # rows per workgroup
    nb         4              # 16-byte weight chunks per lane per K step
    num_warps  4              # wavefronts per workgroup
    tune       mode=dp4a,bytes block_n=32,64 nb=4,8

Problem keys (n, k, m) give the shape `verify` runs on.  KURN's own parser (kurn.spec.parse / parse_overrides /
SpecError) is not available, so this module carries a parser for the same grammar: one `key value` per line, `#`
comments, integer values as ints, and a `tune` line of `key=v1,v2` lists.  Keys, defaults, legality and the tune-space
expansion follow src/komp/spec.py:22-79; `arch` takes gfx950.  The reference's own specs name NVIDIA targets (`arch
sm_80`, examples/q4_0_gemv_triton.kurn:6): `check` and `verify` accept an sm_* value as the spec's foreign target and
run the gfx950 kernels (resolve keeps it as `arch_requested`); `gen`, which writes code objects for the spec's arch,
refuses it.
"""

from __future__ import annotations

import itertools


class SpecError(ValueError):
    """An illegal or malformed spec (kurn.spec.SpecError's role)."""


KEYS = {
    "op": ("gemv",),
    "weights": ("q4_0", "tq2_0"),
    "arch": ("gfx950",),
    "mode": ("dp4a", "bytes"),
    "block_n": (8, 16, 32, 64, 128),
    "nb": (1, 2, 4, 8, 16),
    "num_warps": (1, 2, 4, 8),
}
DEFAULTS = {"arch": "gfx950", "mode": "dp4a", "block_n": 64, "num_warps": 4}
FORMAT_DEFAULTS = {"q4_0": {"nb": 4}, "tq2_0": {"nb": 1}}
BLOCK = {"q4_0": 32, "tq2_0": 256}
PROBLEM = {"q4_0": {"n": 64, "k": 512, "m": 1}, "tq2_0": {"n": 64, "k": 1024, "m": 1}}
COMMON = ("kernel", "target")
TARGETS = ("triton", "hip")
MODE = {"bytes": 0, "dp4a": 2}  # 1 = dp4a emulated with shifts and multiplies


def _value(text):
    t = text.strip()
    try:
        return int(t)
    except ValueError:
        return t


def parse(text):
    """Spec text -> (base dict, tune dict of lists)."""
    base, tune = {}, {}
    for lineno, raw in enumerate(text.splitlines(), 1):
        line = raw.split("#", 1)[0].strip()
        if not line:
            continue
        key, _, rest = line.partition(" ")
        rest = rest.strip()
        if key == "tune":
            for item in rest.split():
                if "=" not in item:
                    raise SpecError(f"line {lineno}: tune entries are key=v1,v2 (got {item!r})")
                k, v = item.split("=", 1)
                tune[k] = [_value(x) for x in v.split(",") if x]
            continue
        if not rest:
            raise SpecError(f"line {lineno}: key {key!r} has no value")
        if " " in rest:
            raise SpecError(f"line {lineno}: one value per key (got {rest!r})")
        if key in base:
            raise SpecError(f"line {lineno}: duplicate key {key!r}")
        base[key] = _value(rest)
    return base, tune


def parse_overrides(args):
    """['k=v', 'k=v1,v2', ...] -> (single values, lists): a comma makes the key a tune list."""
    single, lists = {}, {}
    for a in args:
        if "=" not in a:
            raise SpecError(f"override {a!r} is not key=value")
        k, v = a.split("=", 1)
        if "," in v:
            lists[k] = [_value(x) for x in v.split(",") if x]
        else:
            single[k] = _value(v)
    return single, lists


def resolve(spec, overrides=None):
    """Defaults filled in and legality checked (src/komp/spec.py:39-60); raises SpecError."""
    c = {**spec, **(overrides or {})}
    if c.get("target") not in TARGETS:
        raise SpecError(f"target {c.get('target')!r}: komp handles target triton (and hip)")
    for k in ("op", "weights"):
        if k not in c:
            raise SpecError(f"missing required key {k!r}")
    if c["weights"] not in KEYS["weights"]:
        raise SpecError(f"weights={c['weights']!r} not allowed for target {c['target']}: expected one of "
                        f"{list(KEYS['weights'])}")  # fmt: skip
    for k in c:
        if k not in KEYS and k not in COMMON and k not in ("n", "k", "m"):
            raise SpecError(f"unknown key {k!r} for target {c['target']}: expected one of "
                            f"{sorted((*KEYS, *COMMON, 'n', 'k', 'm'))}")  # fmt: skip
    arch = c.get("arch")
    if isinstance(arch, str) and arch.startswith("sm_") and arch[3:].isdigit():  # the reference's NVIDIA targets
        c["arch_requested"] = arch
        c["arch"] = "gfx950"
    for k, allowed in KEYS.items():
        c.setdefault(k, FORMAT_DEFAULTS[c["weights"]].get(k, DEFAULTS.get(k)))
        if c[k] not in allowed:
            raise SpecError(f"{k}={c[k]!r} not allowed for target {c['target']}: expected one of {list(allowed)}")
    for k, v in PROBLEM[c["weights"]].items():
        c.setdefault(k, v)
    for k in ("n", "k", "m"):
        if not isinstance(c[k], int) or c[k] < 1:
            raise SpecError(f"{k}={c[k]!r} must be a positive integer")
    if c["k"] % BLOCK[c["weights"]]:
        raise SpecError(f"k must be a multiple of {BLOCK[c['weights']]} ({c['weights']} block)")
    c.setdefault("kernel", f"{c['weights']}_{c['op']}_{c['target']}")
    return c


def load(path):
    with open(path) as fh:
        return parse(fh.read())


def configs(spec, tune):
    """Every legal config of the spec's tune space (the spec itself if there is none); illegal combinations are
    skipped (src/komp/spec.py:68-75)."""
    names = list(tune)
    for combo in itertools.product(*(tune[k] for k in names)) if names else [()]:
        try:
            yield resolve(spec, dict(zip(names, combo)))
        except SpecError:
            continue


def label(c):
    return f"mode={c['mode']} block_n={c['block_n']} nb={c['nb']} num_warps={c['num_warps']}"
