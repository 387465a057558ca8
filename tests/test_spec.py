"""Spec parsing, legality and tune-space expansion (src/komp/spec.py; tests/test_komp.py:43-45, 62-66), CLI check."""

import os
import subprocess
import sys

import pytest

from comp_amd import cli, kurn_ext, spec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EX = os.path.join(ROOT, "comp_amd", "examples")
SPEC_Q4 = os.path.join(EX, "q4_0_gemv.kurn")
SPEC_TQ = os.path.join(EX, "tq2_0_gemv.kurn")


def run(*args):
    return subprocess.run([sys.executable, "-m", "comp_amd", *args], capture_output=True, text=True, cwd=ROOT, timeout=120)


def test_parse_example():
    base, tune = spec.load(SPEC_Q4)
    assert base["weights"] == "q4_0" and base["block_n"] == 64 and base["n"] == 37 and base["k"] == 416
    assert tune == {"mode": ["dp4a", "bytes"], "block_n": [32, 64], "nb": [4, 8]}


def test_tune_space_sizes():
    for path in (SPEC_Q4, SPEC_TQ):
        base, tune = spec.load(path)
        cs = list(spec.configs(base, tune))
        assert len(cs) == 8
        assert {c["mode"] for c in cs} == {"dp4a", "bytes"}


def test_defaults_and_format_defaults():
    c = spec.resolve({"op": "gemv", "weights": "tq2_0", "target": "triton"})
    assert (c["mode"], c["block_n"], c["nb"], c["num_warps"], c["arch"]) == ("dp4a", 64, 1, 4, "gfx950")
    assert (c["n"], c["k"], c["m"]) == (64, 1024, 1) and c["kernel"] == "tq2_0_gemv_triton"
    c = spec.resolve({"op": "gemv", "weights": "q4_0", "target": "hip"})
    assert c["nb"] == 4 and c["k"] == 512


@pytest.mark.parametrize("bad,needle", [({"block_n": 33}, "block_n"), ({"nb": 3}, "nb"), ({"num_warps": 16}, "num_warps"),
                                        ({"mode": "wmma"}, "mode"), ({"arch": "gfx942"}, "arch"), ({"k": 100}, "multiple"),
                                        ({"target": "cuda"}, "target"), ({"weights": "q8_0"}, "weights"),
                                        ({"colour": 1}, "unknown key"), ({"m": 0}, "m=")])  # fmt: skip
def test_illegal_specs(bad, needle):
    base, _ = spec.load(SPEC_Q4)
    with pytest.raises(spec.SpecError, match=needle):
        spec.resolve(base, bad)


def test_illegal_tune_combos_are_skipped():
    base, _ = spec.load(SPEC_Q4)
    cs = list(spec.configs(base, {"block_n": [33, 64], "nb": [3, 4]}))
    assert [(c["block_n"], c["nb"]) for c in cs] == [(64, 4)]


def test_overrides():
    single, lists = spec.parse_overrides(["block_n=32", "nb=4,8", "mode=bytes"])
    assert single == {"block_n": 32, "mode": "bytes"} and lists == {"nb": [4, 8]}


def test_parse_errors():
    with pytest.raises(spec.SpecError):
        spec.parse("weights\n")
    with pytest.raises(spec.SpecError):
        spec.parse("tune block_n\n")
    with pytest.raises(spec.SpecError):
        spec.parse("nb 4\nnb 8\n")


def test_cli_check_ok():
    r = run("check", SPEC_TQ)
    assert r.returncode == 0 and "target triton" in r.stdout and "8 legal configs" in r.stdout, r.stderr


def test_cli_bad_spec_rejected(tmp_path):
    p = tmp_path / "bad.kurn"
    p.write_text(open(SPEC_Q4).read().replace("block_n    64", "block_n    33"))
    r = run("check", str(p))
    assert r.returncode == 2 and "block_n" in r.stderr


def test_cli_override_and_fork():
    assert run("check", SPEC_Q4, "nb=16").returncode == 0
    r = run("fork", SPEC_Q4)
    assert r.returncode == 2 and "not available" in r.stderr
    assert run().returncode == 2 and run("--help").returncode == 0


def test_spec_command_and_kurn_registration(capsys):
    class Hooks:
        TARGET_BACKENDS = {}

    kurn_ext.register(Hooks)
    assert Hooks.TARGET_BACKENDS["triton"]("check", [SPEC_Q4]) == 0
    assert "q4_0_gemv_triton" in capsys.readouterr().out
    assert cli.spec_command("gen", [SPEC_Q4]) == 0
    assert cli.spec_command("mix", [SPEC_Q4]) == 2


def test_reference_sm_arch_runs_as_gfx950():
    """An sm_* arch (the reference's NVIDIA targets) resolves to gfx950 and is kept as arch_requested."""
    base, _ = spec.load(SPEC_Q4)
    c = spec.resolve(base, {"arch": "sm_80"})
    assert c["arch"] == "gfx950" and c["arch_requested"] == "sm_80"
    with pytest.raises(spec.SpecError, match="arch"):
        spec.resolve(base, {"arch": "sm_x"})
