"""The reference's import name and command line: `komp` resolves to this build (tests/test_komp.py:62-66)."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SPEC = os.path.join(ROOT, "comp_amd", "examples", "q4_0_gemv.kurn")


def run(*args):
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([ROOT, os.path.join(ROOT, "oracle")]))
    return subprocess.run([sys.executable, "-m", *args], capture_output=True, text=True, env=env, cwd=ROOT, timeout=300)


def test_komp_modules_are_comp_amds():
    import komp
    from komp import host, spec

    import comp_amd.host
    import comp_amd.spec
    import komp.cli
    import komp.verify

    assert host is comp_amd.host and spec is comp_amd.spec and komp.host is comp_amd.host
    assert komp.cli.main is __import__("comp_amd.cli").cli.main and komp.verify.TOL == 1e-5


def test_komp_check_accepts_the_example_spec():
    r = run("komp", "check", SPEC)
    assert r.returncode == 0 and "tune space: 8 legal configs" in r.stdout, r.stdout + r.stderr


def test_bad_spec_rejected(tmp_path):
    p = tmp_path / "bad.kurn"
    p.write_text(open(SPEC).read().replace("block_n    64", "block_n    33"))
    r = run("komp", "check", str(p))
    assert r.returncode == 2 and "block_n" in r.stderr, r.stdout + r.stderr



def test_reference_arch_lines_check_and_gen_refuses(tmp_path):
    """The reference's specs name an NVIDIA arch (examples/q4_0_gemv_triton.kurn:6): check runs them as gfx950, gen
    (which writes code objects for the spec's arch) refuses them."""
    p = tmp_path / "sm80.kurn"
    p.write_text(open(SPEC).read().replace("arch       gfx950", "arch       sm_80"))
    r = run("komp", "check", str(p))
    assert r.returncode == 0 and "sm_80 (run as gfx950)" in r.stdout and "8 legal configs" in r.stdout, r.stdout + r.stderr
    r = run("komp", "gen", str(p))
    assert r.returncode == 2 and "gfx950" in r.stderr, r.stdout + r.stderr
    p.write_text(open(SPEC).read().replace("arch       gfx950", "arch       rdna9"))
    r = run("komp", "check", str(p))
    assert r.returncode == 2 and "arch" in r.stderr, r.stdout + r.stderr


REFERENCE_EXAMPLES = "/root/reference/examples"


@pytest.mark.skipif(not os.path.isdir(REFERENCE_EXAMPLES), reason="the reference tree is not on this machine")
def test_reference_example_specs_check_unchanged():
    """`komp check` on the reference's own example specs, as they are (tests/test_komp.py:43-45 verifies them)."""
    for name in ("q4_0_gemv_triton.kurn", "tq2_0_gemv_triton.kurn"):
        r = run("komp", "check", os.path.join(REFERENCE_EXAMPLES, name))
        assert r.returncode == 0 and "run as gfx950" in r.stdout, r.stdout + r.stderr
