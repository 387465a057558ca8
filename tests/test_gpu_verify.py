"""`komp verify` on the GPU: the full check set and the example specs' tune spaces must report 0 failures
(tests/test_komp.py:36-45)."""

import os
import subprocess
import sys

import pytest

from comp_amd import verify

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_run_all_zero_failures():
    lines = []
    fails = verify.run_all(log=lines.append)
    out = "\n".join(lines)
    assert fails == 0, out
    assert lines[-1] == "0 failures" and len(lines) == 114
    assert "MISMATCH" not in out and "DIFFERS" not in out


@pytest.mark.parametrize("spec", ["q4_0_gemv.kurn", "tq2_0_gemv.kurn"])
def test_cli_verify_spec_tune_space(spec):
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([ROOT, os.path.join(ROOT, "oracle")]))
    r = subprocess.run([sys.executable, "-m", "comp_amd", "verify", os.path.join(ROOT, "comp_amd", "examples", spec)],
                       capture_output=True, text=True, env=env, cwd=ROOT, timeout=600)  # fmt: skip
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert r.stdout.strip().endswith("0 failures")
    assert r.stdout.count("[gfx950]") == 16
