"""`komp gen` / `komp mix` on the gfx950 build (no GPU needed): the code objects inside the built library, their
register and spill metadata, approximate math, and hot-loop instruction mixes; the ISA reader's loop and class logic
on synthetic instruction lists."""

import os
import subprocess
import sys

import pytest

from comp_amd import cli, isa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SPEC_Q4 = os.path.join(ROOT, "comp_amd", "examples", "q4_0_gemv.kurn")
SPEC_TQ2 = os.path.join(ROOT, "comp_amd", "examples", "tq2_0_gemv.kurn")


def run(*args):
    return subprocess.run([sys.executable, "-m", "comp_amd", *args], capture_output=True, text=True, cwd=ROOT)


def test_library_holds_gfx950_code_objects_with_every_kernel_family():
    names = [n for co in isa.library_code_objects() for n in co.kernels]
    for family in ("gemv_impl::gemv_kernel<", "gemv_tq2::tq2_lean_kernel<", "gemv_tq2::tq2_lean_bytes_kernel<",
                   "gemv_tq2::tq2_lean_pre_kernel<", "gemv_tq2::tq2_lean_bytes_pre_kernel<", "gemv_tq2_mfma::tq2_mfma_kernel<",
                   "gemv_q4::q4_lean_kernel<", "gemv_q4k::q4k_lean_kernel<", "gemv_q8::q8_lean_kernel<",
                   "gemm_impl::gemm_kernel<", "quant_q8_0_kernel", "quant_q8_K_kernel", "stream_read_kernel",
                   "split_impl::split_kernel"):
        assert any(family in n for n in names), family


@pytest.mark.parametrize("fmt,bn,nb,nw,name", [("q4_0", 64, 4, 4, "gemv_q4::q4_lean_kernel<0, 4, 4, 1, false, false>"),
                                               ("tq2_0", 32, 2, 4, "gemv_tq2::tq2_lean_kernel<8, 2, 1, false, false, false>"),
                                               ("iq4_nl", 8, 2, 8, "gemv_q4::q4_lean_kernel<3, 64, 2, 1, false, false>"),
                                               ("q4_k", 64, 4, 4, "gemv_q4k::q4k_lean_kernel<4, 4, 1, false, false>")])
def test_single_column_configs_name_their_kernel(fmt, bn, nb, nw, name):
    # one column in dp4a mode runs the single-column kernel with 64 / min(block_n / num_warps, 16) lanes per row
    assert cli._gemv_kernel(fmt, 2, nb, 1, bn, nw) == name
    r = isa.summary(name, cli.VALUES_PER_LOAD[fmt])
    assert r["vgpr_spill"] == 0 and r["sgpr_spill"] == 0 and not r["approx"] and r["loop"].get("dot4", 0) > 0
    three = name.replace(", 1, false, false", ", 3, false, false", 1)
    assert cli._gemv_kernel(fmt, 2, nb, 3, bn, nw) == three  # three columns
    assert cli._gemv_kernel(fmt, 2, 8, 3, bn, nw).startswith("gemv_impl::gemv_kernel<")  # nb 8 at three columns
    if fmt in ("tq2_0", "q4_0"):  # bytes mode: the lean kernel's bytes form, with no dot instruction
        bytes_name = (name.replace("tq2_lean_kernel<", "tq2_lean_bytes_kernel<")
                      .replace(", false, false, false>", ", false, false>")
                      .replace("q4_lean_kernel<0, ", "q4_lean_bytes_kernel<"))
        assert cli._gemv_kernel(fmt, 0, nb, 1, bn, nw) == bytes_name
        r = isa.summary(bytes_name, cli.VALUES_PER_LOAD[fmt])
        assert r["vgpr_spill"] == 0 and r["sgpr_spill"] == 0 and not r["approx"] and r["dot4_total"] == 0
        assert r["loop"].get("ld128", 0) > 0
    else:
        assert cli._gemv_kernel(fmt, 0, nb, 1, bn, nw).startswith("gemv_impl::gemv_kernel<")  # bytes mode


@pytest.mark.parametrize("fmt,bn,nb,nw,k,m,name", [
    ("tq2_0", 16, 4, 4, 2560, 1, "gemv_tq2::tq2_lean_kernel<16, 4, 1, false, true, false>"),   # 10 blocks <= 4 x 4
    ("tq2_0", 16, 4, 4, 6912, 1, "gemv_tq2::tq2_lean_kernel<16, 4, 1, false, false, false>"),  # 27 blocks: two K steps
    # 3 x 10 blocks x 16 threads > 4 waves: staged through an LDS copy
    ("tq2_0", 16, 4, 4, 2560, 3, "gemv_tq2::tq2_lean_kernel<16, 4, 3, false, true, true>"),
    ("tq2_0", 16, 2, 4, 2560, 3, "gemv_tq2::tq2_lean_kernel<16, 2, 3, false, false, true>"),  # 10 blocks > 4 x 2
    # two passes of 3 K steps a wave: 6 tiles, the pipelined loop form
    ("tq2_0", 128, 4, 4, 2560, 1, "gemv_tq2::tq2_lean_pipe_kernel<4, 4, false, false>"),
    ("tq2_0", 64, 1, 4, 6912, 1, "gemv_tq2::tq2_lean_pipe_kernel<4, 4, false, false>"),  # the spec defaults: nb 1 -> 4, 7 tiles
    ("q4_0", 64, 4, 4, 4096, 1, "gemv_q4::q4_lean_pipe_kernel<0, 4, 4, false>"),  # 8 K steps of 16 blocks
    ("q4_0", 64, 4, 4, 4096, 2, "gemv_q4::q4_lean_kernel<0, 4, 4, 2, false, false>"),  # two columns: one buffer
    ("q4_0", 8, 2, 8, 4096, 1, "gemv_q4::q4_lean_kernel<0, 64, 2, 1, false, true>"),    # 128 blocks <= 64 x 2
    ("q4_0", 8, 2, 8, 4096, 3, "gemv_q4::q4_lean_kernel<0, 64, 2, 3, false, true>"),   # any column count
    ("iq4_nl", 8, 2, 8, 8192, 1, "gemv_q4::q4_lean_kernel<3, 64, 2, 1, false, false>"),
    ("q8_0", 8, 4, 8, 4096, 1, "gemv_q8::q8_lean_kernel<64, 4, 1, false, true>"),     # 128 blocks <= 32 x 4
    ("q8_0", 16, 4, 4, 4096, 3, "gemv_q8::q8_lean_kernel<16, 4, 3, false, false>"),    # 32 blocks a step: 4 steps
    ("q4_k", 8, 2, 4, 4096, 1, "gemv_q4k::q4k_lean_kernel<32, 2, 1, false, true>"),    # 16 blocks <= 8 x 2
    ("q4_k", 16, 2, 8, 4096, 3, "gemv_q4k::q4k_lean_kernel<32, 2, 3, false, true>"),   # any column count
    ("q4_k", 16, 2, 16, 14336, 1, "gemv_q4k::q4k_lean_kernel<64, 2, 1, false, false>"),  # 56 blocks: two K steps
])  # fmt: skip
def test_single_pass_form_follows_the_launch(fmt, bn, nb, nw, k, m, name):
    """With K known, the name carries the single-pass flag the launch computes (one pass of rows, one K step), and the
    single-pass form's report is its straight-line weight stream."""
    assert cli._gemv_kernel(fmt, 2, nb, m, bn, nw, k) == name
    r = isa.summary(name, cli.VALUES_PER_LOAD[fmt])
    assert r["vgpr_spill"] == 0 and r["sgpr_spill"] == 0 and not r["approx"]
    assert r["loop"].get("dot4", 0) > 0 and r["loop"].get("ld128", 0) > 0


def test_early_read_form_follows_the_grid():
    """One or two tq2_0 dp4a columns in the single-pass form (nb x columns <= 4, or 2 columns at nb 4 in at most 8
    waves) run the early-LDS-read form when the
    launch has at most one workgroup a CU (N known), the plain form otherwise; both keep their registers."""
    pre = "gemv_tq2::tq2_lean_pre_kernel<16, 4, 1, false, false>"
    assert cli._gemv_kernel("tq2_0", 2, 4, 1, 16, 4, 2560, 4096) == pre  # 256 workgroups
    assert cli._gemv_kernel("tq2_0", 2, 4, 1, 16, 4, 2560, 6912) == "gemv_tq2::tq2_lean_kernel<16, 4, 1, false, true, false>"
    assert cli._gemv_kernel("tq2_0", 2, 4, 3, 16, 4, 2560, 300).startswith("gemv_tq2::tq2_lean_kernel<16, 4, 3,")
    # two columns at nb 2 (4 slots x columns): the early reads too, here with the columns copied global -> LDS
    assert cli._gemv_kernel("tq2_0", 2, 2, 2, 8, 8, 6912, 2048) == "gemv_tq2::tq2_lean_pre_kernel<64, 2, 2, false, true>"
    # two columns at nb 4 (8 slots x columns) in workgroups of at most 8 waves (512-thread bounds: 256 VGPRs a wave)
    pre8 = "gemv_tq2::tq2_lean_pre_kernel<16, 4, 2, false, false>"
    assert cli._gemv_kernel("tq2_0", 2, 4, 2, 32, 8, 2560, 6912) == pre8
    assert cli._gemv_kernel("tq2_0", 2, 4, 2, 64, 16, 2560, 6912).startswith("gemv_tq2::tq2_lean_kernel<16, 4, 2,")
    for name in (pre, pre8):
        r = isa.summary(name, cli.VALUES_PER_LOAD["tq2_0"])
        assert r["vgpr_spill"] == 0 and r["sgpr_spill"] == 0 and r["loop"].get("dot4", 0) > 0
    # bytes mode, one column at nb <= 4: both staged planes read early (no dot instruction)
    pre_b = "gemv_tq2::tq2_lean_bytes_pre_kernel<16, 4, false>"
    assert cli._gemv_kernel("tq2_0", 0, 4, 1, 16, 4, 2560, 4096) == pre_b
    assert cli._gemv_kernel("tq2_0", 0, 4, 1, 16, 4, 2560, 6912).startswith("gemv_tq2::tq2_lean_bytes_kernel<16, 4, 1,")
    r = isa.summary(pre_b, cli.VALUES_PER_LOAD["tq2_0"])
    assert r["vgpr_spill"] == 0 and r["sgpr_spill"] == 0 and r["dot4_total"] == 0


@pytest.mark.parametrize("spec,fmt", [(SPEC_Q4, "q4_0"), (SPEC_TQ2, "tq2_0")])
def test_gen_reports_and_writes(spec, fmt, tmp_path):
    r = run("gen", spec, "-o", str(tmp_path))
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert lines[0].startswith("ok   ") and "spill=0" in lines[0] and "approx-ops=none" in lines[0]
    hot = int(lines[0].rsplit("in hot loop=", 1)[1])
    assert hot > 0  # dp4a mode: v_dot4c_i32_i8 in the hot loop
    assert any(ln.startswith("ok   quant_q8_") for ln in lines)
    files = sorted(os.listdir(tmp_path))
    assert len(files) == 4 and all(f.endswith((".hsaco", ".s")) for f in files)
    for f in files:
        data = open(tmp_path / f, "rb").read()
        if f.endswith(".hsaco"):
            assert data[:4] == b"\x7fELF"
    asm = open(tmp_path / [f for f in files if f.endswith(".s") and "gemv" in f][0]).read()
    assert "v_dot4c_i32_i8" in asm and "s_endpgm" in asm


def test_gen_bytes_mode_has_no_dot4_and_rejects_other_archs():
    r = run("gen", SPEC_Q4, "mode=bytes")
    assert r.returncode == 0 and "in hot loop=0" in r.stdout.splitlines()[0]
    assert run("gen", SPEC_Q4, "arch=sm_80").returncode == 2


def test_mix_lists_every_config():
    r = run("mix")
    assert r.returncode == 0, r.stdout + r.stderr
    for fmt, cfgs in cli.MIX_KOMP.items():
        for bn, nb, nw in cfgs:
            for mode in ("bytes", "dp4a "):
                assert f"KOMP {fmt} {mode} {bn}/{nb}/{nw}w" in r.stdout
    for fmt, cfgs in cli.MIX_MORE.items():
        for bn, nb, nw in cfgs:
            assert f"KOMP {fmt} dp4a  {bn}/{nb}/{nw}w" in r.stdout
    assert "GEMM q4_0 16 rows x 64 cols" in r.stdout and "v_mfma 64" in r.stdout
    assert run("mix", "--archs", "sm_80").stdout.count("not built") == 1


def test_loops_classes_and_approx_on_synthetic_code():
    insts = [(0x100, "s_mov_b32", "s0, 0", None), (0x104, "global_load_dwordx4", "v[0:3]", None),
             (0x10C, "v_dot4c_i32_i8", "v4, v0, v1", None), (0x110, "v_and_b32", "v1, v2, v3", None),
             (0x114, "s_cbranch_scc1", "-4", 0x104), (0x118, "s_branch", "2", 0x120), (0x11C, "s_nop", "0", None),
             (0x120, "s_endpgm", "", None)]  # fmt: skip
    assert isa.loops(insts) == [(1, 4)]
    c = isa.mix(insts, 1, 4)
    assert c["ld128"] == 1 and c["dot4"] == 1 and c["int"] == 2 and c["insts"] == 4
    rcp = [(0, "v_rcp_f32", "", None), (4, "v_div_fixup_f32", "", None)]
    assert isa.approx_ops(rcp) == [] and isa.approx_ops(rcp[:1]) == ["v_rcp_f32"]
    assert isa.approx_ops([(0, "v_exp_f32", "", None)]) == ["v_exp_f32"]
    assert isa.classify("buffer_load_ushort") == "ld16" and isa.classify("ds_read_b128") == "lds"
    assert isa.classify("v_mfma_i32_16x16x32_i8") == "mfma"


def test_lean_and_gemm_instantiations_do_not_spill():
    """Every lean GEMV, matrix-core GEMV and GEMM instantiation of this build keeps its registers: no VGPR or SGPR spills
    to scratch memory (the general kernel's rare explicit-knob forms, nb 16 with 3 columns in bytes or emulated mode,
    are outside this check)."""
    spills = []
    for co in isa.library_code_objects():
        for name, k in co.kernels.items():
            lean_or_gemm = "lean" in name or "gemm_kernel" in name or "mfma_kernel" in name
            if lean_or_gemm and (k["vgpr_spill"] or k["sgpr_spill"] or k["scratch"]):
                spills.append((name[:90], k["vgpr_spill"], k["scratch"]))
    assert not spills, spills
