"""gfx950 ISA of this build's own kernels: the code objects inside libkomp_hip.so, their register/LDS metadata and
the instruction mix of a kernel's hot loop.

This is the gfx950 counterpart of the reference's PTX/SASS inspection behind `komp gen` and `komp mix`
(src/komp/compile.py:53-117, src/komp/cli.py:88-158); it reads only the AMD code objects this repository compiles
from source (the `.hip_fatbin` section of the library: one clang offload bundle per translation unit), with the LLVM
tools of the ROCm install (llvm-objcopy, llvm-objdump, llvm-readelf).
"""

from __future__ import annotations

import atexit
import os
import re
import shutil
import struct
import subprocess
import tempfile

import yaml

from . import _abi

TRIPLE = "hipv4-amdgcn-amd-amdhsa--gfx950"
_FUNC = re.compile(r"^[0-9a-f]+\s.*?\sF\s+\.text\s+[0-9a-f]+\s+(?:\.(?:protected|hidden|internal)\s+)?(.*)$")
_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
_HEAD = re.compile(r"^([0-9a-f]+) <[^>]+>:$")                       # "00000000000a8b00 <symbol>:"
_INST = re.compile(r"^\s+(\S.*?)\s*//\s*([0-9A-Fa-f]+):(.*)$")   # "\tmnemonic ops // ADDR: encoding [<sym+0xOFF>]"
_TARGET = re.compile(r"<[^>+]+\+0x([0-9a-f]+)>")


def llvm_tool(name):
    """Path of an LLVM tool of the ROCm install (ROCM_PATH, /opt/rocm, or PATH)."""
    for root in (os.environ.get("ROCM_PATH"), "/opt/rocm"):
        if root:
            p = os.path.join(root, "llvm", "bin", name)
            if os.path.exists(p):
                return p
    p = shutil.which(name)
    if p is None:
        raise FileNotFoundError(f"{name} not found (ROCm's llvm/bin)")
    return p


def _run(*cmd, binary=False):
    r = subprocess.run(cmd, capture_output=True, text=not binary)
    if r.returncode != 0:
        raise RuntimeError(f"{os.path.basename(cmd[0])} failed: {r.stderr if not binary else r.stderr.decode()}")
    return r.stdout


_CACHE = {}  # (library path, mtime) -> [CodeObject]; removed at exit


@atexit.register
def _cleanup():
    for cos in _CACHE.values():
        for co in cos:
            co.close()
    _CACHE.clear()


def library_code_objects(lib_path=None):
    """The library's gfx950 code objects, parsed once per process (and again when the library file changes)."""
    lib_path = lib_path or _abi.LIB_PATH
    key = (os.path.abspath(lib_path), os.path.getmtime(lib_path))
    if key not in _CACHE:
        _CACHE[key] = [CodeObject(data) for data in code_objects(lib_path)]
    return _CACHE[key]


def code_objects(lib_path=None):
    """The gfx950 code objects (bytes) of the library, one per translation unit with device code."""
    lib_path = lib_path or _abi.LIB_PATH
    with tempfile.TemporaryDirectory() as d:
        fat = os.path.join(d, "fatbin")
        _run(llvm_tool("llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", lib_path, os.path.join(d, "stripped"))
        blob = open(fat, "rb").read()
    out = []
    for m in re.finditer(re.escape(_MAGIC), blob):
        s = m.start()
        (count,) = struct.unpack_from("<Q", blob, s + len(_MAGIC))
        p = s + len(_MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", blob, p)
            p += 24
            triple = blob[p : p + tlen].decode()
            p += tlen
            if triple == TRIPLE and size:
                out.append(blob[s + off : s + off + size])
    return out


class CodeObject:
    """One code object: its kernels (demangled name -> metadata) and their disassembly."""

    def __init__(self, data):
        self.data = data
        self._dir = tempfile.mkdtemp(prefix="komp_isa_")
        self.path = os.path.join(self._dir, "co.hsaco")
        with open(self.path, "wb") as fh:
            fh.write(data)
        self.kernels = self._kernels()

    def close(self):
        shutil.rmtree(self._dir, ignore_errors=True)

    def _kernels(self):
        notes = _run(llvm_tool("llvm-readelf"), "--notes", self.path)
        i = notes.find("amdhsa.kernels:")
        meta = yaml.safe_load(notes[i : notes.find("...", i)] if notes.find("...", i) > 0 else notes[i:])
        def funcs(*flags):  # symbol-table function names: "addr flags F .text size [.visibility] name"
            out = []
            for ln in _run(llvm_tool("llvm-objdump"), "-t", *flags, self.path).splitlines():
                m = _FUNC.match(ln)
                if m:
                    out.append(m.group(1).strip())
            return out

        mangled, demangled = funcs(), funcs("-C")
        names = dict(zip(mangled, demangled))
        out = {}
        for k in meta["amdhsa.kernels"]:
            sym = k[".name"]
            out[names.get(sym, sym)] = {
                "symbol": sym,
                "vgpr": k.get(".vgpr_count", 0),
                "agpr": k.get(".agpr_count", 0),
                "sgpr": k.get(".sgpr_count", 0),
                "vgpr_spill": k.get(".vgpr_spill_count", 0),
                "sgpr_spill": k.get(".sgpr_spill_count", 0),
                "lds": k.get(".group_segment_fixed_size", 0),
                "scratch": k.get(".private_segment_fixed_size", 0),
                "max_threads": k.get(".max_flat_workgroup_size", 0),
            }
        return out

    def disassemble(self, symbol):
        """The kernel's instructions as (address, mnemonic, operands, branch target address or None), in order."""
        text = _run(llvm_tool("llvm-objdump"), "-d", "--no-show-raw-insn", "--mcpu=gfx950",
                    f"--disassemble-symbols={symbol}", self.path)  # fmt: skip
        out = []
        start = None
        for ln in text.splitlines():
            m = _HEAD.match(ln.strip())
            if m:
                start = int(m.group(1), 16)
                continue
            m = _INST.match(ln)
            if not m or start is None:
                continue
            body, addr, rest = m.group(1).strip(), int(m.group(2), 16), m.group(3)
            parts = body.split(None, 1)
            t = _TARGET.search(rest)
            out.append((addr, parts[0], parts[1] if len(parts) > 1 else "", start + int(t.group(1), 16) if t else None))
        return out


def find_kernel(prefix, lib_path=None):
    """(CodeObject, demangled name) of the first kernel whose demangled name contains `prefix` followed by '(' or
    template arguments (e.g. 'gemv_impl::gemv_kernel<0, 2, 1, 4, false>' or 'quant_q8_0_kernel')."""
    for co in library_code_objects(lib_path):
        for name in co.kernels:
            if prefix + "(" in name or (prefix.endswith(">") and prefix in name):
                return co, name
    raise KeyError(f"no kernel {prefix}... in the library")


# ---- instruction classes ----------------------------------------------------------------------------------------------
_LOAD_WIDTH = (("dwordx4", "ld128"), ("b128", "ld128"), ("dwordx3", "ld96"), ("dwordx2", "ld64"), ("b64", "ld64"),
               ("dword", "ld32"), ("b32", "ld32"), ("short", "ld16"), ("b16", "ld16"), ("byte", "ld8"), ("b8", "ld8"))
_APPROX = ("v_rsq_", "v_sqrt_", "v_exp_", "v_log_", "v_sin_", "v_cos_")


def classify(mn):
    """Coarse class of one mnemonic."""
    if mn.startswith(("global_load", "buffer_load", "flat_load")):
        for key, cls in _LOAD_WIDTH:
            if key in mn:
                return cls
        return "ld_other"
    if mn.startswith(("global_store", "buffer_store", "flat_store")):
        return "store"
    if mn.startswith("ds_"):
        return "lds"
    if mn.startswith("v_mfma"):
        return "mfma"
    if mn.startswith(("v_dot4", "v_dot2")):
        return "dot4"
    if mn.startswith("v_"):
        return "valu"
    if mn.startswith(("s_waitcnt", "s_nop", "s_barrier", "s_cbranch", "s_branch", "s_endpgm", "s_setprio")):
        return "ctrl"
    if mn.startswith("s_"):
        return "salu"
    return "other"


_INT_VALU = re.compile(r"^v_(and|or|xor|lshl|lshr|ashr|bfe|bfi|perm|alignbyte|add_u|add_i|sub_u|sub_i|mad_u|mad_i|"
                       r"mul_lo|mul_hi|mul_u|mul_i|cndmask|min_i|max_i|min_u|max_u|med3_i|med3_u|not|mov|lshl_add|add3|"
                       r"lshl_or|and_or|or3|xad|sad|bcnt|ffbh|ffbl|readfirstlane|cmp_.*_[iu]|permlane|mbcnt)")  # fmt: skip


def loops(insts):
    """Loops as (first, last) instruction index ranges: each backward branch and the instruction it jumps to.  A
    backward branch across an `s_endpgm` is the way back from a block the compiler placed after the kernel's end (an
    unlikely path), not a loop."""
    index = {addr: i for i, (addr, _, _, _) in enumerate(insts)}
    ends = [i for i, (_, mn, _, _) in enumerate(insts) if mn.startswith("s_endpgm")]
    spans = set()
    for i, (addr, mn, _, target) in enumerate(insts):
        if mn.startswith(("s_cbranch", "s_branch")) and target is not None and target <= addr and target in index:
            a = index[target]
            if not any(a <= e < i for e in ends):
                spans.add((a, i))
    return sorted(spans)


def mix(insts, first=0, last=None):
    """Instruction counts by class (plus `int` VALU and `insts`) over insts[first .. last]."""
    last = len(insts) - 1 if last is None else last
    counts = {"insts": 0, "int": 0}
    for _, mn, _, _ in insts[first : last + 1]:
        counts["insts"] += 1
        cls = classify(mn)
        counts[cls] = counts.get(cls, 0) + 1
        if (cls == "valu" and _INT_VALU.match(mn)) or cls == "dot4":
            counts["int"] += 1
    return counts


def approx_ops(insts):
    """Approximate-math instructions in the kernel: transcendentals, and v_rcp_f32 beyond the ones that belong to the
    correctly rounded division sequence (one per v_div_fixup_f32)."""
    mns = [mn for _, mn, _, _ in insts]
    found = sorted({mn for mn in mns if mn.startswith(_APPROX)})
    if sum(mn.startswith("v_rcp_f32") for mn in mns) > sum(mn.startswith("v_div_fixup_f32") for mn in mns):
        found.append("v_rcp_f32")
    return found


def hot_loop(insts, weight_bytes_per_load=None):
    """The kernel's hot loop: among its loops, the one with the most weight loads (128-bit) and then VALU work;
    -> (first, last, counts) or None.  A kernel with no loop after its last barrier (the lean kernels' single-pass
    form, whose weight stream after the staged activations are published is straight-line code) reports that stream
    instead, up to the end of the kernel, with the kernel's 128-bit buffer loads (its weight loads) as its loads."""
    spans = loops(insts)
    bars = [i for i, (_, mn, _, _) in enumerate(insts) if mn.startswith("s_barrier")]
    ends = [i for i, (_, mn, _, _) in enumerate(insts) if mn.startswith("s_endpgm")]
    if bars and any(e > bars[-1] for e in ends):
        last = min(e for e in ends if e > bars[-1])
        if not any(bars[-1] <= a <= last for a, _ in spans):
            c = mix(insts, bars[-1], last)
            if c.get("dot4", 0) or c.get("mfma", 0):
                c["ld128"] = sum(mn.startswith("buffer_load_dwordx4") for _, mn, _, _ in insts)
                return bars[-1], last, c
    best = None
    for a, b in spans:
        c = mix(insts, a, b)
        key = (c.get("ld128", 0), c.get("valu", 0) + c.get("dot4", 0) + c.get("mfma", 0))
        if best is None or key > best[0]:
            best = (key, a, b, c)
    return None if best is None else (best[1], best[2], best[3])


def summary(prefix, values_per_load, lib_path=None, keep=False):
    """Metadata, approximate ops and hot-loop mix of one kernel.  values_per_load: weight values per 128-bit load
    of the loop (Q4_0 32, TQ2_0 64), which turns loop counts into per-weight figures."""
    co, name = find_kernel(prefix, lib_path)
    meta = co.kernels[name]
    insts = co.disassemble(meta["symbol"])
    hl = hot_loop(insts)
    counts = hl[2] if hl else {}
    per_thread = counts.get("ld128", 0) * values_per_load
    res = {"kernel": name, **meta, "approx": approx_ops(insts), "dot4_total": mix(insts).get("dot4", 0),
           "loop": counts, "loop_len": counts.get("insts", 0), "values_per_thread": per_thread,
           "insts_per_value": counts.get("insts", 0) / per_thread if per_thread else 0.0,
           "int_per_value": counts.get("int", 0) / per_thread if per_thread else 0.0,
           "dot4_per_value": counts.get("dot4", 0) / per_thread if per_thread else 0.0}  # fmt: skip
    if keep:
        res["code_object"] = co.data
        res["asm"] = "".join(f"{addr:08x}:\t{mn} {ops}".rstrip() + "\n" for addr, mn, ops, _ in insts)
    return res
