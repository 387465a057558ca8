"""ctypes binding of libkomp_hip.so (the C ABI declared in include/komp_abi.h).

torch is imported first on purpose: it loads its own HIP runtime (soname libamdhip64.so.7), and the dynamic linker
then binds this library to that same runtime, so torch's streams and device pointers are valid here.

There is no fallback: if the library is missing or fails to load, every call raises KompError.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (see the module docstring)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkomp_hip.so")

KOMP_OK, KOMP_EINVAL, KOMP_EHIP = 0, 1, 2
TIMING_KINDS = ("quant_q8_0", "quant_q8_K", "q4_0_gemv", "tq2_0_gemv", "probe", "q8_0_gemv", "iq4_nl_gemv",
                "q4_k_gemv")


class KompError(RuntimeError):
    """A call into the HIP library failed (or the library is not available)."""


class KompArgumentError(KompError, ValueError):
    """The HIP library rejected an argument (shape, stride, alignment, knob or mode)."""


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int

# name -> (restype, argtypes); exactly the functions include/komp_abi.h declares
SIGNATURES = {
    "komp_abi_version": (_INT, []),
    "komp_last_error": (ctypes.c_char_p, []),
    "komp_quant_q8_0": (_INT, [_P, _P, _P, _I64, _I64, _INT, _P]),
    "komp_quant_q8_K": (_INT, [_P, _P, _P, _P, _I64, _I64, _P]),
    "komp_q4_0_gemv": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_tq2_0_gemv": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_q4_0_gemv_f32": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_tq2_0_gemv_f32": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_q4_0_gemv_multi": (_INT, [_INT, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_tq2_0_gemv_multi": (_INT, [_INT, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_gemv_auto_config": (_INT, [_INT, _INT, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P]),
    **{f"komp_{f}_gemv": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P])
       for f in ("q8_0", "iq4_nl")},
    **{f"komp_{f}_gemv_f32": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P])
       for f in ("q8_0", "iq4_nl")},
    **{f"komp_{f}_gemv_multi": (_INT, [_INT, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _INT, _P])
       for f in ("q8_0", "iq4_nl")},
    **{f"komp_{f}_gemm": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]) for f in ("q8_0", "iq4_nl")},
    **{f"komp_{f}_split": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]) for f in ("q8_0", "iq4_nl")},
    "komp_q4_k_gemv": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_q4_k_gemv_f32": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_q4_k_gemv_multi": (_INT, [_INT, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _INT, _P]),
    "komp_q4_k_split": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "komp_q4_k_gemm": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "komp_q4_0_gemm": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "komp_tq2_0_gemm": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "komp_gemm_plan": (_INT, [_INT, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "komp_gemv_mfma_plan": (_INT, [_INT, _INT, _INT, _I64, _I64, _I64, _I64, _P, _P]),
    "komp_q4_0_split": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "komp_tq2_0_split": (_INT, [_P, _P, _P, _I64, _I64, _I64, _P]),
    "komp_dp4a_probe": (_INT, [_P, _P, _P, _P, _I64, _INT, _P]),
    "komp_stream_read": (_INT, [_P, _I64, _P, _P]),
    "komp_q4_0_decode": (_INT, [_P, _P, _I64, _P]),
    "komp_tq2_0_decode": (_INT, [_P, _P, _I64, _P]),
    "komp_timing_begin": (_INT, [_I64]),
    "komp_timing_end": (_INT, [_P, _P]),
    "komp_stamps_begin": (_INT, [_P, _I64]),
    "komp_stamps_end": (_INT, [_P, _P]),
    "komp_clock": (_INT, [_P, _P]),
    "komp_clock_khz": (_INT, [_P]),
}
ABI_VERSION = 1

_lib = None


def lib():
    """The loaded library (loaded once).  Raises KompError if it is missing or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise KompError(f"{LIB_PATH} is not built: run `python -m comp_amd.build` (hipcc, gfx950)")
    try:
        handle = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        raise KompError(f"cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    v = handle.komp_abi_version()
    if v != ABI_VERSION:
        raise KompError(f"{LIB_PATH}: ABI version {v}, expected {ABI_VERSION}; rebuild it")
    _lib = handle
    return _lib


def last_error():
    return lib().komp_last_error().decode(errors="replace")


def check(status, what):
    if status == KOMP_OK:
        return
    msg = last_error() or f"{what}: status {status}"
    if status == KOMP_EINVAL:
        raise KompArgumentError(msg)
    raise KompError(msg)


def call(name, *args):
    """Call an ABI function and raise on a nonzero status."""
    check(getattr(lib(), name)(*args), name)


def auto_plan(fmt_id, m, n, k, fused=False, mode=2):
    """(block_n, nb, num_warps, lanes_per_row, passes) of the plan block_n == 0 selects."""
    v = [ctypes.c_int() for _ in range(5)]
    call("komp_gemv_auto_config", fmt_id, int(bool(fused)), mode, m, n, k, *(ctypes.byref(x) for x in v))
    return tuple(x.value for x in v)


def auto_config(fmt_id, m, n, k, fused=False, mode=2):
    return auto_plan(fmt_id, m, n, k, fused, mode)[:3]


def gemm_plan(fmt_id, m, n, k, sw):
    """(rows per workgroup, columns per workgroup, waves) of the matrix-core GEMM, or None past its limits."""
    v = [ctypes.c_int(0) for _ in range(3)]
    st = lib().komp_gemm_plan(fmt_id, m, n, k, sw, *(ctypes.byref(x) for x in v))
    return tuple(x.value for x in v) if st == 0 else None


def gemv_mfma_plan(fmt_id, fused, mode, m, n, k, sw):
    """(rows per workgroup, waves) of the matrix-core GEMV when the library plan runs it for this call, else None."""
    v = [ctypes.c_int(0) for _ in range(2)]
    st = lib().komp_gemv_mfma_plan(fmt_id, int(fused), mode, m, n, k, sw, *(ctypes.byref(x) for x in v))
    if st < 0:
        raise KompArgumentError(last_error())
    return tuple(x.value for x in v) if st == 1 else None


def timing_begin(max_dispatches=1 << 16):
    call("komp_timing_begin", max_dispatches)


def timing_end():
    """-> {kind: (total_ms, dispatches)} for the dispatches since timing_begin()."""
    ms = (ctypes.c_double * len(TIMING_KINDS))()
    cnt = (ctypes.c_int64 * len(TIMING_KINDS))()
    call("komp_timing_end", ms, cnt)
    return {k: (ms[i], cnt[i]) for i, k in enumerate(TIMING_KINDS)}


STAMP_MAGIC = 0x4B535450


def stamps_begin(buf):
    """Start recording wave stamps into `buf`, a 16-byte aligned int32 / uint32 device tensor (komp_stamps_begin)."""
    call("komp_stamps_begin", ctypes.c_void_p(buf.data_ptr()), buf.numel())


def stamps_end():
    """-> (words used, counter rate in kHz) (komp_stamps_end)."""
    used, khz = ctypes.c_int64(0), ctypes.c_int(0)
    call("komp_stamps_end", ctypes.byref(used), ctypes.byref(khz))
    return used.value, khz.value


def parse_stamps(words, clock_khz):
    """Records of a stamp buffer (uint32 numpy array, the words komp_stamps_end reported) -> one dict per launch:
    n, k, waves, and for each of entry / staged / dots / stored the per-wave times in ns from the launch's first
    entry (int64 arrays), plus span_ns = last stored - first entry."""
    import numpy as np

    words = np.asarray(words, dtype=np.uint32)
    ns_per_tick = 1e6 / clock_khz
    out, off = [], 0
    while off + 4 <= words.size:
        magic, waves, n, k = (int(v) for v in words[off:off + 4])
        if magic != STAMP_MAGIC:
            raise KompError(f"stamp buffer: no launch header at word {off}")
        rec = words[off + 4:off + 4 + 4 * waves].reshape(waves, 4).astype(np.int64)
        rel = (rec - rec[0, 0] + (1 << 31)) % (1 << 32) - (1 << 31)  # the counter's low words, wrap-safe
        rel -= rel[:, 0].min()
        t = rel * ns_per_tick
        out.append({"n": n, "k": k, "waves": waves, "entry": t[:, 0], "staged": t[:, 1], "dots": t[:, 2],
                    "stored": t[:, 3], "span_ns": float(t[:, 3].max())})
        off += (4 + 4 * waves + 3) & ~3
    return out


def clock_into(out, stream=None):
    """Write the device's real-time counter to out[0] (an int64 device tensor) when the stream gets there (komp_clock;
    inside a graph capture too).  stream: a torch stream (default: the current one)."""
    st = (stream or torch.cuda.current_stream()).cuda_stream
    call("komp_clock", ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st))


def clock_khz():
    """The rate of komp_clock's counter in kHz."""
    khz = ctypes.c_int(0)
    call("komp_clock_khz", ctypes.byref(khz))
    return khz.value
