"""Host side of the decode path: KURN split layouts from ggml blocks, and the quantizer / GEMV launches.

Same surface as the reference's operator boundary src/komp/host.py:1-85 (FORMATS, MODES, split, split_q4_0,
tq2_0_qplane, q8_0_blocks, q8_K_blocks, act_blocks, device, quantize, gemv), with the same argument meaning.  The
launches go to hand-written gfx950 HIP kernels through the C ABI (comp_amd._abi), on the current torch stream, with
no synchronisation inside.

Differences a caller can observe:
  * quantize / gemv need tensors on a HIP device (like any compiled Triton kernel); there is no CPU path, and the
    call raises if the HIP library is not built.
  * mode 1 runs the packed-word dot products emulated with shifts and multiplies and mode 2 on v_dot4c_i32_i8 (the
    reference's mode 1 is its pure-Triton fallback, mode 2 inline PTX); all modes give identical int32 dots.
  * quantize(..., bsums=True) also returns the q8_K bsums, computed by the kernel.
  * gemv(..., block_n=None) lets the library choose block_n / nb / num_warps for the shape.
  * arguments the kernels cannot take (K not a multiple of the block, misaligned or strided planes, unknown knobs)
    raise KompArgumentError (a ValueError) instead of reading out of bounds.

Beyond the reference: gemm (the matrix-core batched GEMM, which gemv(..., block_n=None) uses from GEMM_MIN_M
columns), gemv_f32 (quantize and GEMV in one launch), gemv_multi (several matrices sharing one input), split_device
(ggml blocks split on the device), the *_into variants that write preallocated outputs, and three more ggml weight
formats in every call: q8_0, iq4_nl (q8_0 activations) and q4_k (q8_K activations; its scale plane holds each
block's 16 leading bytes and its S two int32 per block).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _abi

FORMATS = {  # weights: block values, block bytes, quant offset/bytes, scale offset, activation format
    "q4_0": dict(block=32, nbytes=18, qoff=2, qbytes=16, soff=0, act="q8_0"),
    "tq2_0": dict(block=256, nbytes=66, qoff=0, qbytes=64, soff=64, act="q8_K"),
    # ggml formats beyond the reference's two (its README.md:143 lists them as next): same planes, q8_0 activations
    "q8_0": dict(block=32, nbytes=34, qoff=2, qbytes=32, soff=0, act="q8_0"),
    "iq4_nl": dict(block=32, nbytes=18, qoff=2, qbytes=16, soff=0, act="q8_0"),
    # ggml block_q4_K (d, dmin, 12 bytes of 6-bit sub-block scales and mins, 128 quant bytes) with q8_K activations;
    # its scale plane keeps each block's first 16 bytes: WS int16 [N][8 * K/256], and S holds (sd, sm) per block
    "q4_k": dict(block=256, nbytes=144, qoff=16, qbytes=128, soff=0, sbytes=16, act="q8_K"),
}
for _f in FORMATS.values():
    _f.setdefault("sbytes", 2)  # scale-plane bytes per block
MODES = {"bytes": 0, "dp4a": 2}  # mode 1 = dp4a emulated with shifts and multiplies
FMT_ID = {"q4_0": 0, "tq2_0": 1, "q8_0": 2, "iq4_nl": 3, "q4_k": 4}
_XB_F32 = ("q4_0", "tq2_0", "q4_k")  # formats whose gemv_f32 entry takes the XB (bsums) output
GEMM_MIN_M = {f: 4 for f in FMT_ID}  # columns from which gemv(..., block_n=None, mode=2) runs the matrix-core GEMM


def split(fmt, W, n, k):
    """ggml blocks (bytes, n rows) -> (WQ uint8 [n][quant bytes per row], WS int16 [n][blocks]): KURN's split planes.

    src/komp/host.py:16-22.  q4_k: WS int16 [n][8 * blocks] (each block's d, dmin and 12 scale bytes)."""
    f = FORMATS[fmt]
    nb = k // f["block"]
    sb = f["sbytes"]
    blocks = np.frombuffer(W, dtype=np.uint8).reshape(n, nb, f["nbytes"])
    wq = blocks[:, :, f["qoff"] : f["qoff"] + f["qbytes"]].reshape(n, nb * f["qbytes"]).copy()
    ws = blocks[:, :, f["soff"] : f["soff"] + sb].copy().view(np.int16).reshape(n, nb * sb // 2)
    return wq, ws


def _ws_cols(fmt, nblk):
    """int16 columns of the scale plane for nblk blocks."""
    return nblk * FORMATS[fmt]["sbytes"] // 2


def _s_shape(fmt, m, n, nblk):
    """Shape of S: int32 [M][N][blocks], q4_k [M][N][blocks][2] (the scaled dot sd and the mins dot sm)."""
    return (m, n, nblk, 2) if fmt == "q4_k" else (m, n, nblk)


def split_device(fmt, W, n, k, sw=None):
    """ggml blocks already on the device (uint8 tensor of n * (k / block) blocks) -> (WQ uint8 [n][sw], WS int16
    [n][blocks]) on the same device, bytes equal to split()'s.  sw: WQ row stride in bytes (default the packed row,
    rounded up to 16).  The device counterpart of src/komp/host.py:16-22."""
    f = FORMATS[fmt]
    _need(W, "W", torch.uint8)
    nb = k // f["block"]
    if k % f["block"] or n < 0:
        raise _abi.KompArgumentError(f"split_device: k={k} must be a multiple of {f['block']}")
    if W.numel() != n * nb * f["nbytes"] or not W.is_contiguous():
        raise _abi.KompArgumentError(f"split_device: W must be {n * nb * f['nbytes']} contiguous bytes, got {W.numel()}")
    row = nb * f["qbytes"]
    sw = (row + 15) // 16 * 16 if sw is None else sw
    wq = torch.empty((n, sw), dtype=torch.uint8, device=W.device)
    ws = torch.empty((n, _ws_cols(fmt, nb)), dtype=torch.int16, device=W.device)
    split_into(fmt, W, wq, ws, n, k)
    return wq[:, :row], ws


def split_into(fmt, W, wq, ws, n, k):
    """Allocation-free split_device into preallocated wq uint8 [n][sw] (row stride sw, a multiple of 16) and ws int16
    [n][blocks]."""
    f = FORMATS[fmt]
    _need(W, "W", torch.uint8)
    _need(wq, "wq", torch.uint8, 2)
    _need(ws, "ws", torch.int16, 2)
    nb = k // f["block"]
    if tuple(ws.shape) != (n, _ws_cols(fmt, nb)) or not ws.is_contiguous():
        raise _abi.KompArgumentError(f"split_into: ws must be a contiguous [{n}][{_ws_cols(fmt, nb)}] plane")
    if wq.shape[0] != n or wq.shape[1] < nb * f["qbytes"] or (wq.numel() and wq.stride(1) != 1):
        raise _abi.KompArgumentError(f"split_into: wq must be [{n}][>= {nb * f['qbytes']}] with contiguous rows")
    if W.numel() != n * nb * f["nbytes"] or not W.is_contiguous():
        raise _abi.KompArgumentError(f"split_into: W must be {n * nb * f['nbytes']} contiguous bytes")
    for t, name in ((wq, "wq"), (ws, "ws")):
        if t.device != W.device:
            raise _abi.KompArgumentError(f"{name} is on {t.device}, W on {W.device}")
    fn = f"komp_{fmt}_split"
    with torch.cuda.device(W.device):
        _abi.call(fn, W.data_ptr(), wq.data_ptr(), ws.data_ptr(), n, k, wq.stride(0) if n else 16, _stream(W))


def split_q4_0(W, n, k):
    return split("q4_0", W, n, k)


def tq2_0_qplane(W, nblk):
    """ggml tq2_0 blocks -> the quant plane [nblk][64] (the f16 d goes to the scale plane).  src/komp/host.py:29-31."""
    return np.frombuffer(W, dtype=np.uint8).reshape(nblk, 66)[:, :64].copy()


def _np(a):
    return a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)


def q8_0_blocks(xq, xd):
    """q8_0 split planes -> ggml q8_0 blocks (bytes): f16 d then 32 int8 per block.  src/komp/host.py:34-40."""
    xq, xd = _np(xq), _np(xd)
    m, k = xq.shape
    nb = k // 32
    out = np.empty((m, nb, 34), dtype=np.uint8)
    out[:, :, 0:2] = np.asarray(xd, np.float32).astype(np.float16).view(np.uint8).reshape(m, nb, 2)
    out[:, :, 2:34] = np.asarray(xq, np.int8).view(np.uint8).reshape(m, nb, 32)
    return out.tobytes()


def q8_K_blocks(xq, xd, xb=None):
    """q8_K split planes (numpy) -> ggml q8_K blocks (bytes): f32 d, 256 int8, 16 int16 bsums.

    src/komp/host.py:43-52; the bsums come from `xb` (the kernel's) when given, else from xq."""
    xq, xd = _np(xq), _np(xd)
    xb = None if xb is None else _np(xb)
    m, k = xq.shape
    nb = k // 256
    out = np.empty((m, nb, 292), dtype=np.uint8)
    out[:, :, 0:4] = np.asarray(xd, np.float32).view(np.uint8).reshape(m, nb, 4)
    out[:, :, 4:260] = np.asarray(xq, np.int8).view(np.uint8).reshape(m, nb, 256)
    if xb is None:
        xb = np.asarray(xq, np.int8).astype(np.int32).reshape(m, nb, 16, 16).sum(axis=3).astype(np.int16)
    out[:, :, 260:292] = np.asarray(xb, np.int16).view(np.uint8).reshape(m, nb, 32)
    return out.tobytes()


def act_blocks(fmt, xq, xd, xb=None):
    if FORMATS[fmt]["act"] == "q8_0":
        return q8_0_blocks(xq, xd)
    return q8_K_blocks(xq, xd, xb)


def device():
    return "cuda" if torch.cuda.is_available() else "cpu"


def _stream(t):
    return ctypes_stream(t.device)


def ctypes_stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _need(t, name, dtype, ndim=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise _abi.KompArgumentError(f"{name} is on {t.device}: the decode path runs on a HIP device only")
    if t.dtype != dtype:
        raise _abi.KompArgumentError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise _abi.KompArgumentError(f"{name} must have {ndim} dimensions, got shape {tuple(t.shape)}")


def quantize(fmt, x, bb=4, bsums=False):
    """f32 [M][K] tensor -> (XQ int8 [M][K], XD f32 [M][K/block]) with the q8_0 / q8_K quantizer kernel.

    src/komp/host.py:63-73.  With bsums=True (q8_K only) also returns XB int16 [M][K/16]."""
    act = FORMATS[fmt]["act"]
    _need(x, "x", torch.float32, 2)
    x = x.contiguous()
    m, k = x.shape
    blk = 32 if act == "q8_0" else 256
    if k % blk:
        raise _abi.KompArgumentError(f"quantize {fmt}: K={k} is not a multiple of {blk}")
    xq = torch.empty((m, k), dtype=torch.int8, device=x.device)
    xd = torch.empty((m, k // blk), dtype=torch.float32, device=x.device)
    s = _stream(x)
    with torch.cuda.device(x.device):
        if act == "q8_0":
            if bsums:
                raise _abi.KompArgumentError("bsums are a q8_K field; q8_0 has none")
            _abi.call("komp_quant_q8_0", x.data_ptr(), xq.data_ptr(), xd.data_ptr(), m, k, bb, s)
            return xq, xd
        xb = torch.empty((m, k // 16), dtype=torch.int16, device=x.device) if bsums else None
        _abi.call("komp_quant_q8_K", x.data_ptr(), xq.data_ptr(), xd.data_ptr(), xb.data_ptr() if bsums else None, m,
                  k, s)  # fmt: skip
    return (xq, xd, xb) if bsums else (xq, xd)


def _check_gemv(fmt, wq, ws, xq, xd, n, k):
    """Validate the planes a GEMV reads (the C ABI sees raw pointers and cannot check buffer sizes)."""
    f = FORMATS[fmt]
    _need(wq, "wq", torch.uint8, 2)
    _need(ws, "ws", torch.int16, 2)
    _need(xq, "xq", torch.int8, 2)
    _need(xd, "xd", torch.float32, 2)
    if wq.numel() and wq.stride(1) != 1:
        raise _abi.KompArgumentError("wq rows must be contiguous (stride(1) == 1)")
    nblk = k // f["block"]
    if tuple(ws.shape) != (n, _ws_cols(fmt, nblk)) or not ws.is_contiguous():
        raise _abi.KompArgumentError(f"ws must be a contiguous [{n}][{_ws_cols(fmt, nblk)}] plane, got {tuple(ws.shape)}")
    if wq.shape[0] != n or wq.shape[1] < nblk * f["qbytes"]:
        raise _abi.KompArgumentError(f"wq must be [{n}][>= {nblk * f['qbytes']}], got {tuple(wq.shape)}")
    m = xq.shape[0]
    if tuple(xq.shape) != (m, k) or not xq.is_contiguous():
        raise _abi.KompArgumentError(f"xq must be a contiguous [M][{k}] plane, got {tuple(xq.shape)}")
    if tuple(xd.shape) != (m, nblk) or not xd.is_contiguous():
        raise _abi.KompArgumentError(f"xd must be a contiguous [{m}][{nblk}] plane, got {tuple(xd.shape)}")
    for t, name in ((wq, "wq"), (ws, "ws"), (xd, "xd")):
        if t.device != xq.device:
            raise _abi.KompArgumentError(f"{name} is on {t.device}, xq on {xq.device}")
    return m, nblk


def _launch_gemv(fmt, wq, ws, xq, xd, y, s, n, k, block_n, nb, mode, num_warps):
    if block_n is None:
        block_n, nb, num_warps = 0, 0, 0
    fn = f"komp_{fmt}_gemv"
    with torch.cuda.device(xq.device):
        _abi.call(fn, wq.data_ptr(), ws.data_ptr(), xq.data_ptr(), xd.data_ptr(), y.data_ptr(),
                  None if s is None else s.data_ptr(), xq.shape[0], n, k, wq.stride(0), block_n, nb, mode, num_warps,
                  _stream(xq))  # fmt: skip


def gemv(fmt, wq, ws, xq, xd, n, k, block_n=32, nb=4, mode=0, num_warps=4, store_s=False):
    """-> (Y f32 [M][N], S int32 [M][N][blocks] or None).  mode: 0 bytes, 1 dp4a emulated, 2 dp4a (v_dot4c_i32_i8).

    src/komp/host.py:76-85.  block_n=None lets the library choose block_n, nb and num_warps for the shape."""
    m, nblk = _check_gemv(fmt, wq, ws, xq, xd, n, k)
    y = torch.empty((m, n), dtype=torch.float32, device=xq.device)
    s = torch.zeros(_s_shape(fmt, m, n, nblk), dtype=torch.int32, device=xq.device) if store_s else None
    _launch_gemv(fmt, wq, ws, xq, xd, y, s, n, k, block_n, nb, mode, num_warps)
    return y, s


def _launch_gemm(fmt, wq, ws, xq, xd, y, s, n, k):
    fn = f"komp_{fmt}_gemm"
    with torch.cuda.device(xq.device):
        _abi.call(fn, wq.data_ptr(), ws.data_ptr(), xq.data_ptr(), xd.data_ptr(), y.data_ptr(),
                  None if s is None else s.data_ptr(), xq.shape[0], n, k, wq.stride(0), _stream(xq))  # fmt: skip


def gemm(fmt, wq, ws, xq, xd, n, k, store_s=False):
    """-> (Y f32 [M][N], S int32 [M][N][blocks] or None) on the matrix cores, for any number M of columns.

    The result definition of gemv (exact int32 block dots, then d_w * d_x scaling, src/komp/kernels.py:48-142); the
    weights are read once per 64 columns.  gemv(..., block_n=None, mode=2) runs this kernel from GEMM_MIN_M columns
    on."""
    m, nblk = _check_gemv(fmt, wq, ws, xq, xd, n, k)
    y = torch.empty((m, n), dtype=torch.float32, device=xq.device)
    s = torch.zeros(_s_shape(fmt, m, n, nblk), dtype=torch.int32, device=xq.device) if store_s else None
    _launch_gemm(fmt, wq, ws, xq, xd, y, s, n, k)
    return y, s


def gemm_into(fmt, wq, ws, xq, xd, y, n, k, s=None):
    """Allocation-free gemm into preallocated y f32 [M][N] (and s int32 [M][N][blocks] when given)."""
    m, nblk = _check_gemv(fmt, wq, ws, xq, xd, n, k)
    _need(y, "y", torch.float32, 2)
    if tuple(y.shape) != (m, n) or not y.is_contiguous():
        raise _abi.KompArgumentError(f"gemm_into: y must be a contiguous [{m}][{n}] tensor")
    if s is not None:
        shape = _s_shape(fmt, m, n, nblk)
        _need(s, "s", torch.int32, len(shape))
        if tuple(s.shape) != shape or not s.is_contiguous():
            raise _abi.KompArgumentError(f"gemm_into: s must be a contiguous {list(shape)} tensor")
    _launch_gemm(fmt, wq, ws, xq, xd, y, s, n, k)


def gemm_plan(fmt, m, n, k, sw=None):
    """{rows, cols, waves} per workgroup of the matrix-core GEMM for this shape (sw: the weight row stride in bytes,
    default the packed row), or None when the shape is past the kernel's limits."""
    if sw is None:
        sw = k // FORMATS[fmt]["block"] * FORMATS[fmt]["qbytes"]
    p = _abi.gemm_plan(FMT_ID[fmt], m, n, k, sw)
    return None if p is None else dict(zip(("rows", "cols", "waves"), p))


def uses_gemm(fmt, m, n, k, fused=False, mode=2, sw=None):
    """True when gemv(..., block_n=None) runs the matrix-core GEMM for this shape (unfused, dp4a, from GEMM_MIN_M columns)."""
    return not fused and mode == 2 and m >= GEMM_MIN_M[fmt] and gemm_plan(fmt, m, n, k, sw) is not None


def uses_mfma(fmt, m, n, k, fused=False, mode=2, sw=None):
    """True when gemv(..., block_n=None) (gemv_f32 with fused=True) runs the matrix-core GEMV for this call (TQ2_0,
    dp4a, three columns, more than 8 rows a CU; f32 in from 4 row tiles a CU on): S as the GEMV kernels', Y to f32
    rounding (another order of the f32 sums)."""
    return mfma_plan(fmt, m, n, k, fused, mode, sw) is not None


def mfma_plan(fmt, m, n, k, fused=False, mode=2, sw=None):
    """(rows, waves) per workgroup of the matrix-core GEMV when gemv(..., block_n=None) runs it for this call, else
    None."""
    if sw is None:
        sw = k // FORMATS[fmt]["block"] * FORMATS[fmt]["qbytes"]
    return _abi.gemv_mfma_plan(FMT_ID[fmt], fused, mode, m, n, k, sw)


def quantize_into(fmt, x, xq, xd, xb=None, bb=4):
    """Allocation-free quantize: writes the q8 planes into preallocated xq / xd (and the q8_K bsums into xb).

    For callers that capture HIP graphs or cannot allocate; arguments as quantize()."""
    act = FORMATS[fmt]["act"]
    _need(x, "x", torch.float32, 2)
    _need(xq, "xq", torch.int8, 2)
    _need(xd, "xd", torch.float32, 2)
    if not (x.is_contiguous() and xq.is_contiguous() and xd.is_contiguous()):
        raise _abi.KompArgumentError("quantize_into: x, xq and xd must be contiguous")
    m, k = x.shape
    blk = 32 if act == "q8_0" else 256
    if tuple(xq.shape) != (m, k) or tuple(xd.shape) != (m, k // blk):
        raise _abi.KompArgumentError(f"quantize_into: xq must be [{m}][{k}] and xd [{m}][{k // blk}]")
    with torch.cuda.device(x.device):
        if act == "q8_0":
            _abi.call("komp_quant_q8_0", x.data_ptr(), xq.data_ptr(), xd.data_ptr(), m, k, bb, _stream(x))
        else:
            if xb is not None:
                _need(xb, "xb", torch.int16, 2)
                if tuple(xb.shape) != (m, k // 16) or not xb.is_contiguous():
                    raise _abi.KompArgumentError(f"quantize_into: xb must be a contiguous [{m}][{k // 16}] plane")
            _abi.call("komp_quant_q8_K", x.data_ptr(), xq.data_ptr(), xd.data_ptr(),
                      None if xb is None else xb.data_ptr(), m, k, _stream(x))  # fmt: skip


def gemv_into(fmt, wq, ws, xq, xd, y, n, k, block_n=None, nb=4, mode=2, num_warps=4, s=None):
    """Allocation-free GEMV into preallocated y f32 [M][N] (and s int32 [M][N][blocks] when given).

    For callers that capture HIP graphs or cannot allocate; block_n=None lets the library choose the knobs."""
    m, nblk = _check_gemv(fmt, wq, ws, xq, xd, n, k)
    _need(y, "y", torch.float32, 2)
    if tuple(y.shape) != (m, n) or not y.is_contiguous():
        raise _abi.KompArgumentError(f"gemv_into: y must be a contiguous [{m}][{n}] tensor")
    if s is not None:
        shape = _s_shape(fmt, m, n, nblk)
        _need(s, "s", torch.int32, len(shape))
        if tuple(s.shape) != shape or not s.is_contiguous():
            raise _abi.KompArgumentError(f"gemv_into: s must be a contiguous {list(shape)} tensor")
    _launch_gemv(fmt, wq, ws, xq, xd, y, s, n, k, block_n, nb, mode, num_warps)


def _check_weights(fmt, wq, ws, n, k):
    f = FORMATS[fmt]
    _need(wq, "wq", torch.uint8, 2)
    _need(ws, "ws", torch.int16, 2)
    if wq.numel() and wq.stride(1) != 1:
        raise _abi.KompArgumentError("wq rows must be contiguous (stride(1) == 1)")
    nblk = k // f["block"]
    if tuple(ws.shape) != (n, _ws_cols(fmt, nblk)) or not ws.is_contiguous():
        raise _abi.KompArgumentError(f"ws must be a contiguous [{n}][{_ws_cols(fmt, nblk)}] plane, got {tuple(ws.shape)}")
    if wq.shape[0] != n or wq.shape[1] < nblk * f["qbytes"]:
        raise _abi.KompArgumentError(f"wq must be [{n}][>= {nblk * f['qbytes']}], got {tuple(wq.shape)}")
    return nblk


def gemv_f32_into(fmt, wq, ws, x, y, n, k, block_n=None, nb=4, mode=2, num_warps=4, s=None, xq=None, xd=None,
                  xb=None):  # fmt: skip
    """Quantize-and-GEMV in one launch into preallocated outputs: x f32 [M][K] -> y f32 [M][N] (and s, and the q8
    planes xq / xd / xb when given, as quantize() would return them).  Bit-identical to quantize() then gemv() with
    the same knobs."""
    nblk = _check_weights(fmt, wq, ws, n, k)
    _need(x, "x", torch.float32, 2)
    if x.shape[1] != k or not x.is_contiguous():
        raise _abi.KompArgumentError(f"x must be a contiguous [M][{k}] tensor, got {tuple(x.shape)}")
    m = x.shape[0]
    _need(y, "y", torch.float32, 2)
    if tuple(y.shape) != (m, n) or not y.is_contiguous():
        raise _abi.KompArgumentError(f"y must be a contiguous [{m}][{n}] tensor")
    if s is not None:
        shape = _s_shape(fmt, m, n, nblk)
        _need(s, "s", torch.int32, len(shape))
        if tuple(s.shape) != shape or not s.is_contiguous():
            raise _abi.KompArgumentError(f"s must be a contiguous {list(shape)} tensor")
    ablk = FORMATS[fmt]["block"]
    for t, name, dt, shape in ((xq, "xq", torch.int8, (m, k)), (xd, "xd", torch.float32, (m, k // ablk)),
                               (xb, "xb", torch.int16, (m, k // 16))):  # fmt: skip
        if t is not None:
            _need(t, name, dt, 2)
            if tuple(t.shape) != shape or not t.is_contiguous():
                raise _abi.KompArgumentError(f"{name} must be a contiguous {list(shape)} tensor")
    for t, name in ((wq, "wq"), (ws, "ws"), (y, "y")):
        if t.device != x.device:
            raise _abi.KompArgumentError(f"{name} is on {t.device}, x on {x.device}")
    if block_n is None:
        block_n, nb, num_warps = 0, 0, 0
    fn = f"komp_{fmt}_gemv_f32"
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    planes = (ptr(xq), ptr(xd), ptr(xb)) if fmt in _XB_F32 else (ptr(xq), ptr(xd))  # the others: no XB
    if xb is not None and FORMATS[fmt]["act"] != "q8_K":
        raise _abi.KompArgumentError("xb (bsums) is a q8_K plane; pass None for q8_0 activations")
    with torch.cuda.device(x.device):
        _abi.call(fn, wq.data_ptr(), ws.data_ptr(), x.data_ptr(), y.data_ptr(), ptr(s), *planes, m, n, k, wq.stride(0),
                  block_n, nb, mode, num_warps, _stream(x))  # fmt: skip


def gemv_f32(fmt, wq, ws, x, n, k, block_n=None, nb=4, mode=2, num_warps=4, store_s=False, return_q=False):
    """Quantize-and-GEMV in one launch: x f32 [M][K] -> (Y f32 [M][N], S or None[, (XQ, XD[, XB])]).

    Every workgroup quantizes x (q8_0 for q4_0, q8_K for tq2_0) with the quantizer kernels' arithmetic, so the result
    equals quantize() followed by gemv() with the same knobs bit for bit, with one dispatch instead of two
    (block_n=None plans this launch with auto_config(..., fused=True)).  return_q also returns the q8
    planes (and the q8_K bsums).  No reference counterpart (the reference launches the two kernels separately)."""
    _need(x, "x", torch.float32, 2)
    x = x.contiguous()
    m = x.shape[0]
    blk = FORMATS[fmt]["block"]
    if k % blk:
        raise _abi.KompArgumentError(f"{fmt}: K={k} is not a multiple of {blk}")
    y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    s = torch.zeros(_s_shape(fmt, m, n, k // blk), dtype=torch.int32, device=x.device) if store_s else None
    q = None
    if return_q:
        q = (torch.empty((m, k), dtype=torch.int8, device=x.device),
             torch.empty((m, k // blk), dtype=torch.float32, device=x.device))  # fmt: skip
        if FORMATS[fmt]["act"] == "q8_K":
            q = q + (torch.empty((m, k // 16), dtype=torch.int16, device=x.device),)
    gemv_f32_into(fmt, wq, ws, x, y, n, k, block_n, nb, mode, num_warps, s, *(q or ()))
    return (y, s, q) if return_q else (y, s)


def gemv_multi_into(fmt, mats, ys, k, xq=None, xd=None, x=None, block_n=None, nb=4, mode=2, num_warps=4):
    """Several weight matrices that share one input, in one launch: mats = [(wq, ws, n), ...] (1..4 split planes, as
    gemv takes them), ys = preallocated outputs f32 [M][n] in the same order.  Give xq and xd (q8 planes, as gemv) or
    x (f32 [M][K], quantized inside the launch, as gemv_f32).  With the same knobs each ys[i] equals gemv / gemv_f32
    on matrix i alone, bit for bit; block_n=None plans for the matrices' rows together.  For decoders that store Q, K,
    V (or gate, up) apart: one dispatch, and one quantization per workgroup, instead of one per matrix.  No reference
    counterpart (the reference launches one matrix per kernel)."""
    if not 1 <= len(mats) <= 4 or len(ys) != len(mats):
        raise _abi.KompArgumentError("gemv_multi: 1..4 matrices, one output each")
    if (x is None) == (xq is None or xd is None) or (x is not None and (xq is not None or xd is not None)):
        raise _abi.KompArgumentError("gemv_multi: give either xq and xd (q8 input) or x (f32 input)")
    if x is not None:
        _need(x, "x", torch.float32, 2)
        if x.shape[1] != k or not x.is_contiguous():
            raise _abi.KompArgumentError(f"x must be a contiguous [M][{k}] tensor, got {tuple(x.shape)}")
        ref, m = x, x.shape[0]
        blk = FORMATS[fmt]["block"]
        if k % blk:
            raise _abi.KompArgumentError(f"{fmt}: K={k} is not a multiple of {blk}")
    for i, ((wq, ws, n), y) in enumerate(zip(mats, ys)):
        if x is None:
            m, _ = _check_gemv(fmt, wq, ws, xq, xd, n, k)
            ref = xq
        else:
            _check_weights(fmt, wq, ws, n, k)
        _need(y, f"ys[{i}]", torch.float32, 2)
        if tuple(y.shape) != (m, n) or not y.is_contiguous():
            raise _abi.KompArgumentError(f"ys[{i}] must be a contiguous [{m}][{n}] tensor")
        for t, name in ((wq, "wq"), (ws, "ws"), (y, "y")):
            if t.device != ref.device:
                raise _abi.KompArgumentError(f"matrix {i}: {name} is on {t.device}, the input on {ref.device}")
    if block_n is None:
        block_n, nb, num_warps = 0, 0, 0
    cnt = len(mats)
    P = ctypes.c_void_p * cnt
    I64 = ctypes.c_int64 * cnt
    wqs = P(*(w.data_ptr() for w, _, _ in mats))
    wss = P(*(s.data_ptr() for _, s, _ in mats))
    yps = P(*(y.data_ptr() for y in ys))
    ns = I64(*(n for _, _, n in mats))
    sws = I64(*(w.stride(0) for w, _, _ in mats))
    fn = f"komp_{fmt}_gemv_multi"
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    with torch.cuda.device(ref.device):
        _abi.call(fn, cnt, wqs, wss, yps, ns, sws, ptr(xq), ptr(xd), ptr(x), m, k, block_n, nb, mode, num_warps,
                  _stream(ref))  # fmt: skip


def gemv_multi(fmt, mats, k, xq=None, xd=None, x=None, block_n=None, nb=4, mode=2, num_warps=4):
    """-> [Y f32 [M][n] per matrix]; arguments as gemv_multi_into."""
    ref = x if x is not None else xq
    if ref is None:
        raise _abi.KompArgumentError("gemv_multi: give either xq and xd (q8 input) or x (f32 input)")
    ys = [torch.empty((ref.shape[0], n), dtype=torch.float32, device=ref.device) for _, _, n in mats]
    gemv_multi_into(fmt, mats, ys, k, xq, xd, x, block_n, nb, mode, num_warps)
    return ys


def auto_config(fmt, m, n, k, fused=False, mode=2):
    """(block_n, nb, num_warps) of the plan gemv(..., block_n=None, mode=mode) uses for this shape on the current
    device (gemv_f32 with fused=True).  Passed back as explicit knobs it reproduces the plan only when it is a knob
    set and auto_plan() reports the lanes_per_row and passes that the knob mapping gives."""
    return _abi.auto_config(FMT_ID[fmt], m, n, k, fused, mode)


def auto_plan(fmt, m, n, k, fused=False, mode=2):
    """The plan gemv(..., block_n=None) uses: rows per workgroup, nb, waves, lanes per row, passes per wave."""
    keys = ("block_n", "nb", "waves", "lanes_per_row", "passes")
    return dict(zip(keys, _abi.auto_plan(FMT_ID[fmt], m, n, k, fused, mode)))


def knob_equivalent(fmt, m, n, k, fused=False, mode=2):
    """The explicit knobs that run exactly the auto plan, or None when the plan is beyond the knob mapping (or the
    shape runs on the matrix-core GEMM)."""
    if uses_gemm(fmt, m, n, k, fused, mode):
        return None
    p = auto_plan(fmt, m, n, k, fused, mode)
    bn, w = p["block_n"], p["waves"]
    if bn not in (8, 16, 32, 64, 128) or w not in (1, 2, 4, 8) or bn % w:
        return None
    rpw = bn // w
    if p["lanes_per_row"] != 64 // min(rpw, 16) or p["passes"] != rpw // min(rpw, 16):
        return None
    return bn, p["nb"], w


def dp4a_probe(a, b, c, mode=2):
    """OUT[i] = dp4a(a[i], b[i], c[i]) on the device (kernels.dp4a_probe, src/komp/kernels.py:145-149)."""
    for t, name in ((a, "a"), (b, "b"), (c, "c")):
        _need(t, name, torch.int32, 1)
    a, b, c = a.contiguous(), b.contiguous(), c.contiguous()
    out = torch.empty_like(a)
    with torch.cuda.device(a.device):
        _abi.call("komp_dp4a_probe", a.data_ptr(), b.data_ptr(), c.data_ptr(), out.data_ptr(), a.numel(), mode,
                  _stream(a))  # fmt: skip
    return out


def stream_read_words(nbytes):
    """Words komp_stream_read writes for nbytes: one per wave, a wave reading 64 lanes x 4 x 16 = 4096 bytes."""
    return 8 * -(-nbytes // 32768)


def stream_read_into(src, nbytes, out):
    """Read the first nbytes of the contiguous device tensor src once with the streaming-read probe (one launch) and
    write each wave's XOR of its dwords to out (uint32 viewed as int32, stream_read_words(nbytes) words): the cost of
    moving the bytes alone, which bench.py sets beside each GEMV over as many bytes.  Beyond the reference."""
    if not src.is_cuda or not src.is_contiguous() or src.numel() * src.element_size() < nbytes:
        raise _abi.KompArgumentError("src must be a contiguous device tensor of at least nbytes bytes")
    _need(out, "out", torch.int32, 1)
    if out.numel() < stream_read_words(nbytes):
        raise _abi.KompArgumentError(f"out needs {stream_read_words(nbytes)} words")
    with torch.cuda.device(src.device):
        _abi.call("komp_stream_read", src.data_ptr(), nbytes, out.data_ptr(), _stream(src))


def stream_read(src):
    """stream_read_into over all of src (its byte count a multiple of 16); returns the per-wave XOR words."""
    nbytes = src.numel() * src.element_size()
    out = torch.empty(stream_read_words(nbytes), dtype=torch.int32, device=src.device)
    stream_read_into(src, nbytes, out)
    return out


def q4_0_decode(wq):
    """[R][16] q4_0 quant bytes -> [R][32] int32 values (kernels.q4_0_decode, src/komp/kernels.py:152-157)."""
    _need(wq, "wq", torch.uint8, 2)
    wq = wq.contiguous()
    r = wq.shape[0]
    out = torch.empty((r, 32), dtype=torch.int32, device=wq.device)
    with torch.cuda.device(wq.device):
        _abi.call("komp_q4_0_decode", wq.data_ptr(), out.data_ptr(), r, _stream(wq))
    return out


def tq2_0_decode(wq):
    """[NBLK][64] tq2_0 quant bytes -> [NBLK][256] int32 values (kernels.tq2_0_decode, src/komp/kernels.py:160-170)."""
    _need(wq, "wq", torch.uint8, 2)
    wq = wq.contiguous()
    nblk = wq.shape[0]
    out = torch.empty((nblk, 256), dtype=torch.int32, device=wq.device)
    with torch.cuda.device(wq.device):
        _abi.call("komp_tq2_0_decode", wq.data_ptr(), out.data_ptr(), nblk, _stream(wq))
    return out
