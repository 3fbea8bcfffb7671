"""The reference's device seam on this backend: ``launch_1d_linear_fw`` and
its backward siblings (tensor/gpu/runtime.mojo:504-903), and
``launch_1d_conv2d_fw`` (:360-470), with their exact argument lists and
their contract.

The reference launchers take host buffers (``List[Float32]``), the number of
logical threads, a block size and a ``kernel`` -- a CPU function of the
thread id (the ``Kernel1D_*`` aliases, runtime.mojo:504-535).  When a GPU is
available they run the operation on it; any failure there is swallowed and
the same work is done by calling ``kernel(tid, ...)`` for every thread id in
blocks of ``block_size`` (runtime.mojo:608-631).  They never raise.

Here the GPU path is the host-pointer C ABI of ``libmomijo_hip.so``
(``mj_launch_linear_fw_h`` and siblings: copy in, run, copy out).  A non-OK
status, or no gfx950 device, leads to the caller's kernel exactly as in the
reference; ``strict=True`` raises :class:`momijo_amd._lib.MomijoHipError`
instead.  The library itself must load: a missing extension raises
``ImportError`` (the kernel is the caller's fallback for a failed device
call, not a substitute for the backend).  Each launcher returns which path
ran ("gpu" or "cpu"); the reference returns nothing.

Host buffers are numpy float32 arrays (the stand-in for ``List[Float32]``);
the output buffer is written in place.  The fallback passes the caller's
objects to ``kernel`` unchanged.
"""
from __future__ import annotations

from typing import Callable

import numpy as np

from . import _lib

# Kernel1D_LinearFW (runtime.mojo:504-512): kernel(tid, x, wT, b, y, N, InF, OutF, has_bias)
Kernel1D_LinearFW = Callable[..., None]
# Kernel1D_LinearBW_DX / _DW (runtime.mojo:514-528): kernel(tid, dy, w|x, out, N, InF, OutF)
Kernel1D_LinearBW_DX = Callable[..., None]
Kernel1D_LinearBW_DW = Callable[..., None]
# Kernel1D_LinearBW_DB (runtime.mojo:530-535): kernel(tid, dy, db, N, OutF)
Kernel1D_LinearBW_DB = Callable[..., None]
# Kernel1D_Conv2DFW (runtime.mojo:360-374): kernel(tid, x, w, b, y, N, C, H, W, OH, OW, OC,
# kH, kW, sH, sW, pH, pW, has_bias)
Kernel1D_Conv2DFW = Callable[..., None]


def gpu_available() -> bool:
    """gpu_available() (runtime.mojo:29-36) for this backend: the library
    reports a gfx950 device.  Raises ImportError if the library is missing."""
    return bool(_lib.load().mj_device_available())


def _host_in(a, n: int, name: str) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))
    if arr.size < n:
        raise ValueError(f"{name} holds {arr.size} elements, {n} needed")
    return arr


def _host_out(a, n: int, name: str) -> np.ndarray:
    if not (isinstance(a, np.ndarray) and a.dtype == np.float32 and a.flags.c_contiguous
            and a.flags.writeable):
        raise TypeError(f"{name} must be a writable C-contiguous float32 numpy array "
                        "(written in place, as the reference's mut List[Float32])")
    if a.size < n:
        raise ValueError(f"{name} holds {a.size} elements, {n} needed")
    return a


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def _device_call(fn: str, strict: bool, *args) -> bool:
    """True when the device path completed; False sends the caller to its
    kernel (or raises in strict mode)."""
    lib = _lib.load()
    if not lib.mj_device_available():
        if strict:
            raise _lib.MomijoHipError(_lib.MJ_ERR_NO_DEVICE, fn, "no gfx950 device")
        return False
    st = getattr(lib, fn)(*args)
    if st == _lib.MJ_OK:
        return True
    if strict:
        _lib.check(st, fn)
    return False


def _cpu_fallback(total_threads: int, block_size: int, call) -> None:
    """The reference's fallback loop (runtime.mojo:612-631): thread ids in
    blocks of block_size (256 when block_size <= 0)."""
    if total_threads <= 0:
        return
    bs = block_size if block_size > 0 else 256
    blocks = (total_threads + bs - 1) // bs
    for blk in range(blocks):
        base = blk * bs
        for t in range(bs):
            tid = base + t
            if tid < total_threads:
                call(tid)


def launch_1d_linear_fw(total_threads: int, block_size: int, kernel: Kernel1D_LinearFW,
                        x, wT, b, y: np.ndarray, N: int, InF: int, OutF: int,
                        has_bias: bool, *, strict: bool = False) -> str:
    """launch_1d_linear_fw (runtime.mojo:539-631): y[n,o] = sum_k x[n,k]
    wT[k,o] (+ b[o]) with x [N,InF], wT [InF,OutF], y [N,OutF].  The bias is
    added when has_bias and len(b) == OutF, the rule of the seam's CPU kernel
    (layers.mojo:472-473)."""
    if N * OutF <= 0 and gpu_available():
        return "gpu"   # the reference's GPU path returns here (runtime.mojo:557-559)
    hx = _host_in(x, N * InF, "x")
    hw = _host_in(wT, InF * OutF, "wT")
    bias = has_bias and len(b) == OutF
    hb = _host_in(b, OutF, "b") if bias else None
    hy = _host_out(y, N * OutF, "y")
    if _device_call("mj_launch_linear_fw_h", strict, _ptr(hx), _ptr(hw), _ptr(hb), _ptr(hy),
                    N, InF, OutF, int(bias)):
        return "gpu"
    _cpu_fallback(total_threads, block_size,
                  lambda tid: kernel(tid, x, wT, b, y, N, InF, OutF, has_bias))
    return "cpu"


def launch_1d_linear_bw_dx(total_threads: int, block_size: int, kernel: Kernel1D_LinearBW_DX,
                           dy, w, dx: np.ndarray, N: int, InF: int, OutF: int, *,
                           strict: bool = False) -> str:
    """launch_1d_linear_bw_dx (runtime.mojo:636-713): dx [N,InF] = dy [N,OutF]
    . w [OutF,InF], the layout of the seam's CPU kernel (layers.mojo:624-650)."""
    if N * InF <= 0 and gpu_available():
        return "gpu"
    hdy = _host_in(dy, N * OutF, "dy")
    hw = _host_in(w, OutF * InF, "w")
    hdx = _host_out(dx, N * InF, "dx")
    if _device_call("mj_launch_linear_bw_dx_h", strict, _ptr(hdy), _ptr(hw), _ptr(hdx),
                    N, InF, OutF):
        return "gpu"
    _cpu_fallback(total_threads, block_size,
                  lambda tid: kernel(tid, dy, w, dx, N, InF, OutF))
    return "cpu"


def launch_1d_linear_bw_dw(total_threads: int, block_size: int, kernel: Kernel1D_LinearBW_DW,
                           dy, x, dW: np.ndarray, N: int, InF: int, OutF: int, *,
                           strict: bool = False) -> str:
    """launch_1d_linear_bw_dw (runtime.mojo:714-832): dW [OutF,InF] =
    dy^T . x (layers.mojo:651-690)."""
    if InF * OutF <= 0 and gpu_available():
        return "gpu"
    hdy = _host_in(dy, N * OutF, "dy")
    hx = _host_in(x, N * InF, "x")
    hdw = _host_out(dW, OutF * InF, "dW")
    if _device_call("mj_launch_linear_bw_dw_h", strict, _ptr(hdy), _ptr(hx), _ptr(hdw),
                    N, InF, OutF):
        return "gpu"
    _cpu_fallback(total_threads, block_size,
                  lambda tid: kernel(tid, dy, x, dW, N, InF, OutF))
    return "cpu"


def launch_1d_linear_bw_db(total_threads: int, block_size: int, kernel: Kernel1D_LinearBW_DB,
                           dy, db: np.ndarray, N: int, OutF: int, *,
                           strict: bool = False) -> str:
    """launch_1d_linear_bw_db (runtime.mojo:834-903): db[o] = sum_n dy[n,o]
    (layers.mojo:691-729)."""
    if OutF <= 0 and gpu_available():
        return "gpu"
    hdy = _host_in(dy, N * OutF, "dy")
    hdb = _host_out(db, OutF, "db")
    if _device_call("mj_launch_linear_bw_db_h", strict, _ptr(hdy), _ptr(hdb), N, OutF):
        return "gpu"
    _cpu_fallback(total_threads, block_size, lambda tid: kernel(tid, dy, db, N, OutF))
    return "cpu"


def launch_1d_conv2d_fw(total_threads: int, block_size: int, kernel: Kernel1D_Conv2DFW,
                        x, w, b, y: np.ndarray, N: int, C: int, H: int, W: int, OH: int,
                        OW: int, OC: int, kH: int, kW: int, sH: int, sW: int, pH: int, pW: int,
                        has_bias: bool, *, strict: bool = False) -> str:
    """launch_1d_conv2d_fw (runtime.mojo:376-470): y [N,OC,OH,OW] = conv2d of
    x [N,C,H,W] with w [OC,C,kH,kW] (+ b[oc] when has_bias), NCHW, zero
    padding.  Nothing to compute (N OC OH OW <= 0) returns at once, as the
    reference's GPU path does (:398-400)."""
    total = N * OC * OH * OW
    if total <= 0 and gpu_available():
        return "gpu"
    hx = _host_in(x, N * C * H * W, "x")
    hw = _host_in(w, OC * C * kH * kW, "w")
    hb = _host_in(b, OC, "b") if has_bias else None
    hy = _host_out(y, max(total, 0), "y")
    if _device_call("mj_launch_conv2d_fw_h", strict, _ptr(hx), _ptr(hw), _ptr(hb), _ptr(hy), N,
                    C, H, W, OH, OW, OC, kH, kW, sH, sW, pH, pW, int(bool(has_bias))):
        return "gpu"
    _cpu_fallback(total_threads, block_size,
                  lambda tid: kernel(tid, x, w, b, y, N, C, H, W, OH, OW, OC, kH, kW, sH, sW,
                                     pH, pW, has_bias))
    return "cpu"


__all__ = ["gpu_available", "launch_1d_linear_fw", "launch_1d_linear_bw_dx",
           "launch_1d_linear_bw_dw", "launch_1d_linear_bw_db", "launch_1d_conv2d_fw",
           "Kernel1D_LinearFW", "Kernel1D_LinearBW_DX", "Kernel1D_LinearBW_DW",
           "Kernel1D_LinearBW_DB", "Kernel1D_Conv2DFW"]
