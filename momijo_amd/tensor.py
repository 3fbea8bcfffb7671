"""Host-side mirror of momijo's tensor-engine operator surface on MI355X.

``Tensor`` keeps the reference's ``Tensor[T]`` contract (shape, strides,
zero-copy transpose views; tensor/tensor.mojo:776-905) with its storage in
HBM.  Device memory and streams come from PyTorch-ROCm (plumbing only); every
arithmetic op goes through the C ABI of ``libmomijo_hip.so``.

Error behaviour follows the reference: ``matmul`` of incompatible ranks or
shapes returns an empty tensor (tensor/broadcast.mojo:1613-1616,1677-1684).
Device failures raise :class:`momijo_amd._lib.MomijoHipError`: unlike the
reference's launchers (tensor/gpu/runtime.mojo:608-631) there is no silent
CPU fallback.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np
import torch

from . import _lib

_DTYPES = {
    "float32": torch.float32,
    "float64": torch.float64,
    "bfloat16": torch.bfloat16,
    "int8": torch.int8,
    "int32": torch.int32,
}


def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def gpu_available() -> bool:
    """gpu_available() (tensor/gpu/runtime.mojo:29-36): a gfx950 device and
    the backend library are both present."""
    try:
        return _lib.device_available()
    except ImportError:
        return False


class Tensor:
    """A device tensor with momijo's shape/stride semantics."""

    __slots__ = ("_t",)

    def __init__(self, data, shape: Sequence[int] | None = None, dtype: str | None = None):
        if isinstance(data, Tensor):
            t = data._t
        elif isinstance(data, torch.Tensor):
            t = data
        else:
            arr = np.asarray(data)
            if dtype == "bfloat16":
                t = torch.from_numpy(np.ascontiguousarray(arr, np.float32)).to(torch.bfloat16)
            else:
                t = torch.from_numpy(np.ascontiguousarray(arr))
        if dtype is not None and t.dtype != _DTYPES[dtype]:
            t = t.to(_DTYPES[dtype])
        if shape is not None:
            t = t.reshape(list(shape))
        if t.device.type != "cuda":
            t = t.to(_device())
        self._t = t

    # ---------------------------------------------------------------- info
    @property
    def torch(self) -> torch.Tensor:
        return self._t

    def shape(self) -> list[int]:
        return list(self._t.shape)

    def strides(self) -> list[int]:
        return list(self._t.stride())

    def numel(self) -> int:
        return self._t.numel()

    @property
    def dtype(self) -> torch.dtype:
        return self._t.dtype

    def numpy(self) -> np.ndarray:
        t = self._t
        if t.dtype == torch.bfloat16:
            t = t.float()
        return t.detach().cpu().numpy()

    def copy(self) -> "Tensor":
        return Tensor(self._t.clone())

    def contiguous(self) -> "Tensor":
        return Tensor(self._t.contiguous())

    # ---------------------------------------------------------------- views
    def transpose(self) -> "Tensor":
        """Swap the last two axes as a zero-copy stride view
        (tensor/tensor.mojo:2677-2679 -> tensor/transform.mojo:2132,2107-2125)."""
        if self._t.dim() <= 1:
            return self.copy()
        return Tensor(self._t.transpose(-2, -1))

    # ---------------------------------------------------------------- matmul
    def matmul(self, other: "Tensor") -> "Tensor":
        """Tensor.matmul (tensor/tensor.mojo:3168-3169)."""
        return matmul(self, other)

    def matmul_vec(self, x: "Tensor") -> "Tensor":
        """Tensor.matmul_vec (tensor/tensor.mojo:3167-3181); Tensor[Int]
        operands are upcast to Float32 first (:3174-3178)."""
        a, v = _upcast_int_pair(self, x)
        if a._t.dim() != 2 or v._t.dim() != 1 or v._t.shape[0] != a._t.shape[1]:
            return empty_f64() if a._t.dtype == torch.float64 else empty_f32()
        return _matvec(a, v)

    # ---------------------------------------------------------------- unary
    def _unary(self, epi: int) -> "Tensor":
        if self._t.dtype != torch.float32:
            raise TypeError("activations are defined for Float32 tensors")
        src = self._t.contiguous()
        out = torch.empty_like(src)
        _lib.call("mj_activation_f32", epi, _ptr(src), _ptr(out), src.numel(), _stream())
        return Tensor(out)

    def relu(self) -> "Tensor":
        """Tensor.relu -> apply_unary op 8 (tensor/math.mojo:582-585)."""
        return self._unary(_lib.EPI_RELU_UNARY)

    def gelu(self) -> "Tensor":
        """Tensor.gelu -> gelu32 (tensor/math.mojo:288-295); finite where the
        reference's tanh32 overflows (x > ~10.06)."""
        return self._unary(_lib.EPI_GELU_TANH)

    def silu(self) -> "Tensor":
        """Tensor.silu -> silu32 (tensor/math.mojo:283-285)."""
        return self._unary(_lib.EPI_SILU)

    def maximum_scalar(self, s: float) -> "Tensor":
        """Tensor[Float32].maximum_scalar(s) = where_f32(ge_t(self, s), self, s)
        (tensor/tensor.mojo:4232): x where x >= s, else s, so -0 stays -0 at
        s = 0 and NaN becomes s.  Converted.forward applies it with s = 0
        between the quantized layers (learn/api/sequential.mojo:423)."""
        if self._t.dtype != torch.float32:
            raise TypeError("maximum_scalar is provided for Float32 tensors")
        src = self._t.contiguous()
        out = torch.empty_like(src)
        _lib.call("mj_maximum_scalar_f32", _ptr(src), float(np.float32(s)), _ptr(out),
                  src.numel(), _stream())
        return Tensor(out)

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape()}, dtype={self._t.dtype})"


def empty_f32() -> Tensor:
    """empty_f32(): the reference's result for an unsupported matmul."""
    return Tensor(torch.empty(0, dtype=torch.float32, device=_device()))


def empty_f64() -> Tensor:
    """empty_f64(): the reference's result for an unsupported Float64 matmul."""
    return Tensor(torch.empty(0, dtype=torch.float64, device=_device()))


_INT_DTYPES = (torch.int64, torch.int32)


def astype_f32_from_int(t: torch.Tensor) -> torch.Tensor:
    """astype_f32_from_int (tensor/cast.mojo:5431-5437): Float32(Int) of every
    element, rounded to nearest even, by the library's cast kernel.  The
    reference walks its flat storage in order; a view is taken in logical
    (row-major) order here, as its shape says."""
    src = t.to(torch.int64).contiguous()
    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    _lib.call("mj_cast_i64_f32", _ptr(src), _ptr(out), src.numel(), _stream())
    return out


def _upcast_int_pair(A: Tensor, B: Tensor) -> tuple[Tensor, Tensor]:
    """Tensor[Int] @ Tensor[Int] -> Float32: both operands are converted with
    astype_f32_from_int (tensor/tensor.mojo:3161-3165, 3174-3178), then the
    Float32 product runs.  Other dtypes pass through."""
    if A._t.dtype in _INT_DTYPES and B._t.dtype in _INT_DTYPES:
        return Tensor(astype_f32_from_int(A._t)), Tensor(astype_f32_from_int(B._t))
    return A, B


def _matvec(A: Tensor, x: Tensor) -> Tensor:
    a, v = A._t, x._t
    M, N = a.shape
    fn = "mj_matvec_f64" if a.dtype == torch.float64 else "mj_matvec_f32"
    y = torch.empty(M, dtype=a.dtype, device=a.device)
    _lib.call(fn, M, N, _ptr(a), a.stride(0), a.stride(1), _ptr(v), v.stride(0), _ptr(y),
              _stream())
    return Tensor(y)


def matmul(A: Tensor, B: Tensor) -> Tensor:
    """tensor.matmul (tensor/broadcast.mojo:1677-1684): rank 2 x 1 is a matrix-
    vector product, 2 x 2 a matrix product, anything else an empty tensor.

    Float32 operands run the fp32 engine with their strides (transposed views
    need no copy).  bfloat16 operands run the bf16 MFMA GEMM, which takes B as
    the transpose view of a row-major [N, K] weight (x.matmul(W.transpose())).
    Tensor[Int] operands are upcast to Float32 (tensor/tensor.mojo:3161-3165)."""
    A, B = _upcast_int_pair(A, B)
    a, b = A._t, B._t
    empty = empty_f64 if a.dtype == torch.float64 else empty_f32
    if a.dim() == 2 and b.dim() == 1:
        if a.dtype not in (torch.float32, torch.float64) or b.dtype != a.dtype \
                or b.shape[0] != a.shape[1]:
            return empty()
        return _matvec(A, B)
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        return empty()
    M, K = a.shape
    N = b.shape[1]
    if a.dtype == torch.float64 and b.dtype == torch.float64:
        c = torch.empty((M, N), dtype=torch.float64, device=a.device)
        _lib.call("mj_matmul_f64", M, N, K, _ptr(a), a.stride(0), a.stride(1), _ptr(b),
                  b.stride(0), b.stride(1), _ptr(c), N, _stream())
        return Tensor(c)
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        c = torch.empty((M, N), dtype=torch.float32, device=a.device)
        _lib.call("mj_matmul_f32", M, N, K, _ptr(a), a.stride(0), a.stride(1), _ptr(b),
                  b.stride(0), b.stride(1), None, _lib.EPI_NONE, _ptr(c), N, _stream())
        return Tensor(c)
    if a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16:
        if a.stride(1) != 1 or b.stride(0) != 1:
            raise NotImplementedError(
                "bf16 matmul takes A row-major and B as W.transpose() of a row-major W")
        c = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
        _lib.call("mj_gemm_bf16_nt", M, N, K, _ptr(a), a.stride(0), _ptr(b), b.stride(1), None,
                  _lib.EPI_NONE, _ptr(c), N, _stream())
        return Tensor(c)
    raise TypeError(f"matmul of {a.dtype} and {b.dtype} is not supported")


def matmul2d(a: Tensor, b: Tensor) -> Tensor:
    """matmul2d (tensor/math.mojo:7838-7880): Float64 [m,k] @ [k,n]; bad ranks
    or inner dimensions give zeros([m, n]) as the reference does.  Operands are
    read through their strides; the reference indexes the raw buffer as if
    row-major, which agrees for the contiguous tensors it is called with."""
    at, bt = a._t, b._t
    m = at.shape[0] if at.dim() == 2 else 0
    n = bt.shape[1] if bt.dim() == 2 else 0
    if at.dim() != 2 or bt.dim() != 2 or at.shape[1] != bt.shape[0]:
        return Tensor(torch.zeros((m, n), dtype=torch.float64, device=at.device))
    return matmul(Tensor(at.to(torch.float64)), Tensor(bt.to(torch.float64)))


def matmul_backward(a: Tensor, b: Tensor, g: Tensor, grad_a: Tensor | None = None,
                    grad_b: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """The autograd MATMUL2D rule (tensor/autograd.mojo:1542-1555) for y = a @ b
    in Float64: returns (grad_a + g @ b^T, grad_b + a^T @ g), each sum starting
    from zero where no gradient is given (a fresh tape slot)."""
    at, bt, gt = (t.torch.to(torch.float64).contiguous() for t in (a, b, g))
    M, K = at.shape
    N = bt.shape[1]
    if bt.shape[0] != K or tuple(gt.shape) != (M, N):
        raise ValueError("matmul_backward: a [M,K], b [K,N], g [M,N] expected")
    outs = []
    for grad, shape, which in ((grad_a, (M, K), 0), (grad_b, (K, N), 1)):
        if grad is not None:
            o = grad.torch.to(torch.float64).contiguous().clone()
            if tuple(o.shape) != shape:
                raise ValueError("gradient shape mismatch")
        else:
            o = torch.empty(shape, dtype=torch.float64, device=at.device)
        _lib.call("mj_matmul_backward_f64", M, N, K, _ptr(at), _ptr(bt), _ptr(gt),
                  _ptr(o) if which == 0 else None, _ptr(o) if which == 1 else None,
                  int(grad is not None), _stream())
        outs.append(Tensor(o))
    return outs[0], outs[1]


def tensordot(A: Tensor, B: Tensor, axes: int = 1) -> Tensor:
    """tensordot (tensor/broadcast.mojo:1694-1900) for Float32, axes = 1:
    A (..., M, K) with B (..., K, N) -> (batch..., M, N), the batch dimensions
    broadcasting against each other.  Unsupported axes, ranks below 2, a K
    mismatch or non-broadcastable batches give an empty tensor."""
    a, b = A._t, B._t
    if axes != 1 or a.dim() < 2 or b.dim() < 2:
        return empty_f32()
    M, K = a.shape[-2:]
    Kb, N = b.shape[-2:]
    if K != Kb:
        return empty_f32()
    try:
        batch = tuple(torch.broadcast_shapes(a.shape[:-2], b.shape[:-2]))
    except RuntimeError:
        return empty_f32()
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise TypeError("tensordot is defined for Float32 tensors")
    if len(batch) > 5:
        return empty_f32()   # the reference's generic path nests at most 5 batch loops
    ae = a.expand(batch + (M, K))   # broadcast dims get stride 0
    be = b.expand(batch + (K, N))
    out = torch.empty(batch + (M, N), dtype=torch.float32, device=a.device)
    r = len(batch)
    arr = ctypes.c_int64 * max(r, 1)
    shape = arr(*batch) if r else None
    sa = arr(*ae.stride()[:r]) if r else None
    sb = arr(*be.stride()[:r]) if r else None
    _lib.call("mj_tensordot_f32", r, shape, sa, sb, M, N, K, _ptr(ae), ae.stride(-2),
              ae.stride(-1), _ptr(be), be.stride(-2), be.stride(-1), _ptr(out), _stream())
    return Tensor(out)


def gemm_bf16_nt(A: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None = None,
                 epi: int = _lib.EPI_NONE, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = bf16(epi(A @ W^T + bias)) for bf16 device tensors A [M,K], W [N,K]
    with unit column stride (row strides are passed as leading dimensions)."""
    if A.dtype != torch.bfloat16 or W.dtype != torch.bfloat16:
        raise TypeError(f"gemm_bf16_nt takes bfloat16 A and W, got {A.dtype} and {W.dtype}")
    if A.dim() != 2 or W.dim() != 2 or A.shape[1] != W.shape[1]:
        raise ValueError(f"gemm_bf16_nt: A [M,K] and W [N,K] expected, got {list(A.shape)} "
                         f"and {list(W.shape)}")
    if A.stride(1) != 1 or W.stride(1) != 1:
        raise ValueError("gemm_bf16_nt: A and W need unit column stride")
    M, K = A.shape
    N = W.shape[0]
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != N):
        raise ValueError(f"gemm_bf16_nt: bias must be float32 with {N} elements")
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"gemm_bf16_nt: out must be bfloat16 [{M}, {N}] with unit column "
                         "stride")
    _lib.call("mj_gemm_bf16_nt", M, N, K, _ptr(A), A.stride(0), _ptr(W), W.stride(0), _ptr(bias),
              epi, _ptr(out), out.stride(0), _stream())
    return out
