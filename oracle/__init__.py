"""CPU oracle for momijo's tensor-engine hot path (TEST INFRASTRUCTURE ONLY).

The C restatement lives in ``momijo_oracle.c``; this module loads it with
ctypes and wraps each entry point for numpy arrays.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package; the product (``momijo_amd``) never does.

Parity status of each restated function (how it is pinned, see
``tests/test_oracle_*.py``):

* rng words / randu / randn (creation.mojo:57-131,495-578): pinned by an
  independent numpy restatement of Vigna's splitmix64/xoroshiro128** and by
  committed golden words.  The last-ulp behaviour of Mojo's ``log/cos/sin``
  inside Box-Muller and of ``Float32(UInt64)`` is **parity unpinned** (no Mojo
  toolchain exists here and the reference ships no vectors).
* matmul_f32 / matvec_f32 / linear_fw_f32 / kernel_linear_fw_f32: pinned by
  integer-valued inputs (exact in any order), identity/permutation closed
  forms, and fp64 brute force within K*2^-24*sum|a||b|.  Mojo's FMA
  contraction choice is **parity unpinned** at the last ulp.
* relu / gelu32 / silu32 / sigmoid32 / tanh32: closed forms against libm in
  double.  The Mojo stdlib ``exp`` ulp behaviour is **parity unpinned**.
* maximum_scalar_f32: the -0 / NaN / equal-to-s cases against the mask rule
  x >= s written out, plus numpy's fmax away from those cases.
* conv2d_fw_f32: integer-valued inputs whose sums are exact (against an int64
  restatement with explicit zero padding), the 1 x 1 / stride-1 case against
  the pinned matmul, delta kernels (shifted copies of x, padding zeros),
  valid-tap clipping against the strict-order float32 loop written out, and
  torch's CPU conv2d within the fp32 summation bound.
* astype_f32_from_int: integers above 2^24 with exact ties (2^24 + 1 -> 2^24,
  2^24 + 3 -> 2^24 + 4), 2^63 - 1, negatives, and numpy's int64 -> float32
  cast (round to nearest even) on random 64-bit integers.
* _exp_approx family: exact IEEE op sequence, pinned against a numpy float32
  restatement.
* quantize_symmetric_int8 / matmul_i8_i8_to_i32 / dequantize / minmax scale:
  pinned by constructed ties, the fp32-add artifact, zero rows, clamps and
  int32 brute force.
* quantize_rowwise_rhe / linear_w8a16 / linear_w8a8 / gemm_bf16_nt /
  mlp_w8a16: spec-only (momijo has no such op); pinned by closed forms (exact
  ties, small-integer inputs that make every sum exact, power-of-two scales
  that make the W8A8 epilogue exact) and by torch CPU cross-checks.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmomijo_oracle.so")

EPI_NONE, EPI_RELU, EPI_GELU_TANH, EPI_SILU = 0, 1, 2, 3
EPI_GELU_TANH_APPROX, EPI_SILU_APPROX, EPI_RELU_UNARY = 4, 5, 6


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -O2 -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
        subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float
_D = ctypes.c_double
_I = ctypes.c_int
_U64 = ctypes.c_uint64


def _declare(L):
    sig = {
        "mo_rng_words": (None, [_U64, _P, _I64]),
        "mo_rng_words_from_state": (None, [_U64, _U64, _P, _I64]),
        "mo_randu_f32": (None, [_P, _I64, _D, _D, _U64]),
        "mo_randn_f32": (None, [_P, _I64, _D, _D, _U64]),
        "mo_randn_f32_f32core": (None, [_P, _I64, _U64]),
        "mo_f32_to_bf16_n": (None, [_P, _P, _I64]),
        "mo_bf16_to_f32_n": (None, [_P, _P, _I64]),
        "mo_matmul_f32": (None, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64]),
        "mo_matvec_f32": (None, [_P, _I64, _I64, _P, _I64, _P, _I64, _I64]),
        "mo_linear_fw_f32": (None, [_P, _P, _P, _I, _P, _I64, _I64, _I64]),
        "mo_kernel_linear_fw_f32": (None, [_P, _P, _P, _I, _P, _I64, _I64, _I64]),
        "mo_linear_act_f32": (None, [_P, _P, _P, _I, _I, _P, _I64, _I64, _I64]),
        "mo_epilogue32_n": (None, [_I, _P, _P, _I64]),
        "mo_gelu32_n": (None, [_P, _P, _I64]),
        "mo_maximum_scalar32_n": (None, [_P, _F, _P, _I64]),
        "mo_astype_f32_from_int": (None, [_P, _P, _I64]),
        "mo_exp_approx32": (_F, [_F]),
        "mo_tanh_approx32": (_F, [_F]),
        "mo_quant_legacy_one": (ctypes.c_int8, [_F, _F]),
        "mo_quantize_symmetric_int8": (None, [_P, _I64, _F, _P]),
        "mo_matmul_i8_i8_to_i32": (None, [_P, _P, _P, _I64, _I64, _I64, _I]),
        "mo_dequant_i32_bias": (None, [_P, _F, _P, _P, _I64, _I64]),
        "mo_minmax_scale_symmetric": (_F, [_P, _I64, _F]),
        "mo_quant_linear_fw": (None, [_P, _P, _P, _F, _F, _P, _P, _P, _I64, _I64, _I64, _I]),
        "mo_quantize_rowwise_rhe": (None, [_P, _I64, _I64, _P, _P]),
        "mo_quantize_rowwise_legacy": (None, [_P, _I64, _I64, _P, _P]),
        "mo_linear_w8a16": (None, [_P, _P, _P, _P, _I, _P, _P, _I64, _I64, _I64]),
        "mo_dequant_i32_scaled": (None, [_P, _P, _P, _P, _P, _I64, _I64]),
        "mo_linear_w8a8": (None, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
        "mo_gemm_bf16_nt": (None, [_P, _P, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64]),
        "mo_mlp_w8a16": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P]),
        "mo_matmul_f64": (None, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64]),
        "mo_matvec_f64": (None, [_P, _I64, _I64, _P, _I64, _P, _I64, _I64]),
        "mo_tensordot_f32": (None, [_P, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64]),
        "mo_linear_backward_f32": (None, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64]),
        "mo_matmul_backward_f64": (None, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I]),
        "mo_matmul_backward_f32": (None, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I]),
        "mo_conv2d_fw_f32": (None, [_P, _P, _P, _P] + [_I64] * 15),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ----------------------------------------------------------------- RNG
def rng_words(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().mo_rng_words(seed, _ptr(out), n)
    return out


def rng_words_from_state(s0: int, s1: int, n: int) -> np.ndarray:
    """n raw xoroshiro128** words from the state (s0, s1) (no seeding)."""
    out = np.empty(n, np.uint64)
    lib().mo_rng_words_from_state(s0, s1, _ptr(out), n)
    return out


def randu_f32(shape, low=0.0, high=1.0, seed=0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().mo_randu_f32(_ptr(out), n, low, high, seed)
    return out.reshape(shape)


def randn_f32(shape, mean=0.0, std=1.0, seed=0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().mo_randn_f32(_ptr(out), n, mean, std, seed)
    return out.reshape(shape)


def randn_f32_f32core(shape, seed=0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().mo_randn_f32_f32core(_ptr(out), n, seed)
    return out.reshape(shape)


# ----------------------------------------------------------------- elementwise
def maximum_scalar_f32(x, s: float) -> np.ndarray:
    """Tensor[Float32].maximum_scalar(s) (tensor/tensor.mojo:4232)."""
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.float32)
    lib().mo_maximum_scalar32_n(_ptr(x), float(np.float32(s)), _ptr(y), x.size)
    return y


def astype_f32_from_int(x) -> np.ndarray:
    """astype_f32_from_int (tensor/cast.mojo:5431-5437) of an int64 array."""
    x = _c(x, np.int64)
    y = np.empty(x.shape, np.float32)
    lib().mo_astype_f32_from_int(_ptr(x), _ptr(y), x.size)
    return y


# ----------------------------------------------------------------- bf16
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().mo_f32_to_bf16_n(_ptr(x), _ptr(y), x.size)
    return y


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().mo_bf16_to_f32_n(_ptr(h), _ptr(y), h.size)
    return y


# ----------------------------------------------------------------- fp32 engine
def matmul_f32(A, B) -> np.ndarray:
    """tensor.matmul for 2-D float32 operands given as numpy arrays or views.

    Strides (in elements) of views are honoured, which is what the reference's
    strided path does for transposed views (broadcast.mojo:1647-1673)."""
    A = np.asarray(A, np.float32)
    B = np.asarray(B, np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    sA = [s // 4 for s in A.strides]
    sB = [s // 4 for s in B.strides]
    assert min(sA + sB) >= 0, "negative strides are not views momijo can make"
    C = np.empty((M, N), np.float32)
    lib().mo_matmul_f32(A.ctypes.data, sA[0], sA[1], B.ctypes.data, sB[0], sB[1], _ptr(C), M, N, K)
    return C


def matmul_f64(A, B) -> np.ndarray:
    """tensor.matmul / matmul2d for 2-D float64 operands (views allowed)."""
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    M, K = A.shape
    N = B.shape[1]
    assert B.shape[0] == K
    sA = [s // 8 for s in A.strides]
    sB = [s // 8 for s in B.strides]
    assert min(sA + sB) >= 0
    C = np.empty((M, N), np.float64)
    lib().mo_matmul_f64(A.ctypes.data, sA[0], sA[1], B.ctypes.data, sB[0], sB[1], _ptr(C), M, N, K)
    return C


def linear_backward_f32(x, W, dy):
    """Linear.backward (learn/nn/layers.mojo:519-618) -> (dW, db, dx) for
    x [N, InF], W [OutF, InF], dy [N, OutF], strict summation order."""
    x = _c(x, np.float32)
    W = _c(W, np.float32)
    dy = _c(dy, np.float32)
    N, InF = x.shape
    OutF = W.shape[0]
    assert W.shape == (OutF, InF) and dy.shape == (N, OutF)
    dW = np.empty((OutF, InF), np.float32)
    db = np.empty(OutF, np.float32)
    dx = np.empty((N, InF), np.float32)
    lib().mo_linear_backward_f32(_ptr(x), _ptr(W), _ptr(dy), _ptr(dW), _ptr(db), _ptr(dx),
                                 N, InF, OutF)
    return dW, db, dx


def matmul_backward_f64(a, b, g, da=None, db=None):
    """The autograd MATMUL2D rule (tensor/autograd.mojo:1542-1555): returns
    (da + g @ b^T, db + a^T @ g); with da/db None the sums start from zero."""
    a = _c(a, np.float64)
    b = _c(b, np.float64)
    g = _c(g, np.float64)
    M, K = a.shape
    N = b.shape[1]
    assert b.shape == (K, N) and g.shape == (M, N)
    acc = 1 if (da is not None or db is not None) else 0
    oa = _c(da, np.float64).copy() if da is not None else np.zeros((M, K))
    ob = _c(db, np.float64).copy() if db is not None else np.zeros((K, N))
    lib().mo_matmul_backward_f64(_ptr(a), _ptr(b), _ptr(g), _ptr(oa), _ptr(ob), M, N, K, acc)
    return oa, ob


def matmul_backward_f32(a, b, g, da=None, db=None):
    """The MATMUL2D rule with the tape's Float32 values (tensor/autograd.mojo:
    214-216, 1542-1555): returns (da + g @ b^T, db + a^T @ g), each product
    in strict inner order; with da/db None the sums start from zero."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    g = _c(g, np.float32)
    M, K = a.shape
    N = b.shape[1]
    assert b.shape == (K, N) and g.shape == (M, N)
    acc = 1 if (da is not None or db is not None) else 0
    oa = _c(da, np.float32).copy() if da is not None else np.zeros((M, K), np.float32)
    ob = _c(db, np.float32).copy() if db is not None else np.zeros((K, N), np.float32)
    lib().mo_matmul_backward_f32(_ptr(a), _ptr(b), _ptr(g), _ptr(oa), _ptr(ob), M, N, K, acc)
    return oa, ob


def matvec_f64(A, x) -> np.ndarray:
    A = np.asarray(A, np.float64)
    x = np.asarray(x, np.float64)
    M, N = A.shape
    y = np.empty(M, np.float64)
    lib().mo_matvec_f64(A.ctypes.data, A.strides[0] // 8, A.strides[1] // 8,
                        x.ctypes.data, x.strides[0] // 8, _ptr(y), M, N)
    return y


def tensordot_f32(A, B) -> np.ndarray:
    """tensordot(A, B, axes=1) for float32 arrays of rank >= 2 whose batch
    dimensions (all but the last two) broadcast against each other."""
    A = np.asarray(A, np.float32)
    B = np.asarray(B, np.float32)
    M, K = A.shape[-2:]
    K2, N = B.shape[-2:]
    assert K == K2
    batch = np.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    Ab = np.broadcast_to(A, batch + (M, K))
    Bb = np.broadcast_to(B, batch + (K, N))
    nb = int(np.prod(batch)) if batch else 1
    idx = np.indices(batch).reshape(len(batch), -1).T if batch else np.zeros((1, 0), np.int64)
    a_off = np.array([sum(int(i) * s // 4 for i, s in zip(ix, Ab.strides[:-2])) for ix in idx], np.int64)
    b_off = np.array([sum(int(i) * s // 4 for i, s in zip(ix, Bb.strides[:-2])) for ix in idx], np.int64)
    C = np.empty((nb, M, N), np.float32)
    lib().mo_tensordot_f32(A.ctypes.data, _ptr(a_off), Ab.strides[-2] // 4, Ab.strides[-1] // 4,
                           B.ctypes.data, _ptr(b_off), Bb.strides[-2] // 4, Bb.strides[-1] // 4,
                           _ptr(C), nb, M, N, K)
    return C.reshape(batch + (M, N))


def matvec_f32(A, x) -> np.ndarray:
    A = np.asarray(A, np.float32)
    x = np.asarray(x, np.float32)
    M, N = A.shape
    y = np.empty(M, np.float32)
    lib().mo_matvec_f32(A.ctypes.data, A.strides[0] // 4, A.strides[1] // 4,
                        x.ctypes.data, x.strides[0] // 4, _ptr(y), M, N)
    return y


def linear_fw_f32(x, W, b=None) -> np.ndarray:
    x = _c(x, np.float32)
    W = _c(W, np.float32)
    N, InF = x.shape
    OutF = W.shape[0]
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((N, OutF), np.float32)
    lib().mo_linear_fw_f32(_ptr(x), _ptr(W), _ptr(bb), int(bb is not None), _ptr(y), N, InF, OutF)
    return y


def kernel_linear_fw_f32(x, wT, b=None) -> np.ndarray:
    x = _c(x, np.float32)
    wT = _c(wT, np.float32)
    N, InF = x.shape
    OutF = wT.shape[1]
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((N, OutF), np.float32)
    lib().mo_kernel_linear_fw_f32(_ptr(x), _ptr(wT), _ptr(bb), int(bb is not None), _ptr(y), N, InF, OutF)
    return y


def linear_act_f32(x, W, b, epi) -> np.ndarray:
    x = _c(x, np.float32)
    W = _c(W, np.float32)
    N, InF = x.shape
    OutF = W.shape[0]
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((N, OutF), np.float32)
    lib().mo_linear_act_f32(_ptr(x), _ptr(W), _ptr(bb), int(bb is not None), epi, _ptr(y), N, InF, OutF)
    return y


def epilogue(epi: int, x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().mo_epilogue32_n(epi, _ptr(x), _ptr(y), x.size)
    return y


def gelu32_literal(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().mo_gelu32_n(_ptr(x), _ptr(y), x.size)
    return y


def exp_approx32(x: float) -> float:
    return lib().mo_exp_approx32(x)


def tanh_approx32(x: float) -> float:
    return lib().mo_tanh_approx32(x)


# ----------------------------------------------------------------- int8
def quant_legacy_one(x: float, scale: float) -> int:
    return int(lib().mo_quant_legacy_one(x, scale))


def quantize_symmetric_int8(x, s: float) -> np.ndarray:
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.int8)
    lib().mo_quantize_symmetric_int8(_ptr(x), x.size, s, _ptr(q))
    return q


def matmul_i8_i8_to_i32(A, B, legacy_literal: bool = False) -> np.ndarray:
    """A int8 [M,K]; B int8 [N,K] (w_q layout).  legacy_literal reads
    reshape(B.flat, [K,N]) exactly as functional.mojo:274 does."""
    A = _c(A, np.int8)
    B = _c(B, np.int8)
    M, K = A.shape
    N = B.size // K
    C = np.empty((M, N), np.int32)
    lib().mo_matmul_i8_i8_to_i32(_ptr(A), _ptr(B), _ptr(C), M, N, K, int(legacy_literal))
    return C


def dequant_i32_bias(acc, sf: float, b) -> np.ndarray:
    acc = _c(acc, np.int32)
    b = _c(b, np.float32)
    M, N = acc.shape
    y = np.empty((M, N), np.float32)
    lib().mo_dequant_i32_bias(_ptr(acc), sf, _ptr(b), _ptr(y), M, N)
    return y


def dequant_i32_scaled(acc, sw, b=None, sx=None) -> np.ndarray:
    """y = float(acc) * (sx[m] * sw[n]) + b[n] (momijo_oracle.c's
    mo_dequant_i32_scaled); sx and b optional."""
    acc = _c(acc, np.int32)
    sw = _c(sw, np.float32)
    b = None if b is None else _c(b, np.float32)
    sx = None if sx is None else _c(sx, np.float32)
    M, N = acc.shape
    y = np.empty((M, N), np.float32)
    lib().mo_dequant_i32_scaled(_ptr(acc), _ptr(sx), _ptr(sw), _ptr(b), _ptr(y), M, N)
    return y


def minmax_scale_symmetric(x, max_q: float = 127.0) -> float:
    x = _c(x, np.float32)
    return float(lib().mo_minmax_scale_symmetric(_ptr(x), x.size, max_q))


def quant_linear_fw(x, Wq, b, s_w: float, s_x: float, legacy_literal: bool = False) -> np.ndarray:
    x = _c(x, np.float32)
    Wq = _c(Wq, np.int8)
    b = _c(b, np.float32)
    M, K = x.shape
    N = Wq.shape[0]
    y = np.empty((M, N), np.float32)
    acc = np.empty((M, N), np.int32)
    xq = np.empty((M, K), np.int8)
    lib().mo_quant_linear_fw(_ptr(x), _ptr(Wq), _ptr(b), s_w, s_x, _ptr(y), _ptr(acc), _ptr(xq),
                             M, N, K, int(legacy_literal))
    return y


def quantize_rowwise_rhe(W):
    W = _c(W, np.float32)
    N, K = W.shape
    Q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    lib().mo_quantize_rowwise_rhe(_ptr(W), N, K, _ptr(Q), _ptr(s))
    return Q, s


def quantize_rowwise_legacy(W):
    W = _c(W, np.float32)
    N, K = W.shape
    Q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    lib().mo_quantize_rowwise_legacy(_ptr(W), N, K, _ptr(Q), _ptr(s))
    return Q, s


def linear_w8a16(x_bf16, Q, scales, b=None, epi=EPI_NONE):
    """Returns (y_bf16 as uint16, y_f32 before rounding)."""
    x = _c(x_bf16, np.uint16)
    Q = _c(Q, np.int8)
    s = _c(scales, np.float32)
    M, K = x.shape
    N = Q.shape[0]
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((M, N), np.uint16)
    yf = np.empty((M, N), np.float32)
    lib().mo_linear_w8a16(_ptr(x), _ptr(Q), _ptr(s), _ptr(bb), epi, _ptr(y), _ptr(yf), M, N, K)
    return y, yf


def linear_w8a8(x_bf16, Q, scales, b=None, epi=EPI_NONE, rows=None):
    """W8A8 Linear with per-row dynamic activation scales (momijo_oracle.c's
    mo_linear_w8a8).  rows=(m0,m1) limits the computed rows.  Returns
    (y_bf16 as uint16, y_f32 before rounding, xq, sx) for those rows."""
    x = _c(x_bf16, np.uint16)
    Q = _c(Q, np.int8)
    s = _c(scales, np.float32)
    M, K = x.shape
    N = Q.shape[0]
    m0, m1 = (0, M) if rows is None else rows
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((m1 - m0, N), np.uint16)
    yf = np.empty((m1 - m0, N), np.float32)
    xq = np.empty((m1 - m0, K), np.int8)
    sx = np.empty(m1 - m0, np.float32)
    lib().mo_linear_w8a8(_ptr(x), _ptr(Q), _ptr(s), _ptr(bb), epi, _ptr(y), _ptr(yf), _ptr(xq),
                         _ptr(sx), N, K, m0, m1)
    return y, yf, xq, sx


def gemm_bf16_nt(A_bf16, B_bf16, bias=None, epi=EPI_NONE, rows=None):
    """C = A @ B^T for bf16 (uint16) A [M,K], B [N,K]; rows=(m0,m1) limits the
    computed rows.  Returns (C_bf16 rows, C_f32 rows)."""
    A = _c(A_bf16, np.uint16)
    B = _c(B_bf16, np.uint16)
    M, K = A.shape
    N = B.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    bb = None if bias is None else _c(bias, np.float32)
    C = np.empty((m1 - m0, N), np.uint16)
    Cf = np.empty((m1 - m0, N), np.float32)
    lib().mo_gemm_bf16_nt(_ptr(A), _ptr(B), _ptr(bb), epi, _ptr(C), _ptr(Cf), M, N, K, m0, m1)
    return C, Cf


def mlp_w8a16(x_bf16, Wg, sg, Wu, su, Wd, sd, rows=None):
    """Returns (h_bf16 rows, y_bf16 rows) for x rows [m0,m1)."""
    x = _c(x_bf16, np.uint16)
    Wg, Wu, Wd = _c(Wg, np.int8), _c(Wu, np.int8), _c(Wd, np.int8)
    sg, su, sd = _c(sg, np.float32), _c(su, np.float32), _c(sd, np.float32)
    M, K = x.shape
    I = Wg.shape[0]
    H = Wd.shape[0]
    m0, m1 = rows if rows is not None else (0, M)
    h = np.empty((m1 - m0, I), np.uint16)
    y = np.empty((m1 - m0, H), np.uint16)
    scratch = np.empty(I, np.uint16)
    lib().mo_mlp_w8a16(_ptr(x), _ptr(Wg), _ptr(sg), _ptr(Wu), _ptr(su), _ptr(Wd), _ptr(sd),
                       _ptr(h), _ptr(y), K, I, H, m0, m1, _ptr(scratch))
    return h, y


# ----------------------------------------------------------------- conv2d
def conv_out_size(size: int, k: int, s: int, p: int) -> int:
    """(size + 2 p - k) // s + 1 with floor division, as Conv2d.forward sizes
    its output (learn/nn/conv.mojo:496-497, 682-683)."""
    return (size + 2 * p - k) // s + 1


def conv2d_fw_f32(x, w, b=None, stride=(1, 1), pad=(0, 0), images=None) -> np.ndarray:
    """Conv2d.forward (NCHW, learn/nn/conv.mojo:600-681).  images=(n0, n1)
    limits the computed images; returns y [n1 - n0, OC, OH, OW]."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    N, C, H, W = x.shape
    OC, C2, kH, kW = w.shape
    assert C == C2, "x and w disagree on the input channels"
    sH, sW = stride
    pH, pW = pad
    OH, OW = conv_out_size(H, kH, sH, pH), conv_out_size(W, kW, sW, pW)
    n0, n1 = images if images is not None else (0, N)
    bb = None if b is None else _c(b, np.float32)
    y = np.empty((n1 - n0, OC, max(OH, 0), max(OW, 0)), np.float32)
    if OH > 0 and OW > 0:
        lib().mo_conv2d_fw_f32(_ptr(x), _ptr(w), _ptr(bb), _ptr(y), N, C, H, W, OC, kH, kW,
                               sH, sW, pH, pW, OH, OW, n0, n1)
    return y
