"""The host-memory half of the C ABI on the GPU: every host-pointer (_h)
entry point called through ctypes with host numpy buffers, as a momijo
Tensor's List storage would be passed, against the oracle; the device
memory entry points; and the seam launchers taking their device path.

Bars as in the other GPU tests: bit-exact where the inputs make every sum
exact (integer-valued data) or the operation is exact (int8, quantizers,
min/max), |d| <= 1e-5 + 1e-5 |ref| for fp32 results otherwise.
"""
import ctypes

import numpy as np
import pytest

import momijo_amd as mj
from momijo_amd import _lib, seam
from _util import assert_close_f32

pytestmark = pytest.mark.gpu


def P(a):
    return None if a is None else a.ctypes.data


def call(fn, *args):
    _lib.check(getattr(_lib.load(), fn)(*args), fn)


def ints(rng, shape, lo=-4, hi=5, dtype=np.float32):
    return rng.integers(lo, hi, size=shape).astype(dtype)


def test_matmul_f32_h_strided_views_and_padded_output(oracle, dev):
    M, N, K, ldc = 37, 29, 50, 33
    x = oracle.randn_f32((M, K), seed=1)
    W = oracle.randn_f32((N, K), seed=2)
    b = oracle.randu_f32((N,), -1 / 16, 1 / 16, seed=3)
    B = W.T                                     # zero-copy view: strides (1, K)
    C = np.full((M, ldc), 7.5, np.float32)      # padding columns must survive
    call("mj_matmul_f32_h", M, N, K, P(x), K, 1, W.ctypes.data, B.strides[0] // 4,
         B.strides[1] // 4, P(b), mj.EPI_RELU, P(C), ldc)
    assert_close_f32(C[:, :N], oracle.linear_act_f32(x, W, b, oracle.EPI_RELU))
    assert (C[:, N:] == 7.5).all()
    y = np.empty((M, N), np.float32)
    call("mj_linear_f32_h", P(x), P(W), P(b), mj.EPI_GELU_TANH, P(y), M, K, N)
    assert_close_f32(y, oracle.linear_act_f32(x, W, b, oracle.EPI_GELU_TANH))


def test_matvec_h_strided(oracle, dev):
    A = oracle.randn_f32((64, 40), seed=4)
    xs = oracle.randn_f32((80,), seed=5)
    At, x2 = A.T, xs[::2]                       # [40, 64] view, every other element
    y = np.empty(40, np.float32)
    call("mj_matvec_f32_h", 40, 64, A.ctypes.data, At.strides[0] // 4, At.strides[1] // 4,
         xs.ctypes.data, 2, P(y))
    assert_close_f32(y, oracle.matvec_f32(At, x2))
    rng = np.random.default_rng(6)
    A64 = ints(rng, (30, 20), dtype=np.float64)
    x64 = ints(rng, (20,), dtype=np.float64)
    y64 = np.empty(30, np.float64)
    call("mj_matvec_f64_h", 30, 20, P(A64), 20, 1, P(x64), 1, P(y64))
    np.testing.assert_array_equal(y64, oracle.matvec_f64(A64, x64))


def test_matmul_f64_h_and_backward_h(oracle, dev):
    rng = np.random.default_rng(7)
    M, K, N = 33, 17, 21
    a = ints(rng, (M, K), dtype=np.float64)
    bm = ints(rng, (K, N), dtype=np.float64)
    c = np.empty((M, N), np.float64)
    call("mj_matmul_f64_h", M, N, K, P(a), K, 1, P(bm), N, 1, P(c), N)
    np.testing.assert_array_equal(c, oracle.matmul_f64(a, bm))
    g = ints(rng, (M, N), dtype=np.float64)
    da = ints(rng, (M, K), dtype=np.float64)
    dbm = ints(rng, (K, N), dtype=np.float64)
    ra, rb = oracle.matmul_backward_f64(a, bm, g, da, dbm)
    call("mj_matmul_backward_f64_h", M, N, K, P(a), P(bm), P(g), P(da), P(dbm), 1)
    np.testing.assert_array_equal(da, ra)
    np.testing.assert_array_equal(dbm, rb)


def test_tensordot_h_broadcast(oracle, dev):
    A = oracle.randn_f32((2, 1, 7, 9), seed=8)
    B = oracle.randn_f32((3, 9, 5), seed=9)
    Ab = np.broadcast_to(A, (2, 3, 7, 9))
    Bb = np.broadcast_to(B, (2, 3, 9, 5))
    arr = ctypes.c_int64 * 2
    shape = arr(2, 3)
    sa = arr(*(s // 4 for s in Ab.strides[:2]))
    sb = arr(*(s // 4 for s in Bb.strides[:2]))
    C = np.empty((2, 3, 7, 5), np.float32)
    call("mj_tensordot_f32_h", 2, shape, sa, sb, 7, 5, 9, A.ctypes.data, 9, 1, B.ctypes.data, 5, 1,
         P(C))
    assert_close_f32(C, oracle.tensordot_f32(A, B))


def test_linear_backward_h(oracle, dev):
    rng = np.random.default_rng(10)
    N, InF, OutF = 12, 20, 9
    x, W, dy = ints(rng, (N, InF)), ints(rng, (OutF, InF)), ints(rng, (N, OutF))
    dW = np.empty((OutF, InF), np.float32)
    db = np.empty(OutF, np.float32)
    dx = np.empty((N, InF), np.float32)
    call("mj_linear_backward_f32_h", P(x), P(W), P(dy), P(dW), P(db), P(dx), N, InF, OutF)
    rW, rb, rx = oracle.linear_backward_f32(x, W, dy)
    np.testing.assert_array_equal(dW, rW)
    np.testing.assert_array_equal(db, rb)
    np.testing.assert_array_equal(dx, rx)
    only_db = np.empty(OutF, np.float32)        # outputs may be skipped (NULL)
    call("mj_linear_backward_f32_h", None, None, P(dy), None, P(only_db), None, N, InF, OutF)
    np.testing.assert_array_equal(only_db, rb)


def test_activation_h(oracle, dev):
    x = oracle.randn_f32((1000,), seed=11) * np.float32(4)
    x[:3] = [-0.0, np.nan, 0.0]
    y = np.empty_like(x)
    call("mj_activation_f32_h", mj.EPI_RELU_UNARY, P(x), P(y), x.size)
    np.testing.assert_array_equal(y, oracle.epilogue(oracle.EPI_RELU_UNARY, x))
    call("mj_activation_f32_h", mj.EPI_SILU, P(x), P(y), x.size)
    assert_close_f32(y[3:], oracle.epilogue(oracle.EPI_SILU, x)[3:], atol=1e-6, rtol=1e-6)


def test_gemm_bf16_nt_h_padded(oracle, dev):
    rng = np.random.default_rng(12)
    M, N, K, lda, ldb, ldc = 70, 90, 64, 72, 80, 96
    A = np.zeros((M, lda), np.uint16)
    B = np.zeros((N, ldb), np.uint16)
    A[:, :K] = oracle.f32_to_bf16(ints(rng, (M, K)))
    B[:, :K] = oracle.f32_to_bf16(ints(rng, (N, K)))
    bias = (rng.integers(-8, 9, size=N) / 4).astype(np.float32)
    C = np.full((M, ldc), 0x1357, np.uint16)
    call("mj_gemm_bf16_nt_h", M, N, K, P(A), lda, P(B), ldb, P(bias), mj.EPI_NONE, P(C), ldc)
    ref, _ = oracle.gemm_bf16_nt(np.ascontiguousarray(A[:, :K]), np.ascontiguousarray(B[:, :K]),
                                 bias)
    np.testing.assert_array_equal(C[:, :N], ref)
    assert (C[:, N:] == 0x1357).all()


def test_int8_helpers_h(oracle, dev):
    rng = np.random.default_rng(13)
    x = oracle.randn_f32((300,), seed=14) * np.float32(3)
    x[:4] = [0.49999997, -0.49999997, 2.5, -2.5]
    q = np.empty(300, np.int8)
    call("mj_quantize_symmetric_int8_h", P(x), 300, np.float32(0.05), P(q))
    np.testing.assert_array_equal(q, oracle.quantize_symmetric_int8(x, 0.05))
    mm = np.empty(2, np.float32)
    call("mj_minmax_f32_h", P(x), 300, P(mm))
    assert mm[0] == x.min() and mm[1] == x.max()
    sc = np.empty(1, np.float32)
    call("mj_minmax_scale_symmetric_h", P(x), 300, np.float32(127), P(sc))
    assert sc[0] == np.float32(oracle.minmax_scale_symmetric(x))
    A = rng.integers(-128, 128, size=(19, 48), dtype=np.int8)
    Bq = rng.integers(-128, 128, size=(23, 48), dtype=np.int8)
    C = np.empty((19, 23), np.int32)
    for literal in (0, 1):
        call("mj_matmul_i8_i8_to_i32_h", P(A), P(Bq), P(C), 19, 23, 48, literal)
        np.testing.assert_array_equal(C, oracle.matmul_i8_i8_to_i32(A, Bq, bool(literal)))
    b = oracle.randu_f32((23,), -1, 1, seed=15)
    y = np.empty((19, 23), np.float32)
    call("mj_dequantize_i32_to_f32_add_bias_h", P(C), np.float32(0.001), P(b), P(y), 19, 23)
    np.testing.assert_array_equal(y, oracle.dequant_i32_bias(C, 0.001, b))


def test_quant_linear_h(oracle, dev):
    x = oracle.randn_f32((5, 64), seed=16)
    W = oracle.randn_f32((12, 64), std=0.1, seed=17)
    b = oracle.randu_f32((12,), -0.1, 0.1, seed=18)
    s_x, s_w = oracle.minmax_scale_symmetric(x), oracle.minmax_scale_symmetric(W)
    Wq = oracle.quantize_symmetric_int8(W, s_w)
    y = np.empty((5, 12), np.float32)
    for literal in (0, 1):
        call("mj_quant_linear_f32_h", P(x), P(Wq), P(b), np.float32(s_w), np.float32(s_x), P(y),
             5, 12, 64, literal)
        np.testing.assert_array_equal(y, oracle.quant_linear_fw(x, Wq, b, s_w, s_x, bool(literal)))


def test_w8a16_h(oracle, dev):
    rng = np.random.default_rng(19)
    W = oracle.randn_f32((40, 256), std=0.02, seed=20)
    Q = np.empty((40, 256), np.int8)
    s = np.empty(40, np.float32)
    call("mj_quantize_rowwise_i8_h", P(W), 40, 256, mj.ROUND_RHE, P(Q), P(s))
    Qr, sr = oracle.quantize_rowwise_rhe(W)
    np.testing.assert_array_equal(Q, Qr)
    np.testing.assert_array_equal(s, sr)
    # integer-valued x and power-of-two scales: exact sums, bit-exact outputs
    for M in (1, 3, 300):
        x = oracle.f32_to_bf16(ints(rng, (M, 256)))
        Qi = rng.integers(-127, 128, size=(40, 256), dtype=np.int8)
        si = (2.0 ** rng.integers(-8, -2, size=40)).astype(np.float32)
        bi = (rng.integers(-8, 9, size=40) / 4).astype(np.float32)
        y = np.empty((M, 40), np.uint16)
        call("mj_linear_w8a16_h", P(x), P(Qi), P(si), P(bi), mj.EPI_NONE, P(y), M, 40, 256)
        ref, _ = oracle.linear_w8a16(x, Qi, si, bi)
        np.testing.assert_array_equal(y, ref)


def test_w8a8_and_dequant_scaled_h(oracle, dev):
    """mj_linear_w8a8_h and mj_dequantize_i32_scaled_f32_h on host buffers,
    bit-exact against the oracle (exact int32 sums, step-by-step epilogue)."""
    rng = np.random.default_rng(23)
    N, K = 40, 256
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = oracle.randu_f32((N,), 0.001, 0.01, seed=24)
    b = oracle.randu_f32((N,), -0.5, 0.5, seed=25)
    for M, bias in ((1, b), (3, None), (300, b)):
        x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=26 + M))
        y = np.empty((M, N), np.uint16)
        call("mj_linear_w8a8_h", P(x), P(Q), P(s), P(bias), mj.EPI_RELU, P(y), M, N, K)
        ref, _, _, _ = oracle.linear_w8a8(x, Q, s, bias, mj.EPI_RELU)
        np.testing.assert_array_equal(y, ref)
    acc = rng.integers(-(2 ** 30), 2 ** 30, size=(19, 23)).astype(np.int32)
    sw = oracle.randu_f32((23,), 0.001, 0.01, seed=27)
    sx = oracle.randu_f32((19,), 0.01, 0.1, seed=28)
    bb = oracle.randu_f32((23,), -1, 1, seed=29)
    for rows, bias in ((sx, bb), (None, None)):
        y = np.empty((19, 23), np.float32)
        call("mj_dequantize_i32_scaled_f32_h", P(acc), P(rows), P(sw), P(bias), P(y), 19, 23)
        np.testing.assert_array_equal(y, oracle.dequant_i32_scaled(acc, sw, bias, rows))


def test_mlp_h(oracle, dev):
    M, K, I, H = 20, 256, 160, 96
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=21))
    Wg, sg = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=22))
    Wu, su = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=23))
    Wd, sd = oracle.quantize_rowwise_rhe(oracle.randn_f32((H, I), std=0.02, seed=24))
    hr, yr = oracle.mlp_w8a16(x, Wg, sg, Wu, su, Wd, sd)
    h = np.empty((M, I), np.uint16)
    y = np.empty((M, H), np.uint16)
    call("mj_mlp_w8a16_h", P(x), P(Wg), P(sg), P(Wu), P(su), P(Wd), P(sd), P(h), P(y), M, K, I, H)
    ref_y = oracle.bf16_to_f32(yr)
    got = oracle.bf16_to_f32(y)
    assert np.max(np.abs(got - ref_y)) <= 2e-2 * np.max(np.abs(ref_y))
    assert np.max(np.abs(oracle.bf16_to_f32(h) - oracle.bf16_to_f32(hr))) <= \
        2e-2 * np.max(np.abs(oracle.bf16_to_f32(hr)))
    y2 = np.empty((M, H), np.uint16)            # h may stay on the device
    call("mj_mlp_w8a16_h", P(x), P(Wg), P(sg), P(Wu), P(su), P(Wd), P(sd), None, P(y2), M, K, I, H)
    np.testing.assert_array_equal(y2, y)


def test_device_memory_entry_points(oracle, dev):
    lib = _lib.load()
    rng = np.random.default_rng(25)
    M, N, K = 16, 24, 32
    a, bm = ints(rng, (M, K)), ints(rng, (K, N))
    ptrs = [ctypes.c_void_p() for _ in range(3)]
    stream = ctypes.c_void_p()
    call("mj_stream_create", ctypes.byref(stream))
    try:
        for p_, nbytes in zip(ptrs, (a.nbytes, bm.nbytes, M * N * 4)):
            call("mj_malloc", ctypes.byref(p_), nbytes)
        call("mj_memcpy_htod", ptrs[0], P(a), a.nbytes, stream)
        call("mj_memcpy_htod", ptrs[1], P(bm), bm.nbytes, None)
        call("mj_matmul_f32", M, N, K, ptrs[0], K, 1, ptrs[1], N, 1, None, 0, ptrs[2], N, stream)
        c = np.empty((M, N), np.float32)
        call("mj_memcpy_dtoh", P(c), ptrs[2], c.nbytes, stream)
        np.testing.assert_array_equal(c, oracle.matmul_f32(a, bm))
        call("mj_memcpy_dtod", ptrs[0], ptrs[2], min(a.nbytes, c.nbytes), stream)
        call("mj_device_synchronize")
        back = np.empty(M * K, np.float32)
        call("mj_memcpy_dtoh", P(back), ptrs[0], back.nbytes, None)
        np.testing.assert_array_equal(back[:M * N], c.reshape(-1)[:M * K])
    finally:
        for p_ in ptrs:
            call("mj_free", p_)
        call("mj_stream_destroy", stream)
    z = ctypes.c_void_p(1)
    call("mj_malloc", ctypes.byref(z), 0)
    assert z.value is None
    assert lib.mj_malloc(ctypes.byref(z), -1) == _lib.MJ_ERR_ARG


def _never_called(*_):
    raise AssertionError("the CPU kernel ran: the device path failed")


def test_seam_takes_device_path(oracle, dev):
    N, InF, OutF = 64, 96, 80
    x = oracle.randn_f32((N, InF), seed=26)
    W = oracle.randn_f32((OutF, InF), seed=27)
    wT = np.ascontiguousarray(W.T)
    b = oracle.randu_f32((OutF,), -1 / 16, 1 / 16, seed=28)
    y = np.zeros(N * OutF, np.float32)
    assert seam.launch_1d_linear_fw(N * OutF, 256, _never_called, x, wT, b, y, N, InF, OutF,
                                    True) == "gpu"
    assert_close_f32(y.reshape(N, OutF), oracle.kernel_linear_fw_f32(x, wT, b))
    rng = np.random.default_rng(29)
    xi, Wi, dy = ints(rng, (N, InF)), ints(rng, (OutF, InF)), ints(rng, (N, OutF))
    rW, rb, rx = oracle.linear_backward_f32(xi, Wi, dy)
    dx = np.zeros(N * InF, np.float32)
    dW = np.zeros(OutF * InF, np.float32)
    db = np.zeros(OutF, np.float32)
    assert seam.launch_1d_linear_bw_dx(N * InF, 256, _never_called, dy, Wi, dx, N, InF, OutF,
                                       strict=True) == "gpu"
    assert seam.launch_1d_linear_bw_dw(OutF * InF, 256, _never_called, dy, xi, dW, N, InF,
                                       OutF, strict=True) == "gpu"
    assert seam.launch_1d_linear_bw_db(OutF, 256, _never_called, dy, db, N, OutF,
                                       strict=True) == "gpu"
    np.testing.assert_array_equal(dx.reshape(N, InF), rx)
    np.testing.assert_array_equal(dW.reshape(OutF, InF), rW)
    np.testing.assert_array_equal(db, rb)
