"""GPU parity of the fp32 engine against the oracle (config C1 and edges).

Bar: |gpu - oracle| <= 1e-5 + 1e-5 |oracle| elementwise (
max-abs/rel 1e-5 for fp32).  The oracle sums in strict k order; the MFMA
kernel sums in blocks of 4, so equality is to rounding, not bitwise, except
for integer-valued inputs where every partial sum is exact.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib
from _util import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu


def _mm(A, B, dev):
    return mj.matmul(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev))).numpy()


def test_c1_matmul_256(oracle, dev):
    A = oracle.randn_f32((256, 256), seed=1)
    B = oracle.randn_f32((256, 256), seed=2)
    got = _mm(A, B, dev)
    assert_close_f32(got, oracle.matmul_f32(A, B))


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (33, 17, 70), (64, 64, 16), (65, 129, 257),
                                   (7, 300, 5), (300, 7, 1000)])
def test_matmul_ragged(oracle, dev, M, N, K):
    A = oracle.randn_f32((M, K), seed=M * 7 + K)
    B = oracle.randn_f32((K, N), seed=N * 11 + K)
    assert_close_f32(_mm(A, B, dev), oracle.matmul_f32(A, B))


def test_matmul_integer_inputs_exact(oracle, dev):
    """Small-integer operands: every partial sum is exact in fp32, so the
    result must be bit-identical whatever the summation order."""
    rng = np.random.default_rng(0)
    A = rng.integers(-8, 9, size=(96, 256)).astype(np.float32)
    B = rng.integers(-8, 9, size=(256, 80)).astype(np.float32)
    got = _mm(A, B, dev)
    np.testing.assert_array_equal(got, oracle.matmul_f32(A, B))


def _view(M, dev, transposed):
    """M as a device Tensor, either contiguous or as the transpose view of
    its contiguous transpose (same values, swapped strides)."""
    if not transposed:
        return mj.Tensor(to_dev(M, dev))
    return mj.Tensor(to_dev(np.ascontiguousarray(M.T), dev)).transpose()


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True)])
def test_matmul_large_tiles_integer_exact(oracle, dev, ta, tb):
    """A 3000 x 2900 product runs on 128 x 128 tiles (smaller ones on
    64 x 64); small-integer operands make every sum exact, so the result is
    bit-identical to the oracle, also through transposed views (both loader
    orientations of A and of B)."""
    rng = np.random.default_rng(7 + 2 * ta + tb)
    M, N, K = 3000, 2900, 72
    A = rng.integers(-8, 9, size=(M, K)).astype(np.float32)
    B = rng.integers(-8, 9, size=(K, N)).astype(np.float32)
    got = mj.matmul(_view(A, dev, ta), _view(B, dev, tb)).numpy()
    np.testing.assert_array_equal(got, oracle.matmul_f32(A, B))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("M,N,K", [(100, 90, 200), (31, 33, 130), (256, 256, 256)])
def test_matmul_small_tiles_integer_exact(oracle, dev, dtype, ta, tb, M, N, K):
    """Problems of fewer than 64 tiles of 64 x 64 run on 32 x 32 tiles with
    deep K stages (64 for fp32, 32 for fp64); K here is not a multiple of
    the stage, so the last stage is zero-filled, and the transposed views
    take the k-fast loaders.  Small-integer operands make every sum exact."""
    rng = np.random.default_rng(M + 3 * N + K + 2 * ta + tb)
    A = rng.integers(-8, 9, size=(M, K)).astype(dtype)
    B = rng.integers(-8, 9, size=(K, N)).astype(dtype)
    got = mj.matmul(_view(A, dev, ta), _view(B, dev, tb)).numpy()
    np.testing.assert_array_equal(got, (A.astype(np.float64) @ B.astype(np.float64)).astype(dtype))


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (100, 90, 200), (1, 300, 64), (37, 1000, 252),
                                   (37, 1000, 1004), (250, 3, 4096), (16, 16, 4)])
def test_direct_and_staged_small_tiles_agree_bitwise(oracle, dev, M, N, K):
    """The same product of N(0,1) operands through both fp32 small-problem
    kernels: with B as the transpose of a contiguous [N, K] (k-contiguous
    rows, the LDS-free kernel) and as a contiguous [K, N] (the staged 32 x 32
    kernel).  Both issue the same MFMA sequence in the same k order, so the
    results are identical bit for bit, not just within the fp32 bar (checked
    against the oracle up to K = 256: at K ~ 1000 and beyond, outputs that
    cancel to near zero differ from the strict-order sum by more than 1e-5
    absolute in either kernel)."""
    A = oracle.randn_f32((M, K), seed=M + K)
    B = oracle.randn_f32((K, N), seed=N + 2 * K)
    a = mj.Tensor(to_dev(A, dev))
    direct = mj.matmul(a, mj.Tensor(to_dev(np.ascontiguousarray(B.T), dev)).transpose()).numpy()
    staged = mj.matmul(a, mj.Tensor(to_dev(B, dev))).numpy()
    np.testing.assert_array_equal(direct, staged)
    if K <= 256:
        assert_close_f32(direct, oracle.matmul_f32(A, B))


def test_matmul_transposed_views(oracle, dev):
    """x.matmul(W.transpose()) and A.transpose().matmul(B) run on the stride
    views, as the reference's strided path does (broadcast.mojo:1647-1673)."""
    x = oracle.randn_f32((50, 96), seed=3)
    W = oracle.randn_f32((70, 96), seed=4)
    xt = mj.Tensor(to_dev(x, dev))
    Wt = mj.Tensor(to_dev(W, dev))
    got = xt.matmul(Wt.transpose()).numpy()
    assert_close_f32(got, oracle.matmul_f32(x, W.T))
    At = mj.Tensor(to_dev(W, dev)).transpose()  # [96, 70] view
    got2 = At.matmul(mj.Tensor(to_dev(oracle.randn_f32((70, 33), seed=9), dev))).numpy()
    assert_close_f32(got2, oracle.matmul_f32(W.T, oracle.randn_f32((70, 33), seed=9)))


def test_matmul_rank_and_shape_errors(dev):
    """Unsupported ranks or a K mismatch give an empty tensor, silently, as
    in broadcast.mojo:1613-1616,1677-1684."""
    a = mj.Tensor(torch.ones((4, 5), device=dev))
    b = mj.Tensor(torch.ones((6, 3), device=dev))
    assert a.matmul(b).numel() == 0
    c = mj.Tensor(torch.ones((2, 2, 2), device=dev))
    assert a.matmul(c).numel() == 0


def test_matvec(oracle, dev):
    A = oracle.randn_f32((300, 517), seed=5)
    x = oracle.randn_f32((517,), seed=6)
    got = mj.Tensor(to_dev(A, dev)).matmul_vec(mj.Tensor(to_dev(x, dev))).numpy()
    assert_close_f32(got, oracle.matvec_f32(A, x))
    got2 = mj.matmul(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(x, dev))).numpy()
    assert_close_f32(got2, oracle.matvec_f32(A, x))


@pytest.mark.parametrize("epi", [mj.EPI_NONE, mj.EPI_RELU, mj.EPI_GELU_TANH, mj.EPI_SILU,
                                 mj.EPI_GELU_TANH_APPROX, mj.EPI_SILU_APPROX])
def test_c1_linear_bias_act(oracle, dev, epi):
    """Config C1: Linear(256 -> 256) with bias ~ U(-1/16, 1/16), fused
    activation; oracle = Linear.forward then the activation on fp32."""
    x = oracle.randn_f32((256, 256), seed=1)
    W = oracle.randn_f32((256, 256), seed=2)
    b = oracle.randu_f32((256,), -1.0 / 16, 1.0 / 16, seed=5)
    lin = mj.Linear(256, 256)
    lin.weight.torch.copy_(torch.from_numpy(W))
    lin.bias_t.torch.copy_(torch.from_numpy(b))
    got = lin.forward_act(mj.Tensor(to_dev(x, dev)), epi).numpy()
    assert_close_f32(got, oracle.linear_act_f32(x, W, b, epi))


def test_c1_linear_then_relu_layer(oracle, dev):
    x = oracle.randn_f32((256, 256), seed=1)
    W = oracle.randn_f32((256, 256), seed=2)
    b = oracle.randu_f32((256,), -1.0 / 16, 1.0 / 16, seed=5)
    lin = mj.Linear(256, 256)
    lin.weight.torch.copy_(torch.from_numpy(W))
    lin.bias_t.torch.copy_(torch.from_numpy(b))
    y = mj.ReLU().forward(lin.forward(mj.Tensor(to_dev(x, dev)))).numpy()
    ref = oracle.linear_fw_f32(x, W, b)
    assert_close_f32(y, np.where(ref > 0, ref, 0).astype(np.float32))


def test_linear_default_init_and_bad_shape(oracle, dev):
    """reset_parameters gives W = 0.01/InF, b = 0 (layers.mojo:361-377); a width
    mismatch returns the input unchanged (:385-390)."""
    lin = mj.Linear(10, 32)
    x = oracle.randn_f32((4, 10), seed=7)
    got = lin.forward(mj.Tensor(to_dev(x, dev))).numpy()
    W = np.full((32, 10), np.float32(0.01) / np.float32(10), np.float32)
    assert_close_f32(got, oracle.linear_fw_f32(x, W, np.zeros(32, np.float32)))
    bad = mj.Tensor(to_dev(oracle.randn_f32((4, 9), seed=8), dev))
    np.testing.assert_array_equal(lin.forward(bad).numpy(), bad.numpy())


def test_launch_linear_fw_host_seam(oracle):
    """mj_launch_linear_fw_h: host buffers in/out, wT [InF, OutF], the
    contract of launch_1d_linear_fw's CPU kernel (layers.mojo:436-475)."""
    import ctypes
    N, InF, OutF = 37, 129, 65
    x = oracle.randn_f32((N, InF), seed=11)
    wT = oracle.randn_f32((InF, OutF), seed=12)
    b = oracle.randu_f32((OutF,), -0.0625, 0.0625, seed=13)
    y = np.empty((N, OutF), np.float32)
    lib = _lib.load()
    st = lib.mj_launch_linear_fw_h(x.ctypes.data, wT.ctypes.data, b.ctypes.data, y.ctypes.data,
                                   N, InF, OutF, 1)
    assert st == 0, lib.mj_last_error()
    assert_close_f32(y, oracle.kernel_linear_fw_f32(x, wT, b))
    y2 = np.empty((N, OutF), np.float32)
    st = lib.mj_launch_linear_fw_h(x.ctypes.data, wT.ctypes.data, None, y2.ctypes.data,
                                   N, InF, OutF, 0)
    assert st == 0
    assert_close_f32(y2, oracle.kernel_linear_fw_f32(x, wT, None))
    del ctypes


@pytest.mark.parametrize("epi", [mj.EPI_RELU, mj.EPI_RELU_UNARY, mj.EPI_GELU_TANH, mj.EPI_SILU,
                                 mj.EPI_GELU_TANH_APPROX, mj.EPI_SILU_APPROX])
def test_activation_kernel(oracle, dev, epi):
    x = np.concatenate([np.linspace(-30, 30, 6001, dtype=np.float32),
                        np.array([0.0, -0.0, 10.05, 10.1, 50.0, -50.0, 1e-30, -1e-30], np.float32),
                        oracle.randn_f32((5000,), seed=21)])
    y = torch.empty(x.size, dtype=torch.float32, device=dev)
    xd = to_dev(x, dev)
    _lib.call("mj_activation_f32", epi, xd.data_ptr(), y.data_ptr(), x.size,
              torch.cuda.current_stream().cuda_stream)
    got = y.cpu().numpy()
    ref = oracle.epilogue(epi, x)
    assert np.isfinite(got).all()
    assert_close_f32(got, ref, atol=1e-6, rtol=1e-5)


def test_tensor_gelu_is_finite_where_reference_overflows(oracle, dev):
    """gelu32's literal tanh is NaN past x ~ 10.06 (tensor/math.mojo:277-279);
    the backend returns the limit x there and matches gelu32 elsewhere."""
    x = np.array([10.0, 10.05, 10.1, 20.0, 100.0], np.float32)
    lit = oracle.gelu32_literal(x)
    assert np.isfinite(lit[:2]).all() and np.isnan(lit[2:]).all()
    got = mj.Tensor(to_dev(x, dev)).gelu().numpy()
    assert_close_f32(got[:2], lit[:2])
    np.testing.assert_array_equal(got[2:], x[2:])
