"""GPU parity of the Float64 engine (matmul / matmul_vec Float64, matmul2d)
and tensordot axes=1 against the oracle.

Bars: fp64 -- |gpu - oracle| <= 2 K 2^-53 (|A| @ |B|) elementwise, the
standard bound for two summation orders of the same products (the MFMA
kernel sums in blocks of 4, the oracle in strict k order); bit-equality for
integer-valued operands.  fp32 tensordot -- 1e-5 abs + 1e-5 rel, as the fp32
matmul.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from _util import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu


def _assert_close_f64(got, ref, A, B):
    K = A.shape[1]
    bound = 2.0 * K * 2.0 ** -53 * (np.abs(A) @ np.abs(B)) + 1e-300
    err = np.abs(got - ref)
    assert np.all(err <= bound), f"max err {err.max()} over bound {bound[err > bound].min()}"


def _mm64(A, B, dev):
    return mj.matmul(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev))).numpy()


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (64, 64, 16), (65, 33, 100), (200, 130, 257)])
def test_f64_matmul_ragged(oracle, dev, M, N, K):
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K))
    B = rng.standard_normal((K, N))
    got = _mm64(A, B, dev)
    assert got.dtype == np.float64
    _assert_close_f64(got, oracle.matmul_f64(A, B), A, B)


def test_f64_integer_exact(oracle, dev):
    rng = np.random.default_rng(11)
    A = rng.integers(-2**20, 2**20, size=(70, 130)).astype(np.float64)
    B = rng.integers(-2**20, 2**20, size=(130, 90)).astype(np.float64)
    np.testing.assert_array_equal(_mm64(A, B, dev), oracle.matmul_f64(A, B))


@pytest.mark.parametrize("tb", [False, True])
def test_f64_large_tiles_integer_exact(oracle, dev, tb):
    """3000 x 2900 outputs on the 128 x 128 fp64 tile: integer operands
    below 2^20 keep every sum exact (|sum| < 2^53), so bit-identical."""
    rng = np.random.default_rng(13 + tb)
    M, N, K = 3000, 2900, 40
    A = rng.integers(-2**20, 2**20, size=(M, K)).astype(np.float64)
    B = rng.integers(-2**20, 2**20, size=(K, N)).astype(np.float64)
    b = mj.Tensor(to_dev(B, dev)) if not tb else \
        mj.Tensor(to_dev(np.ascontiguousarray(B.T), dev)).transpose()
    got = mj.matmul(mj.Tensor(to_dev(A, dev)), b).numpy()
    np.testing.assert_array_equal(got, oracle.matmul_f64(A, B))


def test_f64_transposed_views(oracle, dev):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((40, 75))
    W = rng.standard_normal((55, 75))
    got = mj.Tensor(to_dev(x, dev)).matmul(mj.Tensor(to_dev(W, dev)).transpose()).numpy()
    _assert_close_f64(got, oracle.matmul_f64(x, W.T), x, W.T)


def test_f64_matvec(oracle, dev):
    rng = np.random.default_rng(13)
    A = rng.standard_normal((77, 300))
    x = rng.standard_normal(300)
    got = mj.Tensor(to_dev(A, dev)).matmul_vec(mj.Tensor(to_dev(x, dev))).numpy()
    _assert_close_f64(got[:, None], oracle.matvec_f64(A, x)[:, None], A, x[:, None])
    Ai = rng.integers(-1000, 1000, size=(31, 65)).astype(np.float64)
    xi = rng.integers(-1000, 1000, size=65).astype(np.float64)
    got = mj.matmul(mj.Tensor(to_dev(Ai, dev)), mj.Tensor(to_dev(xi, dev))).numpy()
    np.testing.assert_array_equal(got, oracle.matvec_f64(Ai, xi))


def test_matmul2d(oracle, dev):
    rng = np.random.default_rng(14)
    A = rng.integers(-99, 99, size=(12, 20)).astype(np.float64)
    B = rng.integers(-99, 99, size=(20, 9)).astype(np.float64)
    got = mj.matmul2d(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev))).numpy()
    np.testing.assert_array_equal(got, oracle.matmul_f64(A, B))


def test_f64_bad_shapes(dev):
    """matmul2d returns zeros([m, n]) on a bad inner dimension
    (math.mojo:7857-7858); matmul returns an empty tensor."""
    a = mj.Tensor(torch.ones((3, 4), dtype=torch.float64, device=dev))
    b = mj.Tensor(torch.ones((5, 6), dtype=torch.float64, device=dev))
    z = mj.matmul2d(a, b)
    assert z.shape() == [3, 6] and not z.numpy().any()
    assert mj.matmul(a, b).numel() == 0
    assert mj.matmul(a, mj.Tensor(torch.ones(7, dtype=torch.float64, device=dev))).numel() == 0


def _td(A, B, dev):
    return mj.tensordot(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev)))


def test_tensordot_2d(oracle, dev):
    A = oracle.randn_f32((70, 129), seed=21)
    B = oracle.randn_f32((129, 65), seed=22)
    assert_close_f32(_td(A, B, dev).numpy(), oracle.tensordot_f32(A, B))


def test_tensordot_batched(oracle, dev):
    A = oracle.randn_f32((3, 4, 33, 50), seed=23)
    B = oracle.randn_f32((3, 4, 50, 17), seed=24)
    got = _td(A, B, dev)
    assert got.shape() == [3, 4, 33, 17]
    assert_close_f32(got.numpy(), oracle.tensordot_f32(A, B))


def test_tensordot_broadcast(oracle, dev):
    A = oracle.randn_f32((2, 1, 19, 40), seed=25)
    B = oracle.randn_f32((3, 40, 70), seed=26)
    got = _td(A, B, dev)
    assert got.shape() == [2, 3, 19, 70]
    assert_close_f32(got.numpy(), oracle.tensordot_f32(A, B))


def test_tensordot_five_batch_dims(oracle, dev):
    A = oracle.randn_f32((2, 1, 3, 1, 2, 5, 9), seed=27)
    B = oracle.randn_f32((1, 2, 1, 2, 1, 9, 4), seed=28)
    got = _td(A, B, dev)
    assert got.shape() == [2, 2, 3, 2, 2, 5, 4]
    assert_close_f32(got.numpy(), oracle.tensordot_f32(A, B))


def test_tensordot_strided_views(oracle, dev):
    """Transposed inner views (generic strided path, broadcast.mojo:1906-1935)."""
    At = oracle.randn_f32((2, 37, 21), seed=29)   # stored [b, K, M]
    B = oracle.randn_f32((2, 37, 44), seed=30)
    a = mj.Tensor(to_dev(At, dev)).transpose()   # [2, 21, 37] view
    got = mj.tensordot(a, mj.Tensor(to_dev(B, dev))).numpy()
    assert_close_f32(got, oracle.tensordot_f32(np.swapaxes(At, -1, -2), B))


def test_tensordot_many_batches(oracle, dev):
    """More batches than one launch's grid height holds (65535)."""
    rng = np.random.default_rng(31)
    A = rng.integers(-9, 10, size=(70001, 2, 3)).astype(np.float32)
    B = rng.integers(-9, 10, size=(70001, 3, 2)).astype(np.float32)
    got = _td(A, B, dev).numpy()
    ref = np.einsum("bmk,bkn->bmn", A.astype(np.int64), B.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(got, ref)


def test_tensordot_bad_inputs(dev):
    a = mj.Tensor(torch.ones((2, 3, 4), device=dev))
    assert mj.tensordot(a, mj.Tensor(torch.ones((5, 6), device=dev))).numel() == 0
    assert mj.tensordot(a, mj.Tensor(torch.ones((3, 4, 6), device=dev)), axes=2).numel() == 0
    assert mj.tensordot(a, mj.Tensor(torch.ones(4, device=dev))).numel() == 0
    assert mj.tensordot(a, mj.Tensor(torch.ones((4, 4, 6), device=dev))).numel() == 0
    e = mj.tensordot(mj.Tensor(torch.ones((0, 3, 4), device=dev)),
                     mj.Tensor(torch.ones((4, 6), device=dev)))
    assert e.shape() == [0, 3, 6]
