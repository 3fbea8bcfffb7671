"""GPU parity of Linear.backward (learn/nn/layers.mojo:519-618) and of the
autograd MATMUL2D rule (tensor/autograd.mojo:1542-1555) against the oracle.

Bars: dx, dW (fp32 MFMA, blocks of 4 in the reduction) |d| <= 1e-5 + 1e-5|ref|
at C1 size and the fp32 bound 2 K 2^-24 (|A||B|) elsewhere; db bit-exact
while N <= 1024 (strict ascending-n order, as the reference) and within the
bound beyond (row segments); integer-valued inputs bit-exact everywhere;
fp64 within 2 K 2^-53 (|A||B|).
"""
import ctypes

import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib
from _util import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu


def _lin(x, W, dev):
    lin = mj.Linear(x.shape[1], W.shape[0])
    lin.weight = mj.Tensor(to_dev(W, dev))
    return lin


def _bound(A, B, eps):
    K = A.shape[1]
    return 2.0 * K * eps * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))


def test_c1_linear_backward(oracle, dev):
    x = oracle.randn_f32((256, 256), seed=11)
    W = oracle.randn_f32((256, 256), seed=12)
    dy = oracle.randn_f32((256, 256), seed=13)
    dW, db, dx = _lin(x, W, dev).backward(mj.Tensor(to_dev(x, dev)), mj.Tensor(to_dev(dy, dev)))
    rW, rb, rx = oracle.linear_backward_f32(x, W, dy)
    assert_close_f32(dW.numpy(), rW)
    assert_close_f32(dx.numpy(), rx)
    np.testing.assert_array_equal(db.numpy(), rb)


@pytest.mark.parametrize("N,InF,OutF", [(1, 1, 1), (33, 70, 17), (64, 64, 64), (300, 7, 129),
                                        (5, 1000, 40)])
def test_linear_backward_ragged(oracle, dev, N, InF, OutF):
    x = oracle.randn_f32((N, InF), seed=N + InF)
    W = oracle.randn_f32((OutF, InF), seed=OutF + 3)
    dy = oracle.randn_f32((N, OutF), seed=N * 7 + OutF)
    dW, db, dx = _lin(x, W, dev).backward(mj.Tensor(to_dev(x, dev)), mj.Tensor(to_dev(dy, dev)))
    rW, rb, rx = oracle.linear_backward_f32(x, W, dy)
    assert np.all(np.abs(dW.numpy() - rW) <= _bound(dy.T, x, 2.0 ** -24) + 1e-30)
    assert np.all(np.abs(dx.numpy() - rx) <= _bound(dy, W, 2.0 ** -24) + 1e-30)
    np.testing.assert_array_equal(db.numpy(), rb)


def test_linear_backward_integer_exact(oracle, dev):
    rng = np.random.default_rng(21)
    x = rng.integers(-8, 9, size=(200, 96)).astype(np.float32)
    W = rng.integers(-8, 9, size=(72, 96)).astype(np.float32)
    dy = rng.integers(-8, 9, size=(200, 72)).astype(np.float32)
    dW, db, dx = _lin(x, W, dev).backward(mj.Tensor(to_dev(x, dev)), mj.Tensor(to_dev(dy, dev)))
    rW, rb, rx = oracle.linear_backward_f32(x, W, dy)
    np.testing.assert_array_equal(dW.numpy(), rW)
    np.testing.assert_array_equal(db.numpy(), rb)
    np.testing.assert_array_equal(dx.numpy(), rx)


def test_linear_backward_db_segmented(oracle, dev):
    """N > 1024 sums db in row segments: integer data stays exact, random data
    within the fp32 summation bound of the strict-order oracle."""
    rng = np.random.default_rng(22)
    N, InF, OutF = 4096, 8, 300
    x = rng.standard_normal((N, InF)).astype(np.float32)
    W = rng.standard_normal((OutF, InF)).astype(np.float32)
    dy = rng.standard_normal((N, OutF)).astype(np.float32)
    _, db, _ = _lin(x, W, dev).backward(mj.Tensor(to_dev(x, dev)), mj.Tensor(to_dev(dy, dev)))
    _, rb, _ = oracle.linear_backward_f32(x, W, dy)
    exact = dy.astype(np.float64).sum(0)
    bound = 2 * N * 2.0 ** -24 * np.abs(dy).astype(np.float64).sum(0)
    assert np.all(np.abs(db.numpy() - exact) <= bound)
    assert np.all(np.abs(rb - exact) <= bound)
    dyi = rng.integers(-50, 51, size=(N, OutF)).astype(np.float32)
    _, dbi, _ = _lin(x, W, dev).backward(mj.Tensor(to_dev(x, dev)), mj.Tensor(to_dev(dyi, dev)))
    np.testing.assert_array_equal(dbi.numpy(), dyi.astype(np.int64).sum(0).astype(np.float32))


def test_linear_backward_bad_shapes(dev):
    lin = mj.Linear(4, 3)
    x = mj.Tensor(torch.ones((5, 4), device=dev))
    dW, db, dx = lin.backward(x, mj.Tensor(torch.ones((6, 3), device=dev)))
    assert dW.shape() == [3, 4] and db.shape() == [3] and dx.shape() == [5, 4]
    assert not dW.numpy().any() and not db.numpy().any() and not dx.numpy().any()
    dW, db, dx = lin.backward(x, mj.Tensor(torch.ones((5, 2), device=dev)))
    assert not dW.numpy().any()


def _f32p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_host_seams(oracle, dev):
    """mj_launch_linear_bw_{dx,dw,db}_h: host buffers in and out, the layouts
    of the seam's CPU kernels (w, dW [OutF, InF])."""
    N, InF, OutF = 48, 40, 24
    x = oracle.randn_f32((N, InF), seed=31)
    W = oracle.randn_f32((OutF, InF), seed=32)
    dy = oracle.randn_f32((N, OutF), seed=33)
    rW, rb, rx = oracle.linear_backward_f32(x, W, dy)
    dx = np.empty((N, InF), np.float32)
    dW = np.empty((OutF, InF), np.float32)
    db = np.empty(OutF, np.float32)
    _lib.call("mj_launch_linear_bw_dx_h", _f32p(dy), _f32p(W), _f32p(dx), N, InF, OutF)
    _lib.call("mj_launch_linear_bw_dw_h", _f32p(dy), _f32p(x), _f32p(dW), N, InF, OutF)
    _lib.call("mj_launch_linear_bw_db_h", _f32p(dy), _f32p(db), N, OutF)
    assert_close_f32(dx, rx)
    assert_close_f32(dW, rW)
    np.testing.assert_array_equal(db, rb)


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (64, 64, 64), (70, 33, 129), (200, 300, 17)])
def test_matmul_backward_f64(oracle, dev, M, K, N):
    rng = np.random.default_rng(M * 3 + K + N)
    a = rng.standard_normal((M, K))
    b = rng.standard_normal((K, N))
    g = rng.standard_normal((M, N))
    ga, gb = mj.matmul_backward(mj.Tensor(to_dev(a, dev)), mj.Tensor(to_dev(b, dev)),
                                mj.Tensor(to_dev(g, dev)))
    ra, rb = oracle.matmul_backward_f64(a, b, g)
    assert np.all(np.abs(ga.numpy() - ra) <= _bound(g, b.T, 2.0 ** -53) + 1e-300)
    assert np.all(np.abs(gb.numpy() - rb) <= _bound(a.T, g, 2.0 ** -53) + 1e-300)


def test_matmul_backward_f64_accumulate_exact(oracle, dev):
    rng = np.random.default_rng(41)
    a = rng.integers(-2**15, 2**15, size=(90, 40)).astype(np.float64)
    b = rng.integers(-2**15, 2**15, size=(40, 70)).astype(np.float64)
    g = rng.integers(-2**15, 2**15, size=(90, 70)).astype(np.float64)
    ga0 = rng.integers(-2**20, 2**20, size=(90, 40)).astype(np.float64)
    gb0 = rng.integers(-2**20, 2**20, size=(40, 70)).astype(np.float64)
    ga, gb = mj.matmul_backward(mj.Tensor(to_dev(a, dev)), mj.Tensor(to_dev(b, dev)),
                                mj.Tensor(to_dev(g, dev)), mj.Tensor(to_dev(ga0, dev)),
                                mj.Tensor(to_dev(gb0, dev)))
    ra, rb = oracle.matmul_backward_f64(a, b, g, ga0, gb0)
    np.testing.assert_array_equal(ga.numpy(), ra)
    np.testing.assert_array_equal(gb.numpy(), rb)
