"""The autograd matmul node on the GPU (tensor/autograd.mojo:930-1017,
1352-, 1542-1555): mj_matmul_backward_f32 against the oracle's Float32 rule,
GradTensor.matmul / matmul2d recording and backward on a device-resident
tape, directional derivatives of the recorded chain, and the Tensor[Int]
upcast of Tensor.matmul / matmul_vec (tensor/tensor.mojo:3161-3165,
3174-3178).

Bars: bit-exact on integer-valued data (every order exact), |d| <= 1e-5 +
1e-5 |ref| on random fp32 data, directional derivatives within 1e-4
relative (fp64 closed forms).
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib
from momijo_amd.autograd import GradContext, GradTensor, no_grad_begin, no_grad_end
from _util import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu


def _ints(rng, shape):
    return rng.integers(-5, 6, size=shape).astype(np.float32)


@pytest.mark.parametrize("M,K,N", [(7, 5, 9), (64, 48, 80), (300, 130, 257)])
def test_matmul_backward_f32_device(oracle, dev, M, K, N):
    rng = np.random.default_rng(M + K + N)
    a, b, g = _ints(rng, (M, K)), _ints(rng, (K, N)), _ints(rng, (M, N))
    ga0, gb0 = _ints(rng, (M, K)), _ints(rng, (K, N))
    da, db = to_dev(ga0, dev), to_dev(gb0, dev)
    ta, tb, tg = to_dev(a, dev), to_dev(b, dev), to_dev(g, dev)
    _lib.call("mj_matmul_backward_f32", M, N, K, ta.data_ptr(), tb.data_ptr(), tg.data_ptr(),
              da.data_ptr(), db.data_ptr(), 1, torch.cuda.current_stream().cuda_stream)
    ra, rb = oracle.matmul_backward_f32(a, b, g, ga0, gb0)
    np.testing.assert_array_equal(da.cpu().numpy(), ra)
    np.testing.assert_array_equal(db.cpu().numpy(), rb)
    # random data, overwrite mode, one output skipped
    a, b, g = (oracle.randn_f32(s, seed=i) for i, s in enumerate(((M, K), (K, N), (M, N))))
    out = torch.empty((M, K), dtype=torch.float32, device=dev)
    ta, tb, tg = to_dev(a, dev), to_dev(b, dev), to_dev(g, dev)
    _lib.call("mj_matmul_backward_f32", M, N, K, ta.data_ptr(), tb.data_ptr(), tg.data_ptr(),
              out.data_ptr(), None, 0, torch.cuda.current_stream().cuda_stream)
    assert_close_f32(out.cpu().numpy(), oracle.matmul_backward_f32(a, b, g)[0])


def _leaf(ctx, arr, dev, rg=True):
    return GradTensor.from_tensor(ctx, mj.Tensor(to_dev(arr, dev)), rg)


def test_grad_tensor_chain_integer_exact(oracle, dev):
    """y = (A @ B) @ C with C a plain tensor: the tape holds leaf A, leaf B,
    node T = A@B, leaf C, node y; backward seeds ones at y and must give the
    oracle's Float32 rule applied down the chain, bit for bit."""
    rng = np.random.default_rng(40)
    A, B, C = _ints(rng, (6, 4)), _ints(rng, (4, 5)), _ints(rng, (5, 3))
    ctx = GradContext()
    a, b = _leaf(ctx, A, dev), _leaf(ctx, B, dev)
    t = a.matmul(ctx, b)
    y = t.matmul(ctx, mj.Tensor(to_dev(C, dev)))
    assert y.requires_grad and ctx.tape.op_tags == [0, 0, 18, 0, 18]
    np.testing.assert_array_equal(y.value(ctx).numpy(), (A @ B) @ C)
    y.backward(ctx)
    ones = np.ones((6, 3), np.float32)
    gT, gC = oracle.matmul_backward_f32(A @ B, C, ones)
    gA, gB = oracle.matmul_backward_f32(A, B, gT)
    np.testing.assert_array_equal(t.grad(ctx).numpy(), gT)
    np.testing.assert_array_equal(a.grad(ctx).numpy(), gA)
    np.testing.assert_array_equal(b.grad(ctx).numpy(), gB)
    np.testing.assert_array_equal(ctx.tape.grads[3].numpy(), gC)   # C's leaf, as the reference


def test_grad_tensor_directional_derivative(oracle, dev):
    """L = sum((A @ B) @ C): dL/dA . E = sum((E @ B) @ C), dL/dB . F =
    sum((A @ F) @ C), in fp64."""
    rng = np.random.default_rng(41)
    A, B, C = (rng.standard_normal(s).astype(np.float32) for s in ((32, 24), (24, 40), (40, 8)))
    E, F = rng.standard_normal(A.shape), rng.standard_normal(B.shape)
    ctx = GradContext()
    a, b, c = _leaf(ctx, A, dev), _leaf(ctx, B, dev), _leaf(ctx, C, dev, False)
    y = a.matmul2d(ctx, b).matmul2d(ctx, c)
    y.backward(ctx)
    A64, B64, C64 = (t.astype(np.float64) for t in (A, B, C))
    dA, dB = a.grad(ctx).numpy().astype(np.float64), b.grad(ctx).numpy().astype(np.float64)
    np.testing.assert_allclose(np.sum(dA * E), np.sum((E @ B64) @ C64), rtol=1e-4)
    np.testing.assert_allclose(np.sum(dB * F), np.sum((A64 @ F) @ C64), rtol=1e-4)


def test_grad_tensor_tracking_rules(dev):
    ctx = GradContext()
    x = GradTensor.from_tensor(ctx, mj.Tensor(torch.ones((3, 3), device=dev)))
    w = GradTensor.from_tensor(ctx, mj.Tensor(torch.ones((3, 3), device=dev)), True)
    assert not x.matmul(ctx, x).requires_grad          # no parent requires grad: a leaf
    no_grad_begin(ctx)
    assert not x.matmul(ctx, w).requires_grad          # no_grad: a leaf
    assert not GradTensor.from_tensor(ctx, mj.Tensor(torch.ones(2, device=dev)), True).requires_grad
    no_grad_end(ctx)
    assert x.matmul(ctx, w).requires_grad


def test_grad_tensor_self_product(oracle, dev):
    """y = X @ X: both parents are the same node, so its gradient receives
    g X^T and then X^T g (the reference adds p0's, then p1's)."""
    rng = np.random.default_rng(42)
    X = _ints(rng, (5, 5))
    ctx = GradContext()
    x = _leaf(ctx, X, dev)
    y = x.matmul(ctx, x)
    y.backward(ctx)
    ones = np.ones((5, 5), np.float32)
    ga, _ = oracle.matmul_backward_f32(X, X, ones)
    _, gb = oracle.matmul_backward_f32(X, X, ones, None, np.zeros((5, 5), np.float32))
    np.testing.assert_array_equal(x.grad(ctx).numpy(), ga + gb)


def test_int_tensor_matmul_upcasts_to_float32(oracle, dev):
    rng = np.random.default_rng(43)
    A = rng.integers(-1000, 1000, size=(9, 7))
    B = rng.integers(-1000, 1000, size=(7, 4))
    x = rng.integers(-1000, 1000, size=7)
    got = mj.Tensor(torch.from_numpy(A).to(dev)).matmul(mj.Tensor(torch.from_numpy(B).to(dev)))
    assert got.dtype == torch.float32
    np.testing.assert_array_equal(got.numpy(), oracle.matmul_f32(A.astype(np.float32),
                                                                 B.astype(np.float32)))
    v = mj.Tensor(torch.from_numpy(A).to(dev)).matmul_vec(mj.Tensor(torch.from_numpy(x).to(dev)))
    assert v.dtype == torch.float32
    np.testing.assert_array_equal(v.numpy(), oracle.matvec_f32(A.astype(np.float32),
                                                               x.astype(np.float32)))


def test_int_upcast_rounds_like_astype_f32_from_int(oracle, dev):
    """Integers beyond 2^24 round to nearest even in the library's cast
    kernel, as astype_f32_from_int does (tensor/cast.mojo:5431-5437); the
    product then runs on the rounded Float32 values."""
    p24 = 1 << 24
    vals = np.array([p24 + 1, p24 + 3, -(p24 + 1), (1 << 40) + (1 << 16),
                     (1 << 40) + (1 << 16) + 1, (1 << 62) + 12345, -(1 << 63), 5], np.int64)
    rng = np.random.default_rng(44)
    big = rng.integers(-(1 << 63), (1 << 63) - 1, size=4096, dtype=np.int64)
    got = mj.tensor.astype_f32_from_int(torch.from_numpy(np.concatenate([vals, big])).to(dev))
    want = oracle.astype_f32_from_int(np.concatenate([vals, big]))
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    A = rng.integers(p24, 4 * p24, size=(6, 5))
    B = rng.integers(-3, 4, size=(5, 3))
    c = mj.Tensor(torch.from_numpy(A).to(dev)).matmul(mj.Tensor(torch.from_numpy(B).to(dev)))
    # the rounded operands' products are not exact in fp32: the fp32 bar
    assert_close_f32(c.numpy(), oracle.matmul_f32(oracle.astype_f32_from_int(A),
                                                  oracle.astype_f32_from_int(B)))


def test_maximum_scalar_keeps_negative_zero(oracle, dev):
    """Tensor.maximum_scalar(s) = where(x >= s, x, s) (tensor/tensor.mojo:4232)
    for s = 0 and other s, bit for bit (signed zeros, NaN, s itself)."""
    x = np.concatenate([np.array([-0.0, 0.0, np.nan, -np.nan, np.inf, -np.inf, 0.25, -2.0],
                                 np.float32),
                        oracle.randn_f32((10_000,), seed=45)])
    for s in (0.0, 0.25, -2.0, 1.5):
        got = mj.Tensor(to_dev(x, dev)).maximum_scalar(s).numpy()
        want = oracle.maximum_scalar_f32(x, s)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    y0 = mj.Tensor(to_dev(x, dev)).maximum_scalar(0.0).numpy()
    assert np.signbit(y0[0]) and y0[2] == 0
    # ReLU.forward (layers.mojo's _maximum_scalar: v > 0 ? v : 0) maps -0 to +0
    r = mj.ReLU().forward(mj.Tensor(to_dev(x, dev))).numpy()
    assert not np.signbit(r[0])
