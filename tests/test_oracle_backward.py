"""Pins the oracle's Linear.backward (learn/nn/layers.mojo:519-618) and the
autograd MATMUL2D rule (tensor/autograd.mojo:1542-1555).

Independent checks: integer-valued inputs (exact in any order) against int64
products; the strict summation order against one-rounding-per-step numpy
loops; and directional derivatives of the scalar L = <dy, x W^T> (and
L = <g, a b>), which fix which operand is transposed: a swapped or transposed
gradient fails them.
"""
import numpy as np


def test_linear_backward_integer_exact(oracle):
    rng = np.random.default_rng(1)
    x = rng.integers(-20, 21, size=(13, 9))
    W = rng.integers(-20, 21, size=(6, 9))
    dy = rng.integers(-20, 21, size=(13, 6))
    dW, db, dx = oracle.linear_backward_f32(x, W, dy)
    np.testing.assert_array_equal(dW, (dy.T @ x).astype(np.float32))
    np.testing.assert_array_equal(db, dy.sum(0).astype(np.float32))
    np.testing.assert_array_equal(dx, (dy @ W).astype(np.float32))


def test_linear_backward_strict_order(oracle):
    rng = np.random.default_rng(2)
    N, InF, OutF = 37, 11, 19
    x = rng.standard_normal((N, InF)).astype(np.float32)
    W = rng.standard_normal((OutF, InF)).astype(np.float32)
    dy = rng.standard_normal((N, OutF)).astype(np.float32)
    dW, db, dx = oracle.linear_backward_f32(x, W, dy)
    s = np.zeros(OutF, np.float32)
    for n in range(N):
        s = s + dy[n]
    np.testing.assert_array_equal(db, s)
    acc = np.zeros((N, InF), np.float32)
    for o in range(OutF):
        acc = acc + np.multiply.outer(dy[:, o], W[o])
    np.testing.assert_array_equal(dx, acc)
    accw = np.zeros((OutF, InF), np.float32)
    for n in range(N):
        accw = accw + np.multiply.outer(dy[n], x[n])
    np.testing.assert_array_equal(dW, accw)


def test_linear_backward_directional_derivatives(oracle):
    """L(W, x, b) = sum(dy * (x W^T + b)) is linear in each argument, so a
    central difference along any direction equals <grad, direction> to
    rounding."""
    rng = np.random.default_rng(3)
    N, InF, OutF = 8, 5, 7
    x = rng.standard_normal((N, InF))
    W = rng.standard_normal((OutF, InF))
    dy = rng.standard_normal((N, OutF))
    dW, db, dx = oracle.linear_backward_f32(x, W, dy)

    def L(x_, W_, b_):
        return float(np.sum(dy * (x_ @ W_.T + b_)))

    b = np.zeros(OutF)
    V = rng.standard_normal(W.shape)
    U = rng.standard_normal(x.shape)
    c = rng.standard_normal(OutF)
    h = 1e-3
    dL_W = (L(x, W + h * V, b) - L(x, W - h * V, b)) / (2 * h)
    dL_x = (L(x + h * U, W, b) - L(x - h * U, W, b)) / (2 * h)
    dL_b = (L(x, W, b + h * c) - L(x, W, b - h * c)) / (2 * h)
    assert abs(dL_W - np.sum(dW * V)) < 1e-4 * (1 + abs(dL_W))
    assert abs(dL_x - np.sum(dx * U)) < 1e-4 * (1 + abs(dL_x))
    assert abs(dL_b - np.sum(db * c)) < 1e-4 * (1 + abs(dL_b))


def test_matmul_backward_f64(oracle):
    rng = np.random.default_rng(4)
    M, K, N = 6, 9, 4
    a = rng.standard_normal((M, K))
    b = rng.standard_normal((K, N))
    g = rng.standard_normal((M, N))
    da, db = oracle.matmul_backward_f64(a, b, g)

    def L(a_, b_):
        return float(np.sum(g * (a_ @ b_)))

    V = rng.standard_normal(a.shape)
    U = rng.standard_normal(b.shape)
    h = 1e-4
    assert abs((L(a + h * V, b) - L(a - h * V, b)) / (2 * h) - np.sum(da * V)) < 1e-8
    assert abs((L(a, b + h * U) - L(a, b - h * U)) / (2 * h) - np.sum(db * U)) < 1e-8
    # strict inner order of matmul2d (math.mojo:7864-7871)
    acc = np.zeros((M, K))
    for j in range(N):
        acc = acc + np.multiply.outer(g[:, j], b[:, j])
    np.testing.assert_array_equal(da, acc)


def test_matmul_backward_accumulates(oracle):
    rng = np.random.default_rng(5)
    a = rng.integers(-9, 10, size=(5, 3)).astype(np.float64)
    b = rng.integers(-9, 10, size=(3, 4)).astype(np.float64)
    g = rng.integers(-9, 10, size=(5, 4)).astype(np.float64)
    ga0 = rng.integers(-9, 10, size=(5, 3)).astype(np.float64)
    gb0 = rng.integers(-9, 10, size=(3, 4)).astype(np.float64)
    da, db = oracle.matmul_backward_f64(a, b, g, ga0, gb0)
    np.testing.assert_array_equal(da, ga0 + g @ b.T)
    np.testing.assert_array_equal(db, gb0 + a.T @ g)


# ------------------------------------------------------------- Float32 tape rule
def test_matmul_backward_f32_integer_exact(oracle):
    """Integer-valued operands: every product and partial sum is exact in
    fp32, so da = g b^T and db = a^T g must equal the int64 products; a
    swapped or untransposed operand would fail (the shapes are all distinct)."""
    rng = np.random.default_rng(31)
    M, K, N = 7, 5, 9
    a = rng.integers(-6, 7, size=(M, K)).astype(np.float32)
    b = rng.integers(-6, 7, size=(K, N)).astype(np.float32)
    g = rng.integers(-6, 7, size=(M, N)).astype(np.float32)
    da, db = oracle.matmul_backward_f32(a, b, g)
    ai, bi, gi = (t.astype(np.int64) for t in (a, b, g))
    np.testing.assert_array_equal(da, gi @ bi.T)
    np.testing.assert_array_equal(db, ai.T @ gi)


def test_matmul_backward_f32_strict_order(oracle):
    """The Float32 products are summed in ascending inner index with one
    rounding per step, as the Float32 matmul does; the accumulated form adds
    the rounded sum onto the old gradient with one more rounding."""
    rng = np.random.default_rng(32)
    M, K, N = 4, 3, 37
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)
    ga0 = rng.standard_normal((M, K)).astype(np.float32)
    da, _ = oracle.matmul_backward_f32(a, b, g, ga0, None)
    for i in range(M):
        for k in range(K):
            acc = np.float32(0)
            for j in range(N):
                acc = np.float32(acc + np.float32(g[i, j] * b[k, j]))
            assert da[i, k] == np.float32(ga0[i, k] + acc)


def test_matmul_backward_f32_directional_derivative(oracle):
    """For L = <g, a @ b>: dL/da . E = <g, E @ b> and dL/db . F = <g, a @ F>
    (fp64 closed forms)."""
    rng = np.random.default_rng(33)
    M, K, N = 16, 24, 12
    a, b, g = (rng.standard_normal(s).astype(np.float32) for s in ((M, K), (K, N), (M, N)))
    E, F = rng.standard_normal((M, K)), rng.standard_normal((K, N))
    da, db = oracle.matmul_backward_f32(a, b, g)
    a64, b64, g64 = (t.astype(np.float64) for t in (a, b, g))
    np.testing.assert_allclose(np.sum(da * E), np.sum(g64 * (E @ b64)), rtol=1e-5)
    np.testing.assert_allclose(np.sum(db * F), np.sum(g64 * (a64 @ F)), rtol=1e-5)
