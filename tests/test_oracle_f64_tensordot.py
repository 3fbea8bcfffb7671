"""Pins the oracle's Float64 engine (matmul_core_mm / matmul_core_vec Float64,
tensor/broadcast.mojo:1397-1541; matmul2d, tensor/math.mojo:7838-7880) and
tensordot axes=1 (tensor/broadcast.mojo:1694-1900).

Independent checks: integer-valued inputs exact in any order (compared with an
int64 product), identity / permutation closed forms, the strict-k order (equal
to a left-to-right sum done in numpy, one rounding per step), and for
tensordot: per-batch equality with the already-pinned fp32 matmul, broadcast
batches equal to their materialised copies, and an int64 einsum.
"""
import numpy as np
import pytest


def test_f64_integer_inputs_exact(oracle):
    rng = np.random.default_rng(5)
    A = rng.integers(-2**20, 2**20, size=(23, 70))
    B = rng.integers(-2**20, 2**20, size=(70, 31))
    got = oracle.matmul_f64(A.astype(np.float64), B.astype(np.float64))
    np.testing.assert_array_equal(got, (A @ B).astype(np.float64))


def test_f64_identity_and_permutation(oracle):
    A = np.random.default_rng(1).standard_normal((17, 17))
    I = np.eye(17)
    np.testing.assert_array_equal(oracle.matmul_f64(A, I), A)
    np.testing.assert_array_equal(oracle.matmul_f64(I, A), A)
    P = I[np.random.default_rng(2).permutation(17)]
    np.testing.assert_array_equal(oracle.matmul_f64(P, A), P @ A)


def test_f64_strict_k_order(oracle):
    """acc = acc + a[i,t] * b[t,j] for t = 0..K-1, one rounding per op
    (math.mojo:7866-7870): a numpy loop over t does the same steps."""
    rng = np.random.default_rng(3)
    A = rng.standard_normal((9, 41))
    B = rng.standard_normal((41, 7))
    acc = np.zeros((9, 7))
    for t in range(41):
        acc = acc + np.multiply.outer(A[:, t], B[t, :])
    np.testing.assert_array_equal(oracle.matmul_f64(A, B), acc)


def test_f64_views(oracle):
    rng = np.random.default_rng(4)
    W = rng.integers(-50, 50, size=(30, 12)).astype(np.float64)
    x = rng.integers(-50, 50, size=(8, 12)).astype(np.float64)
    np.testing.assert_array_equal(oracle.matmul_f64(x, W.T), (x @ W.T))


def test_matvec_f64(oracle):
    rng = np.random.default_rng(6)
    A = rng.integers(-1000, 1000, size=(33, 57))
    x = rng.integers(-1000, 1000, size=57)
    got = oracle.matvec_f64(A.astype(np.float64), x.astype(np.float64))
    np.testing.assert_array_equal(got, (A @ x).astype(np.float64))
    acc = np.zeros(33)
    Af, xf = rng.standard_normal((33, 57)), rng.standard_normal(57)
    for t in range(57):
        acc = acc + Af[:, t] * xf[t]
    np.testing.assert_array_equal(oracle.matvec_f64(Af, xf), acc)


def test_tensordot_2d_equals_matmul(oracle):
    A = oracle.randn_f32((13, 29), seed=1)
    B = oracle.randn_f32((29, 11), seed=2)
    np.testing.assert_array_equal(oracle.tensordot_f32(A, B), oracle.matmul_f32(A, B))


def test_tensordot_batched_per_slice(oracle):
    A = oracle.randn_f32((3, 4, 9, 20), seed=3)
    B = oracle.randn_f32((3, 4, 20, 6), seed=4)
    got = oracle.tensordot_f32(A, B)
    assert got.shape == (3, 4, 9, 6)
    for i in range(3):
        for j in range(4):
            np.testing.assert_array_equal(got[i, j], oracle.matmul_f32(A[i, j], B[i, j]))


def test_tensordot_broadcast_equals_materialised(oracle):
    A = oracle.randn_f32((2, 1, 5, 8), seed=5)
    B = oracle.randn_f32((3, 8, 4), seed=6)
    got = oracle.tensordot_f32(A, B)
    assert got.shape == (2, 3, 5, 4)
    Am = np.ascontiguousarray(np.broadcast_to(A, (2, 3, 5, 8)))
    Bm = np.ascontiguousarray(np.broadcast_to(B, (2, 3, 8, 4)))
    np.testing.assert_array_equal(got, oracle.tensordot_f32(Am, Bm))


def test_tensordot_integer_einsum(oracle):
    rng = np.random.default_rng(7)
    A = rng.integers(-9, 10, size=(4, 1, 6, 33))
    B = rng.integers(-9, 10, size=(1, 5, 33, 7))
    got = oracle.tensordot_f32(A.astype(np.float32), B.astype(np.float32))
    Ab = np.broadcast_to(A, (4, 5, 6, 33))
    Bb = np.broadcast_to(B, (4, 5, 33, 7))
    ref = np.einsum("abmk,abkn->abmn", Ab, Bb)
    np.testing.assert_array_equal(got, ref.astype(np.float32))


def test_tensordot_strided_inner(oracle):
    """Transposed inner views take the generic strided path
    (broadcast.mojo:1906-1935)."""
    rng = np.random.default_rng(8)
    At = rng.integers(-9, 10, size=(2, 21, 6)).astype(np.float32)  # stored [K, M]
    A = np.swapaxes(At, -1, -2)
    B = rng.integers(-9, 10, size=(2, 21, 5)).astype(np.float32)
    got = oracle.tensordot_f32(A, B)
    np.testing.assert_array_equal(got, np.einsum("bmk,bkn->bmn", A.astype(np.int64),
                                                 B.astype(np.int64)).astype(np.float32))
