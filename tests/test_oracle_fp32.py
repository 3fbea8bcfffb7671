"""Pins the oracle's fp32 engine (tensor/broadcast.mojo:1543-1684,
learn/nn/layers.mojo:383-475) and its bf16 GEMM definition.

Independent checks: integer-valued inputs (exact in any order, compared with
an int64 product), identity / permutation closed forms, an fp64 brute-force
bound K*2^-24*sum|a||b|, torch CPU as a cross-check, and the strict-k order
itself (the oracle must equal a left-to-right fp32 sum done in numpy).
"""
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(__file__), "golden", "small_cases.npz")


def test_integer_inputs_exact(oracle):
    rng = np.random.default_rng(0)
    A = rng.integers(-8, 9, size=(40, 256))
    B = rng.integers(-8, 9, size=(256, 33))
    got = oracle.matmul_f32(A.astype(np.float32), B.astype(np.float32))
    np.testing.assert_array_equal(got, (A @ B).astype(np.float32))


def test_identity_and_permutation(oracle):
    A = oracle.randn_f32((24, 24), seed=1)
    I = np.eye(24, dtype=np.float32)
    np.testing.assert_array_equal(oracle.matmul_f32(A, I), A)
    np.testing.assert_array_equal(oracle.matmul_f32(I, A), A)
    P = I[np.random.default_rng(3).permutation(24)]
    np.testing.assert_array_equal(oracle.matmul_f32(P, A), P @ A)
    np.testing.assert_array_equal(oracle.matmul_f32(A, P), A @ P)


def test_fp64_bound(oracle):
    A = oracle.randn_f32((31, 200), seed=2)
    B = oracle.randn_f32((200, 29), seed=3)
    got = oracle.matmul_f32(A, B).astype(np.float64)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    bound = 200 * 2.0 ** -24 * (np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64))
    assert np.all(np.abs(got - ref) <= bound)


def test_strict_k_order(oracle):
    """acc = acc + a*b left to right in fp32, no FMA: a numpy loop with the
    same rounding sequence reproduces every bit."""
    A = oracle.randn_f32((6, 37), seed=4)
    B = oracle.randn_f32((37, 5), seed=5)
    exp = np.zeros((6, 5), np.float32)
    for k in range(37):
        exp = (exp + (A[:, k:k + 1] * B[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_f32(A, B), exp)


def test_torch_cross_check(oracle):
    A = oracle.randn_f32((64, 300), seed=6)
    B = oracle.randn_f32((300, 48), seed=7)
    ref = (torch.from_numpy(A).double() @ torch.from_numpy(B).double()).numpy()
    np.testing.assert_allclose(oracle.matmul_f32(A, B), ref, rtol=1e-4, atol=1e-4)


def test_strided_path_equals_contiguous(oracle):
    """The strided path (transpose views) keeps the same order, so a view and
    its contiguous copy give identical bits."""
    W = oracle.randn_f32((20, 64), seed=8)
    x = oracle.randn_f32((9, 64), seed=9)
    np.testing.assert_array_equal(oracle.matmul_f32(x, W.T), oracle.matmul_f32(x, W.T.copy()))
    np.testing.assert_array_equal(oracle.matmul_f32(W.T.T, x.T), oracle.matmul_f32(W, x.T.copy()))


def test_linear_contracts(oracle):
    x = oracle.randn_f32((7, 48), seed=10)
    W = oracle.randn_f32((13, 48), seed=11)
    b = oracle.randu_f32((13,), -1 / 16, 1 / 16, seed=12)
    y = oracle.linear_fw_f32(x, W, b)
    # bias added once after the strict-k dot (layers.mojo:426-427)
    np.testing.assert_array_equal(y, (oracle.matmul_f32(x, W.T) + b).astype(np.float32))
    # the device seam's CPU kernel on wT = W^T gives the same bits
    np.testing.assert_array_equal(oracle.kernel_linear_fw_f32(x, W.T.copy(), b), y)
    np.testing.assert_array_equal(oracle.linear_fw_f32(x, W, None), oracle.matmul_f32(x, W.T))
    relu = oracle.linear_act_f32(x, W, b, oracle.EPI_RELU)
    np.testing.assert_array_equal(relu, np.where(y > 0, y, 0).astype(np.float32))


def test_matvec(oracle):
    A = oracle.randn_f32((17, 70), seed=13)
    x = oracle.randn_f32((70,), seed=14)
    np.testing.assert_array_equal(oracle.matvec_f32(A, x), oracle.matmul_f32(A, x[:, None])[:, 0])


def test_bf16_conversion_matches_torch(oracle):
    v = np.concatenate([oracle.randn_f32((10000,), seed=15) * 1e3,
                        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.3895314e38, 1e-40,
                                  1.00390625, 1.01171875], np.float32)])
    ours = oracle.f32_to_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, ref)
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(oracle.bf16_to_f32(nan)).all()


def test_bf16_gemm_definition(oracle):
    """gemm_bf16_nt = strict-k fp32 dot on upcast bf16, bias, epilogue, RNE."""
    A = oracle.f32_to_bf16(oracle.randn_f32((12, 64), seed=16))
    B = oracle.f32_to_bf16(oracle.randn_f32((10, 64), seed=17))
    b = oracle.randu_f32((10,), -1 / 16, 1 / 16, seed=18)
    C, Cf = oracle.gemm_bf16_nt(A, B, b, oracle.EPI_GELU_TANH)
    Af, Bf = oracle.bf16_to_f32(A), oracle.bf16_to_f32(B)
    exp = oracle.epilogue(oracle.EPI_GELU_TANH, oracle.linear_fw_f32(Af, Bf, b))
    np.testing.assert_array_equal(Cf, exp)
    np.testing.assert_array_equal(C, oracle.f32_to_bf16(exp))
    # a row slab equals the same rows of the full product
    C2, _ = oracle.gemm_bf16_nt(A, B, b, oracle.EPI_GELU_TANH, rows=(3, 7))
    np.testing.assert_array_equal(C2, C[3:7])


def test_golden_small_cases(oracle):
    g = np.load(GOLD)
    np.testing.assert_array_equal(oracle.matmul_f32(g["mm_A"], g["mm_B"]), g["mm_C"])
    np.testing.assert_array_equal(
        oracle.linear_act_f32(g["lin_x"], g["lin_W"], g["lin_b"], oracle.EPI_RELU), g["lin_relu_y"])


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 0, 4)])
def test_degenerate_shapes(oracle, shape):
    M, N, K = shape
    A = np.ones((M, K), np.float32)
    B = np.ones((K, N), np.float32)
    C = oracle.matmul_f32(A, B)
    assert C.shape == (M, N)
    np.testing.assert_array_equal(C, np.full((M, N), K, np.float32))
