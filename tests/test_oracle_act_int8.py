"""Pins the oracle's activations (tensor/math.mojo:272-295,
learn/nn/activations.mojo:34-51,137-163) and int8 helpers
(learn/api/functional.mojo:206-302, learn/api/sequential.mojo:217-263), plus
the spec-only per-channel quantizer and W8A16 / MLP references.

Independent checks: closed forms in double precision, a numpy float32
restatement of the _exp_approx IEEE sequence, constructed rounding ties, the
fp32-add artifact, exact int32 products, integer-valued W8A16 inputs whose
sums are exact, and fp64 compositions for the MLP.
"""
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden", "small_cases.npz")
f32 = np.float32


# ------------------------------------------------------------------ activations
def test_tensor_engine_activations_closed_form(oracle):
    x = np.linspace(-9, 9, 20001).astype(np.float32)
    xd = x.astype(np.float64)
    gelu = 0.5 * xd * (1 + np.tanh(0.7978845608028654 * (xd + 0.044715 * xd ** 3)))
    silu = xd / (1 + np.exp(-xd))
    np.testing.assert_allclose(oracle.epilogue(oracle.EPI_GELU_TANH, x), gelu, rtol=2e-6, atol=2e-7)
    np.testing.assert_allclose(oracle.epilogue(oracle.EPI_SILU, x), silu, rtol=2e-6, atol=2e-7)


def test_gelu32_literal_overflow(oracle):
    """tanh32 = (e^{2t}-1)/(e^{2t}+1) overflows to NaN past x ~ 10.06."""
    lit = oracle.gelu32_literal(np.array([10.05, 10.1, -30.0], np.float32))
    assert np.isfinite(lit[0]) and np.isnan(lit[1])
    fin = oracle.epilogue(oracle.EPI_GELU_TANH, np.array([10.05, 10.1, 1e4], np.float32))
    assert fin[0] == lit[0] and fin[1] == f32(10.1) and fin[2] == f32(1e4)


def _exp_approx_np(x):
    xv = np.clip(np.float32(x), f32(-20), f32(20)).astype(np.float32)
    y = f32(f32(1.0) + f32(xv / f32(64.0)))
    for _ in range(6):
        y = f32(y * y)
    return y


def test_exp_approx_exact_sequence(oracle):
    for v in np.linspace(-25, 25, 1001).astype(np.float32):
        assert oracle.exp_approx32(float(v)) == _exp_approx_np(v)
    assert oracle.exp_approx32(0.0) == 1.0
    assert oracle.exp_approx32(50.0) == oracle.exp_approx32(20.0)
    # (1 + 1/64)^64 is 0.8% under e, as the reference's approximation is
    assert abs(oracle.exp_approx32(1.0) / np.e - 1) < 0.01


def test_learn_gelu_silu_compose(oracle):
    x = np.linspace(-6, 6, 241).astype(np.float32)
    g = oracle.epilogue(oracle.EPI_GELU_TANH_APPROX, x)
    s = oracle.epilogue(oracle.EPI_SILU_APPROX, x)
    for xi, gi, si in zip(x, g, s):
        inner = f32(f32(0.7978845608028654) * f32(xi + f32(f32(0.044715) * f32(f32(xi * xi) * xi))))
        assert gi == f32(f32(f32(0.5) * xi) * f32(f32(1.0) + f32(oracle.tanh_approx32(float(inner)))))
        sig = f32(f32(1.0) / f32(f32(1.0) + f32(oracle.exp_approx32(float(-xi)))))
        assert si == f32(xi * sig)


def test_relu_variants(oracle):
    x = np.array([-1.0, -0.0, 0.0, 2.0, np.nan], np.float32)
    layer = oracle.epilogue(oracle.EPI_RELU, x)         # v > 0 ? v : 0
    unary = oracle.epilogue(oracle.EPI_RELU_UNARY, x)   # v < 0 ? 0 : v
    np.testing.assert_array_equal(layer[:4], [0, 0, 0, 2])
    assert not np.signbit(layer[1]) and layer[4] == 0
    assert np.signbit(unary[1]) and np.isnan(unary[4])


# ------------------------------------------------------------------ int8 legacy
@pytest.mark.parametrize("x,s,q", [
    (0.49999997, 1.0, 1),      # fp32 add: 0.49999997 + 0.5 rounds to 1.0
    (-0.49999997, 1.0, -1),
    (0.4999999, 1.0, 0),
    (2.5, 1.0, 3), (-2.5, 1.0, -3), (1.5, 1.0, 2), (0.5, 1.0, 1),
    (1e6, 1.0, 127), (-1e6, 1.0, -128), (-128.4, 1.0, -128), (127.6, 1.0, 127),
    (3.0, 0.0, 3),             # scale 0 replaced by 1 (functional.mojo:235-236)
    (0.3, 0.1, 3),
])
def test_legacy_quantize_cases(oracle, x, s, q):
    got = oracle.quantize_symmetric_int8(np.array([x], np.float32), s)
    assert int(got[0]) == q


def test_legacy_quantize_closed_form(oracle):
    x = oracle.randn_f32((5000,), seed=1) * f32(40)
    s = f32(0.37)
    v = (x / s).astype(np.float32)
    t = (v + np.where(v >= 0, f32(0.5), f32(-0.5))).astype(np.float32)
    exp = np.clip(np.trunc(t), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(oracle.quantize_symmetric_int8(x, s), exp)


def test_int8_gemm_exact(oracle):
    rng = np.random.default_rng(2)
    A = rng.integers(-128, 128, size=(9, 300), dtype=np.int8)
    B = rng.integers(-128, 128, size=(11, 300), dtype=np.int8)
    np.testing.assert_array_equal(oracle.matmul_i8_i8_to_i32(A, B),
                                  A.astype(np.int64) @ B.T.astype(np.int64))


def test_int8_gemm_legacy_literal(oracle):
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, size=(3, 5), dtype=np.int8)
    B = rng.integers(-128, 128, size=(4, 5), dtype=np.int8)
    lit = oracle.matmul_i8_i8_to_i32(A, B, legacy_literal=True)
    np.testing.assert_array_equal(lit, A.astype(np.int64) @ B.reshape(5, 4).astype(np.int64))


def test_dequant_closed_form(oracle):
    acc = np.array([[0, 1, -1, 2 ** 23, -(2 ** 23) + 7]], np.int32)
    b = np.array([0.5, -0.25, 1.0, 0.0, 2.0], np.float32)
    y = oracle.dequant_i32_bias(acc, 0.125, b)
    np.testing.assert_array_equal(y[0], acc[0].astype(np.float64) * 0.125 + b)


def test_minmax_scale_rules(oracle):
    assert oracle.minmax_scale_symmetric(np.zeros(0, np.float32)) == 1.0
    assert oracle.minmax_scale_symmetric(np.zeros(10, np.float32)) == 1.0
    assert oracle.minmax_scale_symmetric(np.ones(3, np.float32), 0.0) == 1.0
    x = np.array([-3.5, 1.0, 2.0], np.float32)
    assert oracle.minmax_scale_symmetric(x) == f32(3.5) / f32(127)
    assert oracle.minmax_scale_symmetric(-x) == f32(3.5) / f32(127)


def test_minmax_nan_rule(oracle):
    """observe() starts min/max at x[0] and replaces them only on v < mn /
    v > mx (sequential.mojo:232-240): under IEEE comparisons a NaN first
    element stays (both bounds NaN, so scale_symmetric returns NaN / max_q,
    its m <= 0 guard being false for NaN), and any later NaN is skipped."""
    nan = np.float32(np.nan)
    assert np.isnan(oracle.minmax_scale_symmetric(np.array([nan, 1.0, -2.0], np.float32)))
    assert oracle.minmax_scale_symmetric(np.array([1.0, nan, -2.0], np.float32)) == f32(2) / f32(127)
    assert oracle.minmax_scale_symmetric(np.array([0.5, -0.25, nan], np.float32)) == f32(0.5) / f32(127)


def test_rhe_quantize_nan(oracle):
    """Per-channel RHE: a NaN weight quantizes to 0 and does not enter the
    row's absmax (a > m is false for NaN); an all-NaN row keeps scale 1."""
    nan = np.float32(np.nan)
    W = np.array([[nan, 0.5, -1.0, 0.25], [nan, nan, nan, nan]], np.float32)
    Q, s = oracle.quantize_rowwise_rhe(W)
    assert s[0] == f32(1.0) / f32(127) and s[1] == 1.0
    np.testing.assert_array_equal(Q, np.array([[0, 64, -127, 32], [0, 0, 0, 0]], np.int8))
    Ql, sl = oracle.quantize_rowwise_legacy(W)
    assert np.isnan(sl[0]) and np.isnan(sl[1])   # NaN first element: the observer's NaN scale
    assert not Ql.any()                           # and every q from a NaN quotient is 0


def test_quant_linear_composition(oracle):
    x = oracle.randn_f32((6, 32), seed=4)
    W = oracle.randn_f32((8, 32), std=0.1, seed=5)
    b = oracle.randu_f32((8,), -0.1, 0.1, seed=6)
    s_x, s_w = oracle.minmax_scale_symmetric(x), oracle.minmax_scale_symmetric(W)
    Wq = oracle.quantize_symmetric_int8(W, s_w)
    xq = oracle.quantize_symmetric_int8(x, s_x)
    acc = xq.astype(np.int64) @ Wq.T.astype(np.int64)
    sf = f32(f32(s_x) * f32(s_w))
    exp = (acc.astype(np.float32) * sf).astype(np.float32) + b
    np.testing.assert_array_equal(oracle.quant_linear_fw(x, Wq, b, s_w, s_x), exp.astype(np.float32))


# ------------------------------------------------------------------ per-channel spec
def test_rhe_quantize_ties_and_edges(oracle):
    s = f32(2.0 ** -6)
    ks = np.arange(-126, 126, dtype=np.float32)
    row = np.concatenate([(ks + 0.5) * s, [127 * s, -127 * s, 0, 0]]).astype(np.float32)
    W = np.stack([row, np.zeros_like(row), -np.abs(row)])
    Q, sc = oracle.quantize_rowwise_rhe(W)
    assert sc[0] == s and sc[1] == 1.0 and sc[2] == s
    np.testing.assert_array_equal(Q[0, :252], np.rint(ks + 0.5).astype(np.int8))  # half to even
    assert Q[0, 252] == 127 and Q[0, 253] == -127
    assert not Q[1].any()
    Ql, sl = oracle.quantize_rowwise_legacy(W)
    np.testing.assert_array_equal(Ql[0, :252], np.trunc(ks + 0.5 + np.where(ks + 0.5 >= 0, 0.5, -0.5))
                                  .astype(np.int8))
    assert sl[1] == 1.0


def test_rhe_quantize_closed_form(oracle):
    W = oracle.randn_f32((37, 513), std=0.02, seed=7)
    Q, s = oracle.quantize_rowwise_rhe(W)
    exp_s = (np.abs(W).max(axis=1) / f32(127)).astype(np.float32)
    np.testing.assert_array_equal(s, exp_s)
    exp_q = np.clip(np.rint((W / exp_s[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    np.testing.assert_array_equal(Q, exp_q)
    assert (np.abs(Q).max(axis=1) == 127).all()


def test_w8a16_integer_inputs_exact(oracle):
    """bf16-exact small-integer activations: every partial sum is an exact
    integer in fp32, so the reference is (sum)*scale + b in two roundings."""
    rng = np.random.default_rng(8)
    xi = rng.integers(-3, 4, size=(3, 256)).astype(np.float32)
    x = oracle.f32_to_bf16(xi)
    Q = rng.integers(-127, 128, size=(20, 256), dtype=np.int8)
    s = oracle.randu_f32((20,), 0.001, 0.01, seed=9)
    b = oracle.randu_f32((20,), -0.1, 0.1, seed=10)
    yb, yf = oracle.linear_w8a16(x, Q, s, b)
    acc = (xi.astype(np.int64) @ Q.T.astype(np.int64)).astype(np.float32)
    exp = ((acc * s).astype(np.float32) + b).astype(np.float32)
    np.testing.assert_array_equal(yf, exp)
    np.testing.assert_array_equal(yb, oracle.f32_to_bf16(exp))


def test_w8a8_activation_quantize_is_rowwise_rhe(oracle):
    """The W8A8 Linear quantizes each row of x with the per-channel RHE rule
    applied to the exact fp32 upcast: xq, sx equal quantize_rowwise_rhe's,
    and on a row whose absmax is 31.75 (scale 0.25 exactly) the quotients
    (2j+1)/2 are ties that round half to even."""
    rng = np.random.default_rng(21)
    x = oracle.f32_to_bf16(oracle.randn_f32((5, 96), seed=22))
    j = np.arange(-48, 48, dtype=np.float32)
    ties = ((2 * j + 1) / 8).astype(np.float32)   # x / 0.25 = j + 0.5
    ties[0] = -31.75                             # the absmax: scale 127 * 0.25 / 127
    x[1] = oracle.f32_to_bf16(ties)
    x[2] = 0                                     # zero row: scale 1, q 0
    Q = rng.integers(-127, 128, size=(3, 96), dtype=np.int8)
    _, _, xq, sx = oracle.linear_w8a8(x, Q, np.ones(3, np.float32))
    q_ref, s_ref = oracle.quantize_rowwise_rhe(oracle.bf16_to_f32(x))
    np.testing.assert_array_equal(xq, q_ref)
    np.testing.assert_array_equal(sx, s_ref)
    assert sx[1] == np.float32(0.25) and sx[2] == 1.0 and not xq[2].any()
    np.testing.assert_array_equal(xq[1, 1:], np.rint(j[1:] + 0.5).astype(np.int8))
    assert xq[1, 0] == -127


def test_w8a8_exact_epilogue(oracle):
    """Rows whose absmax is 127 with integer entries quantize to themselves
    with sx = 1 exactly; power-of-two weight scales and dyadic biases then
    make acc * sw exact, so every fp32 output is the correctly rounded value
    of the exact acc * sw + b (computed in float64, where it is exact)."""
    rng = np.random.default_rng(23)
    M, N, K = 4, 24, 256
    xi = rng.integers(-127, 128, size=(M, K)).astype(np.float32)
    xi[:, 0] = 127
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = (2.0 ** rng.integers(-12, -6, size=N)).astype(np.float32)
    b = (rng.integers(-64, 65, size=N) / 16).astype(np.float32)
    for epi in (oracle.EPI_NONE, oracle.EPI_RELU):
        yb, yf, xq, sx = oracle.linear_w8a8(oracle.f32_to_bf16(xi), Q, sw, b, epi)
        assert (sx == 1.0).all()
        np.testing.assert_array_equal(xq, xi.astype(np.int8))
        acc = xi.astype(np.int64) @ Q.T.astype(np.int64)
        exact = (acc.astype(np.float64) * sw.astype(np.float64) + b).astype(np.float32)
        if epi == oracle.EPI_RELU:
            exact = np.maximum(exact, 0)
        np.testing.assert_array_equal(yf, exact)
        np.testing.assert_array_equal(yb, oracle.f32_to_bf16(exact))


def test_w8a8_against_torch_cpu(oracle):
    """An independent restatement with torch CPU ops: fp32 division and
    torch.round (half to even) for the row quantize, an int64 matmul for the
    sums, then (acc * (sx * sw)) + b in fp32 and RNE to bf16.  Random
    inputs, so a different scale association or rounding rule shows up."""
    torch = pytest.importorskip("torch")
    M, N, K = 9, 40, 200
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=24))
    x[3, 7] = oracle.f32_to_bf16(np.array([40.0], np.float32))[0]   # one outlier row
    rng = np.random.default_rng(25)
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = oracle.randu_f32((N,), 0.0005, 0.004, seed=26)
    b = oracle.randu_f32((N,), -0.25, 0.25, seed=27)
    xt = torch.from_numpy(oracle.bf16_to_f32(x))
    s = xt.abs().amax(dim=1) / 127.0
    s = torch.where(s == 0, torch.ones_like(s), s)
    q = torch.clamp(torch.round(xt / s[:, None]), -127, 127).to(torch.int64)
    acc = q @ torch.from_numpy(Q.astype(np.int64)).T
    sf = s[:, None] * torch.from_numpy(sw)[None, :]
    for epi in (oracle.EPI_NONE, oracle.EPI_RELU):
        v = acc.to(torch.float32) * sf + torch.from_numpy(b)[None, :]
        if epi == oracle.EPI_RELU:
            v = torch.relu(v)
        want = v.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        yb, yf, _, _ = oracle.linear_w8a8(x, Q, sw, b, epi)
        np.testing.assert_array_equal(yf, v.numpy())
        np.testing.assert_array_equal(yb, want)
        yb2, _, _, _ = oracle.linear_w8a8(x, Q, sw, b, epi, rows=(2, 6))
        np.testing.assert_array_equal(yb2, want[2:6])


def test_dequant_scaled_closed_form(oracle):
    """Power-of-two scales make float(acc) * (sx * sw) exact for |acc| < 2^24,
    so y is the correctly rounded value of the exact acc * sx * sw + b; with
    sx omitted it is the scalar rule's form per column, and with a uniform
    sw and no sx it equals dequant_i32_bias."""
    rng = np.random.default_rng(31)
    M, N = 7, 33
    acc = rng.integers(-(2 ** 23), 2 ** 23, size=(M, N)).astype(np.int32)
    sw = (2.0 ** rng.integers(-20, -5, size=N)).astype(np.float32)
    sx = (2.0 ** rng.integers(-6, 3, size=M)).astype(np.float32)
    b = oracle.randu_f32((N,), -1, 1, seed=32)
    exact = (acc.astype(np.float64) * sx[:, None].astype(np.float64) * sw.astype(np.float64)
             + b.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(oracle.dequant_i32_scaled(acc, sw, b, sx), exact)
    exact_nb = (acc.astype(np.float64) * sw.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(oracle.dequant_i32_scaled(acc, sw), exact_nb)
    acc2 = rng.integers(-(2 ** 30), 2 ** 30, size=(M, N)).astype(np.int32)
    sf = np.float32(0.0123)
    np.testing.assert_array_equal(oracle.dequant_i32_scaled(acc2, np.full(N, sf, np.float32), b),
                                  oracle.dequant_i32_bias(acc2, sf, b))


def test_mlp_fp64_composition(oracle):
    rng = np.random.default_rng(11)
    M, K, I, H = 3, 64, 48, 40
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=12))
    mk = lambda shape, seed: oracle.quantize_rowwise_rhe(oracle.randn_f32(shape, std=0.05, seed=seed))
    (Wg, sg), (Wu, su), (Wd, sd) = mk((I, K), 13), mk((I, K), 14), mk((H, I), 15)
    h, y = oracle.mlp_w8a16(x, Wg, sg, Wu, su, Wd, sd)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    g = (xf @ Wg.T.astype(np.float64)) * sg
    u = (xf @ Wu.T.astype(np.float64)) * su
    hd = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(oracle.bf16_to_f32(h), hd, rtol=1e-2, atol=1e-2 * np.abs(hd).max())
    yd = (oracle.bf16_to_f32(h).astype(np.float64) @ Wd.T.astype(np.float64)) * sd
    np.testing.assert_allclose(oracle.bf16_to_f32(y), yd, rtol=1e-2, atol=1e-2 * np.abs(yd).max())
    del rng


def test_golden_int8_cases(oracle):
    g = np.load(GOLD)
    Q, s = oracle.quantize_rowwise_rhe(g["q_W"])
    np.testing.assert_array_equal(Q, g["q_rhe"])
    np.testing.assert_array_equal(s, g["q_rhe_s"])
    Ql, sl = oracle.quantize_rowwise_legacy(g["q_W"])
    np.testing.assert_array_equal(Ql, g["q_legacy"])
    np.testing.assert_array_equal(sl, g["q_legacy_s"])
    yb, yf = oracle.linear_w8a16(g["gemv_x"], g["gemv_Q"], g["gemv_s"], g["gemv_b"])
    np.testing.assert_array_equal(yb, g["gemv_y_bf16"])
    np.testing.assert_array_equal(yf, g["gemv_y_f32"])
