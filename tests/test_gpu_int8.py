"""GPU parity of the int8 path against the oracle.

* quantize/pack (per-channel RHE and legacy rules, per-tensor legacy):
  bit-exact int8 and scales;
* int8 x int8 -> int32 GEMM (legacy W8A8): bit-exact int32, and QuantLinear
  (fused dequantize, no FMA contraction): bit-exact fp32;
* W8A16 GEMV (C3), prefill GEMM + GELU (C4), MLP (C5): bf16 outputs within
  max|gpu - oracle| / max|oracle| <= 2e-2, on row slabs at full size.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from _util import (assert_tiles_covered, bf16_dev, bf16_host_bits, bf16_host_f32,
                   normwise_rel, slab_cols, slab_rows, to_dev)

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _quant_dev(W, dev, rounding=mj.ROUND_RHE):
    q, s = mj.quantize_rowwise_int8(to_dev(W, dev), rounding)
    torch.cuda.synchronize()
    return q, s


# ------------------------------------------------------------- quantize/pack
def test_c3_pack_rhe_bit_exact(oracle, dev):
    W = oracle.randn_f32((11008, 4096), std=0.02, seed=4)
    q, s = _quant_dev(W, dev)
    Qr, sr = oracle.quantize_rowwise_rhe(W)
    np.testing.assert_array_equal(s.cpu().numpy(), sr)
    np.testing.assert_array_equal(q.cpu().numpy(), Qr)


@pytest.mark.parametrize("N,K", [(5, 256), (3, 4096), (7, 100), (2, 8192), (9, 4352)])
@pytest.mark.parametrize("rounding", [mj.ROUND_RHE, mj.ROUND_LEGACY])
def test_pack_shapes_and_rules(oracle, dev, N, K, rounding):
    W = oracle.randn_f32((N, K), std=0.5, seed=N * K)
    W[0, :] = 0.0                       # all-zero row: scale 1, q 0
    if N > 2:
        W[1, :] = -np.abs(W[1, :])      # absmax from a negative value
        W[1, K // 2] = -3.0
        W[2, :] = np.abs(W[2, :])       # absmax appearing twice
        W[2, 0] = W[2, K - 1] = 2.0
    q, s = _quant_dev(W, dev, rounding)
    ref = oracle.quantize_rowwise_rhe(W) if rounding == mj.ROUND_RHE else \
        oracle.quantize_rowwise_legacy(W)
    np.testing.assert_array_equal(s.cpu().numpy(), ref[1])
    np.testing.assert_array_equal(q.cpu().numpy(), ref[0])


def test_pack_exact_ties(oracle, dev):
    """Values (k + 1/2) * scale with a power-of-two scale, so w/scale is exact:
    RHE rounds ties to even, the legacy rule away from zero."""
    K = 256
    s = np.float32(2.0 ** -6)
    ks = np.arange(-127, 127, dtype=np.float32)[:K - 2]
    row = np.concatenate([(ks + 0.5) * s, [127 * s, -127 * s]]).astype(np.float32)
    W = row[None, :]
    for rounding in (mj.ROUND_RHE, mj.ROUND_LEGACY):
        q, sc = _quant_dev(W, dev, rounding)
        ref = oracle.quantize_rowwise_rhe(W) if rounding == mj.ROUND_RHE else \
            oracle.quantize_rowwise_legacy(W)
        np.testing.assert_array_equal(q.cpu().numpy(), ref[0])
        np.testing.assert_array_equal(sc.cpu().numpy(), ref[1])


def test_quantize_symmetric_int8_per_tensor(oracle, dev):
    x = oracle.randn_f32((257, 129), seed=3) * np.float32(3)
    x[0, :6] = [0.49999997, -0.49999997, 2.5, -2.5, 1e6, -1e6]
    for s in (0.0, 1.0, 0.05, 1.0 / 127):
        got = mj.quantize_symmetric_int8(mj.Tensor(to_dev(x, dev)), s).numpy()
        np.testing.assert_array_equal(got, oracle.quantize_symmetric_int8(x, s))


@pytest.mark.parametrize("s", [1.0, 0.05, 1.0 / 127, 0.0123])
def test_quantize_symmetric_int8_ties_and_tails(oracle, dev, s):
    """The per-tensor quantizer converts four elements per thread from
    r = 1 / s and takes the division only within 2^-14 of a half-integer
    quotient: x = (k + 0.5) s and x within 1e-4 s of it must still match the
    oracle's division bit for bit, on an element count with a tail (not a
    multiple of 4) and on a view whose start is not 16-byte aligned (the
    one-element path)."""
    rng = np.random.default_rng(int(s * 1e4))
    n = 1_000_003
    k = rng.integers(-300, 300, n).astype(np.float64) + 0.5
    x = np.where(rng.random(n) < 0.5, k * s, (k + rng.uniform(-1e-4, 1e-4, n)) * s).astype(np.float32)
    x[:1000] = (rng.standard_normal(1000) * 3).astype(np.float32)
    x[1000:1006] = [0.49999997, -0.49999997, 2.5, -2.5, 1e6, -1e6]
    xs = np.float32(s)
    got = mj.quantize_symmetric_int8(mj.Tensor(to_dev(x, dev)), float(xs)).numpy()
    np.testing.assert_array_equal(got, oracle.quantize_symmetric_int8(x, xs))
    xd = to_dev(x, dev)[1:]  # 4-byte offset: not 16-byte aligned
    got_u = mj.quantize_symmetric_int8(mj.Tensor(xd), float(xs)).numpy()
    np.testing.assert_array_equal(got_u, oracle.quantize_symmetric_int8(x[1:], xs))


def test_minmax_scale(oracle, dev):
    x = oracle.randn_f32((1000, 37), seed=9)
    x[5, 5] = -7.25
    got = mj.functional.scale_symmetric_device(mj.Tensor(to_dev(x, dev)))
    assert np.float32(got) == np.float32(oracle.minmax_scale_symmetric(x))
    obs = mj.MinMaxObserver()
    obs.observe(mj.Tensor(to_dev(x, dev)))
    obs.observe(mj.Tensor(to_dev(x * 0.5, dev)))
    assert np.float32(obs.scale_symmetric()) == np.float32(oracle.minmax_scale_symmetric(x))
    zero = mj.functional.scale_symmetric_device(mj.Tensor(to_dev(np.zeros(10, np.float32), dev)))
    assert zero == 1.0


def test_minmax_and_quantize_nan(oracle, dev):
    """NaN semantics against the oracle: the observer's first-element rule
    (sequential.mojo:232-240) for mj_minmax_* and the legacy per-row scale,
    NaN -> 0 for both quantizers."""
    nan = np.float32(np.nan)
    x = oracle.randn_f32((3000,), seed=11)
    x[[7, 1500, 2999]] = nan
    got = mj.functional.scale_symmetric_device(mj.Tensor(to_dev(x, dev)))
    assert np.float32(got) == np.float32(oracle.minmax_scale_symmetric(x))
    x[0] = nan
    assert np.isnan(mj.functional.scale_symmetric_device(mj.Tensor(to_dev(x, dev))))
    obs = mj.MinMaxObserver()
    obs.observe(mj.Tensor(to_dev(x, dev)))
    assert np.isnan(obs.min_v) and np.isnan(obs.max_v) and np.isnan(obs.scale_symmetric())
    W = oracle.randn_f32((6, 4096), std=0.02, seed=12)   # register path (K % 256 == 0)
    W[0, 0] = W[1, 100] = W[2, :] = nan
    W2 = oracle.randn_f32((3, 100), std=0.02, seed=13)   # generic path
    W2[0, 0] = W2[1, 7] = nan
    for w in (W, W2):
        for rounding in (mj.ROUND_RHE, mj.ROUND_LEGACY):
            q, sc = _quant_dev(w, dev, rounding)
            ref = oracle.quantize_rowwise_rhe(w) if rounding == mj.ROUND_RHE else \
                oracle.quantize_rowwise_legacy(w)
            np.testing.assert_array_equal(q.cpu().numpy(), ref[0])
            np.testing.assert_array_equal(sc.cpu().numpy(), ref[1])   # NaN == NaN here


# ------------------------------------------------------------- int8 GEMM (legacy)
@pytest.mark.parametrize("M,N,K", [(1, 11008, 4096), (64, 64, 64), (37, 53, 80), (5, 7, 10), (200, 300, 1024),
                                   (130, 129, 16)])
def test_int8_gemm_bit_exact(oracle, dev, M, N, K):
    rng = np.random.default_rng(M * N + K)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    a = mj.Tensor(to_dev(A, dev))
    w = mj.Tensor(to_dev(B, dev))
    got = mj.matmul_i8_i8_to_i32(a, w.transpose()).numpy()
    np.testing.assert_array_equal(got, oracle.matmul_i8_i8_to_i32(A, B))


def _exact_i8_products(A, B):
    """A [M,K] . B [N,K]^T of int8 matrices, exactly: every product and
    partial sum is an integer below 2^53 in magnitude (|acc| <= 2^14 K), so
    float64 arithmetic is exact in any order."""
    return (A.astype(np.float64) @ B.astype(np.float64).T).astype(np.int64)


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 4096),    # 128 tiles of 256 x 128
                                   (2000, 2100, 4112),    # partial tiles, K % 128 != 0
                                   (512, 4096, 11008),    # long K
                                   (3072, 4096, 1040)])   # 192 tiles of 256 x 256, K tail
def test_int8_gemm_large_tiles_bit_exact(dev, M, N, K):
    """Shapes that take the one-wave-per-SIMD int8 kernel (256 x 256 tiles
    from 192 of them, else 256 x 128): the int32 sums must be exact."""
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K), dtype=np.int8)
    got = mj.matmul_i8_i8_to_i32(mj.Tensor(to_dev(A, dev)),
                                 mj.Tensor(to_dev(B, dev)).transpose()).numpy()
    np.testing.assert_array_equal(got.astype(np.int64), _exact_i8_products(A, B))


def test_quant_linear_large_bit_exact(oracle, dev):
    """QuantLinear.forward at 2048 x 2048 x 4096 (the 256 x 256 int8 kernel with
    the dequantize fused): the oracle's quantize and dequantize around exact
    int32 sums."""
    M, N, K = 2048, 2048, 4096
    x = oracle.randn_f32((M, K), seed=41)
    W = oracle.randn_f32((N, K), std=0.02, seed=42)
    b = oracle.randu_f32((N,), -0.0625, 0.0625, seed=43)
    s_x = oracle.minmax_scale_symmetric(x)
    s_w = oracle.minmax_scale_symmetric(W)
    Wq = oracle.quantize_symmetric_int8(W, s_w)
    xq = oracle.quantize_symmetric_int8(x, s_x)
    ql = mj.QuantLinear(K, N, mj.Tensor(to_dev(Wq, dev)), mj.Tensor(to_dev(b, dev)), s_w, s_x)
    got = ql.forward(mj.Tensor(to_dev(x, dev))).numpy()
    acc = _exact_i8_products(xq, Wq).astype(np.int32)
    ref = oracle.dequant_i32_bias(acc, np.float32(s_x) * np.float32(s_w), b)
    np.testing.assert_array_equal(got, ref)


def test_int8_gemm_legacy_literal(oracle, dev):
    """The reference's stride-ignoring read of w_q.transpose() (bug i):
    result is A @ reshape(w_q.flat, [K, N])."""
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, size=(3, 5), dtype=np.int8)
    B = rng.integers(-128, 128, size=(4, 5), dtype=np.int8)  # w_q [N=4, K=5]
    got = mj.matmul_i8_i8_to_i32(mj.Tensor(to_dev(A, dev)), mj.Tensor(to_dev(B, dev)).transpose(),
                                 legacy_literal=True).numpy()
    ref = oracle.matmul_i8_i8_to_i32(A, B, legacy_literal=True)
    np.testing.assert_array_equal(got, ref)
    lit = A.astype(np.int32) @ B.reshape(5, 4).astype(np.int32)
    np.testing.assert_array_equal(got, lit)
    assert not np.array_equal(got, A.astype(np.int32) @ B.T.astype(np.int32))


def test_dequantize(oracle, dev):
    rng = np.random.default_rng(6)
    acc = rng.integers(-2 ** 26, 2 ** 26, size=(33, 65), dtype=np.int32)
    b = oracle.randu_f32((65,), -1, 1, seed=2)
    got = mj.dequantize_i32_to_f32_add_bias(mj.Tensor(to_dev(acc, dev)), 3.0517578e-05,
                                            mj.Tensor(to_dev(b, dev))).numpy()
    np.testing.assert_array_equal(got, oracle.dequant_i32_bias(acc, np.float32(3.0517578e-05), b))


@pytest.mark.parametrize("M,N,K,literal", [(256, 256, 256, False), (1, 11008, 4096, False),
                                           (17, 40, 24, True), (64, 96, 100, False)])
def test_quant_linear_bit_exact(oracle, dev, M, N, K, literal):
    x = oracle.randn_f32((M, K), seed=M + 1)
    W = oracle.randn_f32((N, K), std=0.02, seed=N + 2)
    b = oracle.randu_f32((N,), -0.0625, 0.0625, seed=3)
    s_x = oracle.minmax_scale_symmetric(x)
    s_w = oracle.minmax_scale_symmetric(W)
    Wq = oracle.quantize_symmetric_int8(W, s_w)
    ql = mj.QuantLinear(K, N, mj.Tensor(to_dev(Wq, dev)), mj.Tensor(to_dev(b, dev)), s_w, s_x,
                        legacy_literal=literal)
    got = ql.forward(mj.Tensor(to_dev(x, dev))).numpy()
    np.testing.assert_array_equal(got, oracle.quant_linear_fw(x, Wq, b, s_w, s_x, literal))


def test_ptq_flow(oracle, dev):
    """prepare -> calibrate -> convert -> Converted.forward on the
    Linear(10,32) -> ReLU -> Linear(32,2) model of sequential_min.mojo."""
    l1, l2 = mj.Linear(10, 32), mj.Linear(32, 2)
    W1 = oracle.randn_f32((32, 10), std=0.3, seed=1)
    W2 = oracle.randn_f32((2, 32), std=0.3, seed=2)
    b1 = oracle.randu_f32((32,), -0.1, 0.1, seed=3)
    b2 = oracle.randu_f32((2,), -0.1, 0.1, seed=4)
    l1.weight.torch.copy_(torch.from_numpy(W1)); l1.bias_t.torch.copy_(torch.from_numpy(b1))
    l2.weight.torch.copy_(torch.from_numpy(W2)); l2.bias_t.torch.copy_(torch.from_numpy(b2))
    x = oracle.randn_f32((4, 10), seed=5)
    p = mj.prepare(l1, mj.ReLU(), l2)
    p.forward(mj.Tensor(to_dev(x, dev)))
    conv = mj.convert(p)
    got = conv.forward(mj.Tensor(to_dev(x, dev))).numpy()
    # oracle: same flow on the CPU.  The ReLU-output scale comes from an fp32
    # Linear, equal to the oracle's to rounding; the rest of the chain is
    # then exact given that scale.
    y1 = oracle.linear_fw_f32(x, W1, b1)
    y2 = np.where(y1 > 0, y1, 0).astype(np.float32)
    s_in = oracle.minmax_scale_symmetric(x)
    s_w1, s_w2 = oracle.minmax_scale_symmetric(W1), oracle.minmax_scale_symmetric(W2)
    assert np.float32(conv.q1.s_x) == np.float32(s_in)
    assert np.float32(conv.q1.s_w) == np.float32(s_w1)
    assert np.float32(conv.q2.s_w) == np.float32(s_w2)
    assert abs(conv.q2.s_x - oracle.minmax_scale_symmetric(y2)) <= 1e-6 * conv.q2.s_x
    s_relu = conv.q2.s_x
    q1 = oracle.quant_linear_fw(x, oracle.quantize_symmetric_int8(W1, s_w1), b1, s_w1, s_in)
    q1 = np.where(q1 > 0, q1, 0).astype(np.float32)
    ref = oracle.quant_linear_fw(q1, oracle.quantize_symmetric_int8(W2, s_w2), b2, s_w2, s_relu)
    np.testing.assert_array_equal(got, ref)


# ------------------------------------------------------------- W8A16
def _w8_case(oracle, dev, M, N, K, seed):
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=seed))
    W = oracle.randn_f32((N, K), std=0.02, seed=seed + 1)
    Q, s = oracle.quantize_rowwise_rhe(W)
    b = oracle.randu_f32((N,), -1.0 / 16, 1.0 / 16, seed=seed + 2)
    return x, Q, s, b


def test_c3_gemv(oracle, dev):
    M, N, K = 1, 11008, 4096
    x, Q, s, b = _w8_case(oracle, dev, M, N, K, 3)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev))
    y = lin.forward(bf16_dev(x, dev))
    _, ref = oracle.linear_w8a16(x, Q, s, b)
    err = normwise_rel(bf16_host_f32(y), ref)
    print(f"C3 gemv normwise rel err {err:.3e}", flush=True)
    assert err <= BF16_TOL


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 11, 16, 17, 32, 33, 48])
@pytest.mark.parametrize("N,K", [(64, 256), (37, 1040), (300, 4096), (5, 16), (17, 48),
                                 (130, 11008), (48, 6160)])
def test_gemv_shapes(oracle, dev, M, N, K):
    x, Q, s, b = _w8_case(oracle, dev, M, N, K, M * 100 + N)
    for bias, epi in ((b, mj.EPI_NONE), (None, mj.EPI_GELU_TANH), (b, mj.EPI_SILU)):
        lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev),
                          None if bias is None else to_dev(bias, dev), epi)
        y = lin.forward(bf16_dev(x, dev))
        _, ref = oracle.linear_w8a16(x, Q, s, bias, epi)
        assert normwise_rel(bf16_host_f32(y), ref) <= BF16_TOL


def test_c4_prefill_gelu(oracle, dev):
    """C4 at full size, every output tile checked at full K: one row in every
    128-row block over all 4096 columns, two columns in every 256-wide block
    over all 2048 rows."""
    M, N, K = 2048, 4096, 4096
    x, Q, s, b = _w8_case(oracle, dev, M, N, K, 40)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), mj.EPI_GELU_TANH)
    y = bf16_host_f32(lin.forward(bf16_dev(x, dev)))
    rows, cols = slab_rows(M), slab_cols(N)
    worst = 0.0
    for r in rows:
        _, ref = oracle.linear_w8a16(x[r:r + 1], Q, s, b, mj.EPI_GELU_TANH)
        worst = max(worst, normwise_rel(y[r:r + 1], ref))
    _, ref_cols = oracle.linear_w8a16(x, np.ascontiguousarray(Q[cols]), s[cols], b[cols],
                                      mj.EPI_GELU_TANH)
    worst = max(worst, normwise_rel(y[:, cols], ref_cols))
    assert_tiles_covered(M, N, rows, cols)
    print(f"C4 prefill: {len(rows)} rows, {len(cols)} columns; worst normwise rel err "
          f"{worst:.3e}", flush=True)
    assert worst <= BF16_TOL


@pytest.mark.parametrize("M,N,K", [(17, 64, 256), (100, 300, 1040), (257, 520, 512),
                                   # 256 x 128 tiles (waves of 256 x 32) with K % 64 != 0: a
                                   # 2-way and a 4-way K split whose last slice ends inside a
                                   # stage, and partial tiles in M and N
                                   (512, 384, 1040), (384, 1000, 2064), (1000, 1300, 528)])
def test_w8a16_gemm_shapes(oracle, dev, M, N, K):
    x, Q, s, b = _w8_case(oracle, dev, M, N, K, M + N)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), mj.EPI_RELU)
    y = bf16_host_f32(lin.forward(bf16_dev(x, dev)))
    _, ref = oracle.linear_w8a16(x, Q, s, b, mj.EPI_RELU)
    assert normwise_rel(y, ref) <= BF16_TOL


@pytest.mark.parametrize("M,N,K", [(256, 256, 512),      # 256 x 128 tiles, one K slice
                                   (512, 384, 1040),     # 2-way K split, partial last stage
                                   (384, 1000, 2064),    # 4-way K split, partial N tile
                                   (1000, 1300, 528),    # partial M and N tiles, one K slice
                                   (256, 256, 16384),    # 8-way K split: one K slice per XCD
                                   # skinny-M MFMA GEMV (K % 1024 != 0): partial
                                   # 16-row tile of weights, K % 64 != 0, x rows < 16
                                   (3, 4104, 1040), (7, 37, 80),
                                   # skinny-M GEMV through LDS (K = 1024 j <= 4096):
                                   # every K share, partial 48-row workgroups, the
                                   # C3 weight at 3 and 16 x rows
                                   (16, 1000, 4096), (3, 11008, 4096), (16, 11008, 4096),
                                   (5, 4104, 1024), (8, 1000, 2048), (11, 37, 3072),
                                   # two x-row groups (17..32 rows)
                                   (17, 1000, 4096), (32, 11008, 4096), (24, 37, 1024),
                                   # 17..255 rows past the GEMV: 128- and 256-row tiles
                                   (33, 11008, 4096), (128, 1000, 4096), (129, 300, 2048),
                                   (255, 520, 1024),
                                   # M = 1: the persistent streaming GEMV (K a
                                   # multiple of 1024) at every rows-per-wave
                                   # (1..32) and K-chunk count (1..4), with
                                   # partial last workgroups and waves; other K
                                   # take the 2-rows-per-wave kernel
                                   (1, 37, 1024), (1, 1500, 2048), (1, 4104, 3072),
                                   (1, 7001, 3072),
                                   (1, 16001, 1024), (1, 24000, 2048), (1, 70001, 1024),
                                   # M = 1, K = 4096: the K-split GEMV at 4, 8,
                                   # 12, 24, 44 and 64 rows per workgroup with a
                                   # partial last workgroup, and past 252 * 64
                                   # rows the streaming GEMV
                                   (1, 37, 4096), (1, 2000, 4096), (1, 3000, 4096),
                                   (1, 5000, 4096), (1, 11008, 4096), (1, 16001, 4096),
                                   (1, 16200, 4096),
                                   (1, 37, 80), (1, 4104, 2064),
                                   # M = 1, 4096 < K <= 16384: the K-split GEMV
                                   # at 2, 3 and 4 chunks per lane (a partial
                                   # last chunk round at K = 4112 and 12304),
                                   # 4 to 48 rows per workgroup, grids of one
                                   # to several rounds over the 256 CUs
                                   (1, 5, 4112), (1, 37, 5008), (1, 3000, 8192),
                                   (1, 20000, 6000), (1, 4096, 11008), (1, 9000, 12288),
                                   (1, 100, 12304), (1, 13000, 16384),
                                   # 2-4 x rows, K <= 16384: the two- and
                                   # four-row K-split GEMVs (1-4 chunks per lane)
                                   (2, 4096, 11008), (2, 20000, 6000), (2, 11008, 4096),
                                   (3, 4096, 11008), (4, 37, 5008), (4, 1000, 16384),
                                   (4, 300, 1040),
                                   # 5-16 x rows, 4096 < K <= 16384: the skinny
                                   # MFMA GEMV with one tile per workgroup, 5-16
                                   # passes of 1 KB (the last one past K),
                                   # partial tiles
                                   (5, 300, 5008), (9, 37, 12304), (16, 4100, 8192),
                                   (16, 1000, 16384),
                                   # 33-48 x rows at K = 1024 j: the skinny
                                   # GEMV's four x-row groups over 1-KB passes
                                   # (64: the tile GEMM again)
                                   (33, 300, 1024), (40, 37, 2048), (48, 4100, 4096),
                                   (48, 11008, 4096), (64, 1000, 3072),
                                   # M <= 256 on the tile GEMM's three-stage
                                   # load ring: K slices of one, two and three
                                   # stages (shorter than the ring), a partial
                                   # last stage, 128- and 256-row tiles
                                   (64, 300, 64), (100, 520, 128), (128, 130, 176),
                                   (200, 260, 192), (256, 1000, 336), (255, 4100, 4096),
                                   # 128 x 192 tiles where they fill more CUs:
                                   # 27 tiles x 8 K slices; 209 unsplit tiles
                                   # (full ones store their odd third block
                                   # directly, a partial last column tile)
                                   (64, 5000, 4096), (128, 40000, 256)])
def test_w8a16_integer_inputs_bit_exact(oracle, dev, M, N, K):
    """Small-integer activations, int8 weights and power-of-two scales make
    every product and partial sum exact in fp32 (|sum| <= 4 * 127 * K < 2^24),
    in any order and under any K split, so the bf16 outputs (after scale,
    bias and rounding) must equal the oracle's bit for bit; this pins every
    tile, fragment and swizzle index of the one-wave-per-SIMD W8A16 kernels, of
    the skinny-M MFMA GEMV and of the M = 1 GEMVs."""
    rng = np.random.default_rng(M + N + K)
    x = oracle.f32_to_bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, size=N)).astype(np.float32)
    b = rng.integers(-8, 9, size=N).astype(np.float32) / np.float32(4)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), mj.EPI_NONE)
    y = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    ref, _ = oracle.linear_w8a16(x, Q, s, b, mj.EPI_NONE)
    np.testing.assert_array_equal(y, ref)


def test_w8a16_integer_inputs_bit_exact_c4_shape(oracle, dev):
    """C4's 2048 x 4096 x 4096 on exact integer sums: every checked row (two
    or more in each of the eight 256-row tiles, at fragment and tile edges)
    must equal the oracle bit for bit over all 4096 columns, i.e. every
    column tile of the 256 x 128 W8A16 tiles."""
    M, N, K = 2048, 4096, 4096
    rng = np.random.default_rng(2048)
    x = oracle.f32_to_bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, size=N)).astype(np.float32)
    b = rng.integers(-8, 9, size=N).astype(np.float32) / np.float32(4)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), mj.EPI_NONE)
    y = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    rows = [0, 1, 15, 16, 255, 256, 300, 511, 512, 700, 767, 768, 1023, 1024, 1300, 1535,
            1536, 1800, 1791, 1792, 2046, 2047]
    for r in rows:
        ref, _ = oracle.linear_w8a16(x[r:r + 1], Q, s, b, mj.EPI_NONE)
        np.testing.assert_array_equal(y[r:r + 1], ref, err_msg=f"row {r}")


@pytest.mark.parametrize("M", [1, 5, 12, 40, 256])
@pytest.mark.parametrize("epi", [mj.EPI_GELU_TANH, mj.EPI_SILU])
def test_w8a16_gelu_silu_epilogue_exact_sums(oracle, dev, M, epi):
    """The bf16-output epilogues evaluate GELU as x / (1 + 2^(-2t log2 e))
    and SiLU as x / (1 + 2^(-x log2 e)) with the hardware exp2 and
    reciprocal, where the oracle follows the reference's literal expf and
    division forms.  With integer inputs the sums are exact, so the only
    difference left is the activation itself: every bf16 output is within one
    bf16 step (2^-7 relative) of the oracle's fp32 value before rounding, or
    within 1e-6 absolute.  For GELU at x < -2 the literal form's 1 + tanh(t)
    cancels (its own error there exceeds a bf16 step of the tiny result) and
    the bits differ there; elsewhere, and for SiLU everywhere, at most 1 % of
    the outputs differ in any bit.  M = 1 is the streaming GEMV, 5 and 12 the
    MFMA GEMV (1 and 4 row tiles), 40 and 256 GEMM kernels."""
    N, K = 256, 512
    rng = np.random.default_rng(M * 10 + epi)
    x = oracle.f32_to_bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-13, -8, size=N)).astype(np.float32)
    b = rng.integers(-8, 9, size=N).astype(np.float32) / np.float32(4)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), epi)
    got_t = lin.forward(bf16_dev(x, dev))
    got_bits, got = bf16_host_bits(got_t), bf16_host_f32(got_t)
    ref_bits, ref = oracle.linear_w8a16(x, Q, s, b, epi)
    ref = ref.astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    bound = np.maximum(np.abs(ref) * 2.0 ** -7, 1e-6)
    worst = int(np.argmax(err - bound))
    assert np.all(err <= bound), (worst, got.flat[worst], ref.flat[worst])
    _, pre = oracle.linear_w8a16(x, Q, s, b, mj.EPI_NONE)  # exact pre-activation
    keep = pre >= -2.0 if epi == mj.EPI_GELU_TANH else np.ones(pre.shape, bool)
    frac = float(np.mean(got_bits[keep] != ref_bits[keep]))
    print(f"M={M} epi={epi}: {frac:.4%} of {int(keep.sum())} outputs differ in some bit", flush=True)
    assert frac <= 0.01
    # the case spans the activation's range
    assert float(pre.min()) < -4.0 and float(pre.max()) > 4.0 and np.mean(np.abs(pre) < 2) > 0.2


def _mlp_case(oracle, M, K, I, H, seed):
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=seed))
    Wg, sg = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=seed + 6))
    Wu, su = oracle.quantize_rowwise_rhe(oracle.randn_f32((I, K), std=0.02, seed=seed + 7))
    Wd, sd = oracle.quantize_rowwise_rhe(oracle.randn_f32((H, I), std=0.02, seed=seed + 8))
    return x, Wg, sg, Wu, su, Wd, sd


def _run_mlp(dev, x, Wg, sg, Wu, su, Wd, sd):
    mk = lambda q, s: mj.W8Linear(to_dev(q, dev), to_dev(s, dev))
    mlp = mj.W8MLP(mk(Wg, sg), mk(Wu, su), mk(Wd, sd))
    y, h = mlp.forward(bf16_dev(x, dev))
    return bf16_host_f32(y), bf16_host_f32(h)


def test_c5_mlp(oracle, dev):
    """C5 at full size, every tile of both GEMMs checked at full K:
    - h = silu(x Wg^T) * (x Wu^T) and y on one row per 128-row block (all
      11008 / 4096 columns) against the oracle's FFN;
    - h on two columns per 256-wide block over all 512 rows (the oracle's FFN
      restricted to those gate/up rows);
    - y on two columns per 256-wide block over all rows, from the device's h
      (checked above) through the oracle's W8A16 Linear: this pins every tile
      and K slice of the down projection by itself."""
    M, K, I, H = 512, 4096, 11008, 4096
    x, Wg, sg, Wu, su, Wd, sd = case = _mlp_case(oracle, M, K, I, H, 0)
    y, h = _run_mlp(dev, *case)
    rows = slab_rows(M)
    worst_h = worst_y = 0.0
    for r in rows:
        hr, yr = oracle.mlp_w8a16(*case, rows=(r, r + 1))
        worst_h = max(worst_h, normwise_rel(h[r:r + 1], oracle.bf16_to_f32(hr)))
        worst_y = max(worst_y, normwise_rel(y[r:r + 1], oracle.bf16_to_f32(yr)))
    hc = slab_cols(I)
    sub = (x, np.ascontiguousarray(Wg[hc]), sg[hc], np.ascontiguousarray(Wu[hc]), su[hc],
           np.ascontiguousarray(Wd[:, hc]), sd)
    hr_cols, _ = oracle.mlp_w8a16(*sub)
    worst_h = max(worst_h, normwise_rel(h[:, hc], oracle.bf16_to_f32(hr_cols)))
    yc = slab_cols(H)
    h_bits = oracle.f32_to_bf16(h)              # h is bf16: this is exact
    _, yr_cols = oracle.linear_w8a16(h_bits, np.ascontiguousarray(Wd[yc]), sd[yc])
    worst_y = max(worst_y, normwise_rel(y[:, yc], yr_cols))
    assert_tiles_covered(M, I, rows, hc)
    assert_tiles_covered(M, H, rows, yc)
    print(f"C5 mlp: {len(rows)} rows, {len(hc)} + {len(yc)} columns; worst normwise rel err "
          f"h {worst_h:.3e} y {worst_y:.3e}", flush=True)
    assert worst_h <= BF16_TOL and worst_y <= BF16_TOL


@pytest.mark.parametrize("M,K,I", [(512, 1024, 2000),   # 2 row tiles, partial last column tile
                                   (300, 528, 400),     # partial row tile, K % 64 != 0
                                   (1024, 256, 4096),   # 4 x 43 tiles, one K slice of 4 stages
                                   (257, 64, 112),      # one-row second tile, one stage
                                   # one x row: the gate/up K-split GEMV at 1-4
                                   # chunks per lane, 8 to 88 rows per workgroup
                                   (1, 4096, 11008), (1, 1040, 400), (1, 6000, 304),
                                   (1, 9008, 12000), (1, 16384, 3008),
                                   # 33-128 x rows: the gate/up GEMM's narrow tiles
                                   (33, 1024, 1008), (64, 4096, 11008), (128, 1040, 720),
                                   (200, 1024, 2000), (256, 4096, 11008),
                                   # K of one and two stages, shorter than the
                                   # three-stage load ring of M <= 256
                                   (64, 64, 272), (200, 128, 400),
                                   # 2-4 x rows: the two- and four-row K-split
                                   # GEMVs' gate/up
                                   (2, 4096, 11008), (2, 1040, 400), (3, 5008, 304),
                                   (4, 12288, 1008),
                                   # 3-32 x rows at K = 1024 j: the skinny MFMA
                                   # GEMV's gate/up tile pairs, one and two
                                   # x-row groups, a partial last column tile
                                   (3, 1024, 400), (16, 4096, 11008), (20, 2048, 1008),
                                   (32, 3072, 112)])
def test_mlp_gateup_integer_sums(oracle, dev, M, K, I):
    """The gate/up GEMM on exact sums: small-integer x, int8 weights and
    power-of-two scales make g = x Wg^T sg and u = x Wu^T su exact in fp32, so
    every h = silu(g) u must lie within one bf16 step (2^-8 relative, or 1e-6
    absolute) of the float64 value from those exact sums.  A wrong pairing of
    gate and up rows, a swapped exchange half or a shifted column of the
    split layout's epilogue (gate sums in waves 0-1, up sums in waves 2-3,
    paired through LDS) is off by far more."""
    rng = np.random.default_rng(M + K + I)
    x = oracle.f32_to_bf16(rng.integers(-4, 5, size=(M, K)).astype(np.float32))
    Wg = rng.integers(-127, 128, size=(I, K), dtype=np.int8)
    Wu = rng.integers(-127, 128, size=(I, K), dtype=np.int8)
    sg = (2.0 ** rng.integers(-14, -10, size=I)).astype(np.float32)
    su = (2.0 ** rng.integers(-14, -10, size=I)).astype(np.float32)
    Wd = rng.integers(-127, 128, size=(64, I), dtype=np.int8)
    sd = np.full(64, 2.0 ** -20, np.float32)
    _, h = _run_mlp(dev, x, Wg, sg, Wu, su, Wd, sd)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    g = (xf @ Wg.astype(np.float64).T) * sg.astype(np.float64)
    u = (xf @ Wu.astype(np.float64).T) * su.astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    err = np.abs(h.astype(np.float64) - ref)
    bound = np.maximum(np.abs(ref) * 2.0 ** -8, 1e-6)
    bad = np.argwhere(err > bound)
    assert bad.size == 0, f"{len(bad)} outputs off, first at {bad[0]}: {h[tuple(bad[0])]} vs {ref[tuple(bad[0])]}"


@pytest.mark.parametrize("M,K,I,H", [(4, 256, 384, 128), (12, 256, 400, 130), (40, 512, 256, 320), (300, 256, 528, 64),
                                     # gate/up on 192-row tiles (a partial one), K % 64 != 0
                                     (384, 1040, 400, 272),
                                     # one x row: the gate/up GEMV, then the down
                                     # GEMV at K = I (the K-split one past 4096)
                                     (1, 256, 384, 128), (1, 4096, 11008, 4096),
                                     (1, 5008, 304, 272), (1, 1040, 12304, 100),
                                     # 2-4 x rows: the K-split GEMVs for both
                                     # projections; 5-32 at K = 1024 j: the
                                     # gate/up on the skinny MFMA GEMV
                                     (2, 1024, 400, 130), (2, 4096, 11008, 4096),
                                     (4, 4096, 11008, 4096), (3, 1040, 304, 64),
                                     (5, 2048, 1008, 272), (16, 4096, 11008, 4096),
                                     (17, 3072, 304, 64), (32, 1024, 48, 16),
                                     # gate/up GEMV, down on the GEMM
                                     (24, 2048, 1008, 272),
                                     # 33-128 x rows: the gate/up GEMM's narrow
                                     # tiles (a partial last one), down GEMM
                                     (33, 1024, 1008, 272), (64, 4096, 11008, 512),
                                     (100, 2048, 400, 64), (128, 1040, 720, 130),
                                     # 129-256 x rows on 64-column gate/up tiles
                                     (200, 1024, 2000, 272), (256, 4096, 11008, 256)])
def test_mlp_shapes(oracle, dev, M, K, I, H):
    case = _mlp_case(oracle, M, K, I, H, M)
    y, h = _run_mlp(dev, *case)
    hr, yr = oracle.mlp_w8a16(*case)
    assert normwise_rel(h, oracle.bf16_to_f32(hr)) <= BF16_TOL
    assert normwise_rel(y, oracle.bf16_to_f32(yr)) <= BF16_TOL
