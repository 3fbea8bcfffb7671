"""W8A8 Linear with dynamic per-row activation scales (mj_linear_w8a8) and its
activation quantizer (mj_quantize_rows_bf16_i8) against the oracle.

The quantizer is bit-exact to quantize_rowwise_rhe on the fp32 upcast of x.
The Linear's int32 sums are exact and its epilogue is rounded step by step, so
EPI_NONE / RELU outputs are bit-exact to the oracle at every shape; GELU and
SiLU use the bf16-output activation forms of the other bf16 kernels and are
held to one bf16 step.  Shapes cover both tile widths of the int8 kernel
(256 x 128 below 192 tiles of 256 x 256, 256 x 256 from there), ragged M, N
and K tails, bias present and absent.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from _util import assert_tiles_covered, bf16_dev, bf16_host_bits, bf16_host_f32, slab_rows, to_dev

pytestmark = pytest.mark.gpu


def _x_with_edges(oracle, M, K, seed):
    """bf16 [M, K] normal data plus, where M allows, a zero row, a row with a
    NaN among finite values, and a row of exact RHE ties."""
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=seed))
    if M >= 4:
        x[1] = 0
        x[2, 3] = 0x7FC0                       # NaN: skipped by the absmax, quantizes to 0
        j = np.arange(K, dtype=np.float32) % 64 - 32
        ties = ((2 * j + 1) / 8).astype(np.float32)
        ties[0] = 31.75                        # absmax 31.75: scale 0.25, quotients j + 0.5
        x[3] = oracle.f32_to_bf16(ties)
    return x


@pytest.mark.parametrize("M,K", [(1, 512), (5, 4096), (300, 8192), (7, 48), (3, 1000),
                                 (2, 8704), (129, 2560), (3, 1024), (5, 3072), (6, 6144),
                                 # large row counts (C4's x among them)
                                 (2048, 4096), (2047, 4096), (16385, 512), (5101, 1536),
                                 (1030, 8192), (2050, 3072)])
def test_quantize_rows_bf16_bit_exact(oracle, dev, M, K):
    """Register paths with 1, 2 and 4 waves per row (K = 512 n), odd row
    counts (a workgroup's last row past M), and the two-pass kernel."""
    x = _x_with_edges(oracle, M, K, seed=M + K)
    xq, sx = mj.quantize_rows_bf16_int8(bf16_dev(x, dev))
    q_ref, s_ref = oracle.quantize_rowwise_rhe(oracle.bf16_to_f32(x))
    np.testing.assert_array_equal(xq.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sx.cpu().numpy(), s_ref)


def test_quantize_rows_bf16_unaligned(oracle, dev):
    """x 8 bytes off a 16-byte boundary: the register path needs 16-byte rows,
    so the generic two-pass kernel runs; results are the same."""
    M, K = 6, 1024
    x = _x_with_edges(oracle, M, K, seed=5)
    buf = torch.empty(M * K + 4, dtype=torch.bfloat16, device=dev)
    xv = buf[4:].view(M, K)
    xv.copy_(bf16_dev(x, dev))
    assert xv.data_ptr() % 16 == 8
    xq, sx = mj.quantize_rows_bf16_int8(xv)
    q_ref, s_ref = oracle.quantize_rowwise_rhe(oracle.bf16_to_f32(x))
    np.testing.assert_array_equal(xq.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sx.cpu().numpy(), s_ref)


def _w8a8_case(oracle, M, N, K, seed):
    x = _x_with_edges(oracle, M, K, seed)
    rng = np.random.default_rng(seed)
    Q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = oracle.randu_f32((N,), 0.0005, 0.004, seed=seed + 1)
    b = oracle.randu_f32((N,), -0.25, 0.25, seed=seed + 2)
    return x, Q, sw, b


@pytest.mark.parametrize("M,N,K,epi,with_bias", [
    (1, 384, 512, mj.EPI_NONE, True),
    (37, 200, 160, mj.EPI_RELU, True),          # ragged N, K % 128 = 32
    (256, 1000, 4096, mj.EPI_NONE, False),      # 256 x 128 tiles, no bias
    (300, 520, 1040, mj.EPI_RELU_UNARY, True),  # two row tiles, ragged
    (513, 768, 2048, mj.EPI_NONE, True),
])
def test_w8a8_linear_bit_exact(oracle, dev, M, N, K, epi, with_bias):
    x, Q, sw, b = _w8a8_case(oracle, M, N, K, seed=M + N + K)
    bias = b if with_bias else None
    lin = mj.W8A8Linear(to_dev(Q, dev), to_dev(sw, dev), None if bias is None else to_dev(b, dev),
                        epi)
    got = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    ref, _, _, _ = oracle.linear_w8a8(x, Q, sw, bias, epi)
    np.testing.assert_array_equal(got, ref)
    assert np.any(got != 0)


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096),    # C4's shape: 256 tiles of 256 x 128
                                   (3072, 4096, 1040)])   # 192 tiles of 256 x 256, K tail
def test_w8a8_linear_large_bit_exact(oracle, dev, M, N, K):
    """Full-size shapes checked bit for bit on one row of every 128-row block
    (whole rows, so every column tile is covered)."""
    x, Q, sw, b = _w8a8_case(oracle, M, N, K, seed=7)
    lin = mj.W8A8Linear(to_dev(Q, dev), to_dev(sw, dev), to_dev(b, dev), mj.EPI_NONE)
    got = bf16_host_bits(lin.forward(bf16_dev(x, dev)))
    rows = slab_rows(M)
    assert_tiles_covered(M, N, rows, [])
    for r in rows:
        ref, _, _, _ = oracle.linear_w8a8(x, Q, sw, b, mj.EPI_NONE, rows=(r, r + 1))
        np.testing.assert_array_equal(got[r:r + 1], ref, err_msg=f"row {r}")


@pytest.mark.parametrize("epi", [mj.EPI_GELU_TANH, mj.EPI_SILU])
def test_w8a8_gelu_silu_epilogue(oracle, dev, epi):
    """GELU / SiLU in the bf16-output forms (hardware exp2 and reciprocal):
    every output within one bf16 step (2^-7 relative) of the oracle's fp32
    value before rounding, or 1e-6 absolute; apart from GELU below -2 (where
    the literal 1 + tanh(t) cancels), at most 1 % of the outputs differ in any
    bit.  The pre-activations span [-4, 4] and beyond."""
    M, N, K = 300, 256, 512
    x, Q, sw, b = _w8a8_case(oracle, M, N, K, seed=30 + epi)
    lin = mj.W8A8Linear(to_dev(Q, dev), to_dev(sw, dev), to_dev(b, dev), epi)
    got_t = lin.forward(bf16_dev(x, dev))
    got_bits, got = bf16_host_bits(got_t), bf16_host_f32(got_t)
    ref_bits, ref, _, _ = oracle.linear_w8a8(x, Q, sw, b, epi)
    ref = ref.astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    bound = np.maximum(np.abs(ref) * 2.0 ** -7, 1e-6)
    worst = int(np.argmax(err - bound))
    assert np.all(err <= bound), (worst, got.flat[worst], ref.flat[worst])
    _, pre, _, _ = oracle.linear_w8a8(x, Q, sw, b, mj.EPI_NONE)
    keep = pre >= -2.0 if epi == mj.EPI_GELU_TANH else np.ones(pre.shape, bool)
    frac = float(np.mean(got_bits[keep] != ref_bits[keep]))
    print(f"epi={epi}: {frac:.4%} of {int(keep.sum())} outputs differ in some bit", flush=True)
    assert frac <= 0.01
    assert float(pre.min()) < -4.0 and float(pre.max()) > 4.0 and np.mean(np.abs(pre) < 2) > 0.2


@pytest.mark.parametrize("M,N,with_rows,with_bias", [(1, 1, True, True), (37, 1001, True, True),
                                                    (300, 514, False, True), (5, 7, True, False)])
def test_dequantize_i32_scaled_bit_exact(oracle, dev, M, N, with_rows, with_bias):
    rng = np.random.default_rng(M * 7 + N)
    acc = rng.integers(-(2 ** 31), 2 ** 31 - 1, size=(M, N)).astype(np.int32)
    sw = oracle.randu_f32((N,), 1e-4, 1e-2, seed=N)
    sx = oracle.randu_f32((M,), 1e-3, 1e-1, seed=M) if with_rows else None
    b = oracle.randu_f32((N,), -1, 1, seed=N + 1) if with_bias else None
    got = mj.dequantize_i32_scaled(mj.Tensor(to_dev(acc, dev)), mj.Tensor(to_dev(sw, dev)),
                                   None if b is None else mj.Tensor(to_dev(b, dev)),
                                   None if sx is None else mj.Tensor(to_dev(sx, dev))).numpy()
    np.testing.assert_array_equal(got, oracle.dequant_i32_scaled(acc, sw, b, sx))


def test_w8a8_is_quantize_matmul_dequantize(oracle, dev):
    """The W8A8 Linear equals its three steps run as separate operators: the
    row quantize, the int8 x int8 -> int32 GEMM, and the per-row/per-channel
    dequantize + bias, rounded to bf16."""
    M, N, K = 200, 300, 1024
    x, Q, sw, b = _w8a8_case(oracle, M, N, K, seed=61)
    xd, Qd = bf16_dev(x, dev), to_dev(Q, dev)
    y = bf16_host_bits(mj.W8A8Linear(Qd, to_dev(sw, dev), to_dev(b, dev)).forward(xd))
    xq, sx = mj.quantize_rows_bf16_int8(xd)
    acc = mj.matmul_i8_i8_to_i32(mj.Tensor(xq), mj.Tensor(Qd).transpose())
    yf = mj.dequantize_i32_scaled(acc, mj.Tensor(to_dev(sw, dev)), mj.Tensor(to_dev(b, dev)),
                                  mj.Tensor(sx))
    np.testing.assert_array_equal(y, bf16_host_bits(yf.torch.to(torch.bfloat16)))


def test_w8a8_close_to_w8a16(oracle, dev):
    """Quantizing the activations costs at most about half an int8 step per
    element: W8A8 and W8A16 outputs of the same layer agree to a few percent
    of the output range."""
    M, N, K = 64, 512, 1024
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=51))
    W = oracle.randn_f32((N, K), std=0.02, seed=52)
    q, s = mj.quantize_rowwise_int8(to_dev(W, dev))
    xd = bf16_dev(x, dev)
    y8 = bf16_host_f32(mj.W8A8Linear(q, s).forward(xd)).astype(np.float64)
    y16 = bf16_host_f32(mj.W8Linear(q, s).forward(xd)).astype(np.float64)
    rel = np.abs(y8 - y16).max() / np.abs(y16).max()
    assert rel < 0.03, rel


def test_w8a8_rejects_unsupported(dev):
    q = torch.zeros((32, 40), dtype=torch.int8, device=dev)
    s = torch.ones(32, dtype=torch.float32, device=dev)
    with pytest.raises(mj.MomijoHipError):
        mj.W8A8Linear(q, s).forward(torch.zeros((4, 40), dtype=torch.bfloat16, device=dev))
