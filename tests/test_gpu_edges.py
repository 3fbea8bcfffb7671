"""Edge cases of the GEMM entry points through the C ABI: padded leading
dimensions (the kernel must read only K of each row and write only N of each
output row), the split-K reduce path with bias and activation, the GEMV/GEMM
switch of the W8A16 Linear, and every epilogue.

Bars as elsewhere: max|d| / max|ref| <= 2e-2 for bf16 outputs against the
oracle; the padding columns of C must keep their sentinel bits exactly.
"""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib
from _util import bf16_dev, bf16_host_f32, normwise_rel, to_dev

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
SENTINEL = 0x1357  # bf16 bits written into C's padding before the call


def _ptr(t):
    return t.data_ptr()


def _padded_gemm(oracle, dev, M, N, K, pad_a, pad_b, pad_c, bias, epi, seed):
    A = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=seed))
    B = oracle.f32_to_bf16(oracle.randn_f32((N, K), seed=seed + 1))
    lda, ldb, ldc = K + pad_a, K + pad_b, N + pad_c
    rng = np.random.default_rng(seed)
    A_pad = rng.integers(0, 2**16, size=(M, lda), dtype=np.uint16)  # garbage in the padding
    B_pad = rng.integers(0, 2**16, size=(N, ldb), dtype=np.uint16)
    A_pad[:, :K] = A
    B_pad[:, :K] = B
    C_pad = np.full((M, ldc), SENTINEL, np.uint16)
    a, b_, c = bf16_dev(A_pad, dev), bf16_dev(B_pad, dev), bf16_dev(C_pad, dev)
    bt = None if bias is None else to_dev(bias, dev)
    _lib.call("mj_gemm_bf16_nt", M, N, K, _ptr(a), lda, _ptr(b_), ldb,
              None if bt is None else _ptr(bt), epi, _ptr(c), ldc,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got_bits = c.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.all(got_bits[:, N:] == SENTINEL), "padding columns of C were written"
    got = bf16_host_f32(c)[:, :N]
    rows = sorted({0, 1, M // 2, M - 1})
    for r in rows:
        _, ref = oracle.gemm_bf16_nt(A, B, bias, epi, rows=(r, r + 1))
        err = np.max(np.abs(got[r] - ref[0])) / max(np.max(np.abs(ref[0])), 1e-30)
        assert err <= BF16_TOL, f"row {r}: {err:.3e}"


@pytest.mark.parametrize("M,N,K,pad_c", [(300, 200, 520, 24),    # 128 x 128 tiles
                                         (300, 200, 520, 3),     # ldc % 8 != 0: scalar stores
                                         (3000, 2600, 136, 24),  # 256 x 256, distance-2 pipeline
                                         (32, 512, 8192, 24)])   # split-K with the reduce kernel
def test_bf16_padded_leading_dims(oracle, dev, M, N, K, pad_c):
    bias = oracle.randu_f32((N,), -0.5, 0.5, seed=N)
    _padded_gemm(oracle, dev, M, N, K, 64, 40, pad_c, bias, mj.EPI_SILU, seed=M + N)


@pytest.mark.parametrize("epi", [mj.EPI_NONE, mj.EPI_RELU, mj.EPI_GELU_TANH, mj.EPI_SILU,
                                 mj.EPI_GELU_TANH_APPROX, mj.EPI_SILU_APPROX,
                                 mj.EPI_RELU_UNARY])
def test_bf16_split_k_every_epilogue(oracle, dev, epi):
    """The split-K reduce kernel applies scale, bias and the activation."""
    bias = oracle.randu_f32((256,), -0.5, 0.5, seed=epi)
    _padded_gemm(oracle, dev, 16, 256, 4096, 0, 0, 8, bias, epi, seed=100 + epi)


def _w8(oracle, M, N, K, seed):
    x = oracle.f32_to_bf16(oracle.randn_f32((M, K), seed=seed))
    W = oracle.randn_f32((N, K), std=0.02, seed=seed + 1)
    Q, s = oracle.quantize_rowwise_rhe(W)
    b = oracle.randu_f32((N,), -1.0 / 16, 1.0 / 16, seed=seed + 2)
    return x, Q, s, b


@pytest.mark.parametrize("M", [2, 3, 16, 17])
@pytest.mark.parametrize("epi", [mj.EPI_NONE, mj.EPI_RELU, mj.EPI_GELU_TANH, mj.EPI_SILU,
                                 mj.EPI_GELU_TANH_APPROX, mj.EPI_SILU_APPROX,
                                 mj.EPI_RELU_UNARY])
def test_w8a16_gemv_gemm_switch_every_epilogue(oracle, dev, M, epi):
    """M = 2 is the last streaming-GEMV size, M = 3 the first skinny-MFMA GEMV
    size, M = 16 its last and M = 17 the first MFMA GEMM size."""
    x, Q, s, b = _w8(oracle, M, 192, 512, M * 10 + epi)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), epi)
    y = bf16_host_f32(lin.forward(bf16_dev(x, dev)))
    _, ref = oracle.linear_w8a16(x, Q, s, b, epi)
    assert normwise_rel(y, ref) <= BF16_TOL


def test_w8a16_split_k_bias_gelu(oracle, dev):
    """M = 64 against K = 4096 runs the int8 GEMM with a K split, so bias and
    GELU go through the reduce kernel."""
    x, Q, s, b = _w8(oracle, 64, 1024, 4096, 7)
    lin = mj.W8Linear(to_dev(Q, dev), to_dev(s, dev), to_dev(b, dev), mj.EPI_GELU_TANH)
    y = bf16_host_f32(lin.forward(bf16_dev(x, dev)))
    _, ref = oracle.linear_w8a16(x, Q, s, b, mj.EPI_GELU_TANH)
    assert normwise_rel(y, ref) <= BF16_TOL


def test_w8a16_split_k_unaligned_scales_bias(oracle, dev):
    """Scales and bias 4 bytes past a 16-byte boundary: the split-K reduce
    reads them per element (its 16-byte loads need aligned vectors), with the
    same result."""
    x, Q, s, b = _w8(oracle, 64, 1024, 4096, 8)
    s_store = torch.zeros(1025, dtype=torch.float32, device=dev)
    b_store = torch.zeros(1025, dtype=torch.float32, device=dev)
    s_store[1:].copy_(to_dev(s, dev))
    b_store[1:].copy_(to_dev(b, dev))
    s_dev, b_dev = s_store[1:], b_store[1:]
    assert s_dev.data_ptr() % 16 == 4 and b_dev.data_ptr() % 16 == 4
    lin = mj.W8Linear(to_dev(Q, dev), s_dev, b_dev, mj.EPI_GELU_TANH)
    y = bf16_host_f32(lin.forward(bf16_dev(x, dev)))
    _, ref = oracle.linear_w8a16(x, Q, s, b, mj.EPI_GELU_TANH)
    assert normwise_rel(y, ref) <= BF16_TOL


def test_unaligned_operands_are_rejected(dev):
    """The bf16 GEMM needs 16-byte aligned operands and K % 8 == 0: anything
    else is MJ_ERR_UNSUPPORTED, not a fault."""
    a = torch.zeros((64, 72), dtype=torch.bfloat16, device=dev)
    b = torch.zeros((64, 72), dtype=torch.bfloat16, device=dev)
    c = torch.zeros((64, 64), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    st = lib.mj_gemm_bf16_nt(64, 64, 70, _ptr(a), 72, _ptr(b), 72, None, 0, _ptr(c), 64, None)
    assert st == 3  # MJ_ERR_UNSUPPORTED: K % 8
    st = lib.mj_gemm_bf16_nt(64, 64, 64, _ptr(a) + 2, 72, _ptr(b), 72, None, 0, _ptr(c), 64, None)
    assert st == 3  # misaligned A
    assert not c.any()


# fp32 bit patterns whose bf16 rounding is easy to get wrong: ties to even in
# both directions, just below / above a tie, denormals (and a denormal tie),
# the largest finite values (one rounds up to Inf), infinities, signed zeros
# and quiet / signalling NaNs with payloads.
_SPECIAL_BITS = [
    0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001, 0xBF808000, 0xBF818000, 0x3F80C000,
    0x00000001, 0x00008000, 0x00018000, 0x007FFFFF, 0x80000001, 0x80018000, 0x00800000,
    0x7F7FFFFF, 0x7F7F7FFF, 0x7F7F8000, 0xFF7FFFFF, 0x7F800000, 0xFF800000,
    0x00000000, 0x80000000, 0x7FC00000, 0x7FC12345, 0xFFC00000, 0x7F800001, 0x7FA00000,
    0x40490FDB, 0xC2F6E979, 0x3EAAAAAB,
]


def _special_bias(n, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    bits[:len(_SPECIAL_BITS)] = np.array(_SPECIAL_BITS, np.uint32)
    return bits.view(np.float32)


def _expected_bf16(oracle, bias):
    # the kernels compute 0.0f + bias in fp32 and round that to bf16
    with np.errstate(invalid="ignore"):
        return oracle.f32_to_bf16((np.float32(0.0) + bias).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(16, 256, 16),        # small tiles
                                   (4096, 4096, 64)])    # 256 x 256 tiles
def test_bf16_output_rounding_special_values(oracle, dev, M, N, K):
    """Zero operands make every output exactly bf16(0 + bias[n]), so the bias
    drives the kernels' fp32 -> bf16 rounding through special values; the bits
    must equal the oracle's round-to-nearest-even conversion."""
    bias = _special_bias(N, seed=N)
    A = torch.zeros((M, K), dtype=torch.bfloat16, device=dev)
    B = torch.zeros((N, K), dtype=torch.bfloat16, device=dev)
    C = mj.gemm_bf16_nt(A, B, to_dev(bias, dev), mj.EPI_NONE)
    got = C.view(torch.int16).cpu().numpy().view(np.uint16)
    want = _expected_bf16(oracle, bias)
    bad = np.nonzero(got != want[None, :])
    assert bad[0].size == 0, (f"{bad[0].size} mismatches, first at {bad[0][0]},{bad[1][0]}: "
                              f"in {bias.view(np.uint32)[bad[1][0]]:#010x} "
                              f"got {got[bad[0][0], bad[1][0]]:#06x} want {want[bad[1][0]]:#06x}")


@pytest.mark.parametrize("M", [1, 64])
def test_w8a16_output_rounding_special_values(oracle, dev, M):
    """The same check through the W8A16 GEMV (M = 1) and GEMM (M = 64)."""
    N, K = 512, 256
    bias = _special_bias(N, seed=M)
    q = torch.zeros((N, K), dtype=torch.int8, device=dev)
    s = torch.ones((N,), dtype=torch.float32, device=dev)
    x = torch.zeros((M, K), dtype=torch.bfloat16, device=dev)
    y = mj.W8Linear(q, s, to_dev(bias, dev)).forward(x)
    got = y.view(torch.int16).cpu().numpy().view(np.uint16)
    want = _expected_bf16(oracle, bias)
    bad = np.nonzero(got != want[None, :])
    assert bad[0].size == 0, (f"{bad[0].size} mismatches, first at {bad[0][0]},{bad[1][0]}: "
                              f"in {bias.view(np.uint32)[bad[1][0]]:#010x} "
                              f"got {got[bad[0][0], bad[1][0]]:#06x} want {want[bad[1][0]]:#06x}")


# ------------------------------------------------------------- host-side validation
def test_quant_linear_shape_mismatch_returns_empty(oracle, dev):
    """QuantLinear.forward on a non-2-D x or a width other than in_features
    returns the reference's empty [0, 0] result (matmul_i8_i8_to_i32's
    fallback, functional.mojo:253-263) instead of reading past w_q."""
    Wq = np.zeros((8, 16), np.int8)
    q = mj.QuantLinear(16, 8, mj.Tensor(to_dev(Wq, dev)),
                       mj.Tensor(to_dev(np.zeros(8, np.float32), dev)), 0.1, 0.1)
    for shape in ((4, 32), (4, 8), (16,), (2, 4, 16)):
        y = q.forward(mj.Tensor(to_dev(np.ones(shape, np.float32), dev)))
        assert y.shape() == [0, 0] and y.dtype == torch.float32
    assert q.forward(mj.Tensor(to_dev(np.ones((3, 16), np.float32), dev))).shape() == [3, 8]
    with pytest.raises(ValueError):   # w_q not [out, in]
        mj.QuantLinear(16, 8, mj.Tensor(to_dev(np.zeros((16, 8), np.int8), dev)),
                       mj.Tensor(to_dev(np.zeros(8, np.float32), dev)), 0.1, 0.1)
    with pytest.raises(ValueError):   # bias length
        mj.QuantLinear(16, 8, mj.Tensor(to_dev(Wq, dev)),
                       mj.Tensor(to_dev(np.zeros(7, np.float32), dev)), 0.1, 0.1)


def test_w8_layers_reject_bad_operands(dev):
    q = torch.zeros((32, 64), dtype=torch.int8, device=dev)
    s = torch.ones(32, dtype=torch.float32, device=dev)
    lin = mj.W8Linear(q, s)
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device=dev)
    assert lin.forward(x).shape == (4, 32)
    with pytest.raises(TypeError):
        lin.forward(x.float())
    with pytest.raises(ValueError):
        lin.forward(torch.zeros((4, 128), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):   # row-strided view: the ABI takes lda = K
        lin.forward(torch.zeros((4, 128), dtype=torch.bfloat16, device=dev)[:, :64])
    with pytest.raises(ValueError):
        lin.forward(x, out=torch.empty((4, 31), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):
        mj.W8Linear(q, s[:31])
    down = mj.W8Linear(torch.zeros((64, 32), dtype=torch.int8, device=dev),
                       torch.ones(64, dtype=torch.float32, device=dev))
    mlp = mj.W8MLP(lin, mj.W8Linear(q, s), down)
    y, h = mlp.forward(x)
    assert y.shape == (4, 64) and h.shape == (4, 32)
    with pytest.raises(ValueError):   # x wider than the gate's in_features
        mlp.forward(torch.zeros((4, 96), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):
        mlp.forward(x, h=torch.empty((4, 16), dtype=torch.bfloat16, device=dev))
    with pytest.raises(TypeError):
        mlp.forward(x.float())


def test_gemm_bf16_nt_rejects_bad_operands(dev):
    A = torch.zeros((8, 32), dtype=torch.bfloat16, device=dev)
    W = torch.zeros((16, 32), dtype=torch.bfloat16, device=dev)
    assert mj.gemm_bf16_nt(A, W).shape == (8, 16)
    with pytest.raises(TypeError):
        mj.gemm_bf16_nt(A.float(), W)
    with pytest.raises(ValueError):   # K mismatch
        mj.gemm_bf16_nt(A, torch.zeros((16, 48), dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):   # transposed operand (column stride != 1)
        mj.gemm_bf16_nt(A, torch.zeros((32, 16), dtype=torch.bfloat16, device=dev).t())
    with pytest.raises(ValueError):
        mj.gemm_bf16_nt(A, W, out=torch.empty((8, 8), dtype=torch.bfloat16, device=dev))
