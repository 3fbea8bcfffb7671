"""Conv2d.forward (learn/nn/conv.mojo:600-681) on the implicit-GEMM fp32
kernel against the oracle: bit for bit on integer-valued data (every sum
exact in any order) over geometries that reach each tile size, padding
clipping, strides and empty outputs; N(0,1) data at the fp32 bar; the
reference seam launch_1d_conv2d_fw (tensor/gpu/runtime.mojo:376-470) on host
buffers."""
import numpy as np
import pytest
import torch

import momijo_amd as mj
from momijo_amd import _lib, seam
from _util import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu


def _int_case(shape, seed):
    N, C, H, W, OC, kH, kW = shape[:7]
    rng = np.random.default_rng(seed)
    x = rng.integers(-8, 9, size=(N, C, H, W)).astype(np.float32)
    w = rng.integers(-8, 9, size=(OC, C, kH, kW)).astype(np.float32)
    b = rng.integers(-64, 65, size=OC).astype(np.float32)
    return x, w, b


def _conv(dev, x, w, b, stride, pad, epi=mj.EPI_NONE):
    OC, C, kH, kW = w.shape
    layer = mj.Conv2d(C, OC, (kH, kW), stride, pad, bias=b is not None)
    layer.weight = mj.Tensor(to_dev(w, dev))
    if b is not None:
        layer.bias_t = mj.Tensor(to_dev(b, dev))
    return layer.forward_act(mj.Tensor(to_dev(x, dev)), epi).numpy()


@pytest.mark.parametrize("shape", [
    # N, C, H, W, OC, kH, kW, sH, sW, pH, pW
    (1, 1, 5, 5, 1, 3, 3, 1, 1, 1, 1),          # tiny: 32 x 32 tiles
    (2, 3, 9, 7, 5, 3, 3, 1, 1, 1, 1),
    (4, 16, 28, 28, 32, 3, 3, 1, 1, 1, 1),      # 64 x 64 tiles
    (2, 8, 31, 17, 40, 5, 3, 2, 3, 2, 1),       # ragged, strided, asymmetric
    (8, 16, 64, 64, 256, 3, 3, 1, 1, 1, 1),     # 128 x 128 tiles
    (3, 4, 10, 11, 6, 1, 1, 1, 1, 0, 0),        # 1 x 1
    (2, 2, 5, 5, 3, 3, 3, 1, 1, 4, 4),          # windows entirely in the padding
    (1, 6, 4, 9, 7, 4, 9, 1, 1, 0, 0),          # kernel as wide as the input
    (2, 24, 12, 12, 20, 7, 7, 3, 3, 3, 3),      # K = 1176: many K stages, carries of every digit
    (3, 5, 33, 47, 70, 5, 3, 2, 1, 2, 1),       # ragged channel and pixel tiles, K = 75
    (9, 8, 60, 60, 96, 3, 3, 1, 1, 1, 1),       # 224-pixel tiles: ragged channels and pixels
    (96, 8, 61, 59, 64, 4, 2, 2, 3, 1, 0),      # 224-pixel tiles: strided, even kernel
])
@pytest.mark.parametrize("with_bias", [True, False])
def test_conv2d_integer_inputs_bit_exact(oracle, dev, shape, with_bias):
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    x, w, b = _int_case(shape, seed=sum(shape))
    b = b if with_bias else None
    got = _conv(dev, x, w, b, (sH, sW), (pH, pW))
    want = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW))
    assert got.shape == want.shape
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape", [
    (2, 16, 14, 14, 24, 3, 3, 1, 1, 1, 1),
    (1, 64, 28, 28, 64, 3, 3, 2, 2, 1, 1),
    (2, 3, 33, 35, 16, 7, 7, 2, 2, 3, 3),
])
def test_conv2d_random_fp32(oracle, dev, shape):
    """N(0,1) x, He-scaled weights, bias U(-1/16, 1/16): the fp32 bar
    |d| <= 1e-5 + 1e-5 |ref| against the strict-order oracle."""
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    seed = sum(shape)
    x = oracle.randn_f32((N, C, H, W), seed=seed)
    w = oracle.randn_f32((OC, C, kH, kW), std=float(np.sqrt(2.0 / (C * kH * kW))), seed=seed + 1)
    b = oracle.randu_f32((OC,), -1 / 16, 1 / 16, seed=seed + 2)
    got = _conv(dev, x, w, b, (sH, sW), (pH, pW))
    want = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW))
    assert_close_f32(got, want)


def test_conv2d_fused_relu_and_empty_outputs(oracle, dev):
    shape = (2, 5, 8, 9, 7, 3, 3, 1, 2, 1, 0)
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    x, w, b = _int_case(shape, seed=3)
    got = _conv(dev, x, w, b, (sH, sW), (pH, pW), mj.EPI_RELU)
    want = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW))
    np.testing.assert_array_equal(got, np.where(want > 0, want, np.float32(0)))
    # kernel larger than the padded input: OH <= 0, an empty result
    layer = mj.Conv2d(2, 3, (5, 5))
    y = layer.forward(mj.Tensor(torch.ones((1, 2, 3, 3), device=dev)))
    assert tuple(y.torch.shape) == (1, 3, 0, 0)
    with pytest.raises(ValueError):
        layer.forward(mj.Tensor(torch.ones((1, 4, 9, 9), device=dev)))   # wrong channels


def test_conv2d_seam_host_buffers(oracle, dev):
    """launch_1d_conv2d_fw on numpy buffers takes the device path and writes
    the oracle's result in place; OH / OW that disagree with the geometry
    are refused by the library (the caller's kernel then runs, as the
    reference's fallback does)."""
    shape = (2, 3, 9, 7, 5, 3, 3, 2, 1, 1, 1)
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    x, w, b = _int_case(shape, seed=17)
    OH, OW = oracle.conv_out_size(H, kH, sH, pH), oracle.conv_out_size(W, kW, sW, pW)
    y = np.zeros(N * OC * OH * OW, np.float32)
    calls = []
    path = seam.launch_1d_conv2d_fw(N * OC * OH * OW, 256, lambda *a: calls.append(a),
                                    x.reshape(-1), w.reshape(-1), b, y, N, C, H, W, OH, OW, OC,
                                    kH, kW, sH, sW, pH, pW, True)
    assert path == "gpu" and not calls
    np.testing.assert_array_equal(y.reshape(N, OC, OH, OW),
                                  oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW)))
    st = _lib.load().mj_launch_conv2d_fw_h(x.ctypes.data, w.ctypes.data, b.ctypes.data,
                                           y.ctypes.data, N, C, H, W, OH + 1, OW, OC, kH, kW,
                                           sH, sW, pH, pW, 1)
    assert st == _lib.MJ_ERR_SHAPE


def _conv_path(M, Ng, N):
    """The launcher's choice (gemm_f32.hip launch_conv2d_f32): for OC >= 64
    the 224- or 256-pixel tile kernel when its grid has >= 192 workgroups,
    else the square tiles of the matmul engine."""
    if M >= 64:
        best, pick, wgs_pick = None, None, 0
        for c in (8, 7):
            tbn = 32 * c
            wgs = ((M + 63) // 64) * ((Ng + tbn - 1) // tbn) * N
            cost = (wgs + 255) // 256 * tbn
            if best is None or cost < best:
                best, pick, wgs_pick = cost, tbn, wgs
        if wgs_pick >= 192:
            return pick
    return "square"


_IM2COL_SHAPES = [
    # N, C, H, W, OC, kH, kW, sH, sW, pH, pW
    (2, 16, 14, 14, 64, 3, 3, 1, 1, 1, 1),      # square tiles
    (3, 5, 33, 47, 70, 5, 3, 2, 1, 2, 1),       # square tiles, ragged
    (8, 32, 40, 40, 96, 3, 3, 1, 1, 1, 1),      # square tiles, two channel tiles
    (32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1),     # 224: the bench layer
    (9, 8, 60, 60, 96, 3, 3, 1, 1, 1, 1),       # 224, ragged channel and pixel tiles
    (96, 8, 61, 59, 64, 4, 2, 2, 3, 1, 0),      # 224, strided, even kernel, no vertical padding
    (8, 16, 64, 64, 256, 3, 3, 1, 1, 1, 1),     # 256
]


def test_im2col_shapes_reach_every_conv_path():
    paths = set()
    for (N, C, H, W, OC, kH, kW, sH, sW, pH, pW) in _IM2COL_SHAPES:
        OH, OW = (H + 2 * pH - kH) // sH + 1, (W + 2 * pW - kW) // sW + 1
        paths.add(_conv_path(OC, OH * OW, N))
    assert paths == {"square", 224, 256}


@pytest.mark.parametrize("shape", _IM2COL_SHAPES)
@pytest.mark.parametrize("epi", [mj.EPI_NONE, mj.EPI_RELU])
def test_conv2d_equals_library_matmul_on_im2col(dev, shape, epi):
    """N(0,1) data: the convolution is, bit for bit, the library's fp32
    matmul of the flattened weight with torch's unfold of each image (an
    exact copy of the taps, zeros in the padding), plus the bias in one fp32
    rounding, then the activation: both run the MFMA sums in the same k
    order."""
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn((N, C, H, W), generator=g)
    w = torch.randn((OC, C, kH, kW), generator=g) * (2.0 / (C * kH * kW)) ** 0.5
    b = torch.rand(OC, generator=g) / 8 - 1 / 16
    got = _conv(dev, x.numpy(), w.numpy(), b.numpy(), (sH, sW), (pH, pW), epi)
    cols = torch.nn.functional.unfold(x.to(dev), (kH, kW), padding=(pH, pW), stride=(sH, sW))
    wf = mj.Tensor(w.reshape(OC, -1).contiguous().to(dev))
    for n in range(N):
        prod = mj.matmul(wf, mj.Tensor(cols[n].contiguous())).torch
        want = prod + b.to(dev)[:, None]
        if epi == mj.EPI_RELU:
            want = torch.where(want > 0, want, torch.zeros_like(want))
        np.testing.assert_array_equal(got[n].reshape(OC, -1), want.cpu().numpy())
