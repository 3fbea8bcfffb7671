"""Pins the oracle's Conv2d.forward (learn/nn/conv.mojo:600-681) without the
reference: exact integer sums, the 1 x 1 case against the pinned matmul,
delta kernels, the strict-order float32 loop, and torch's CPU conv2d within
the fp32 summation bound."""
import numpy as np
import pytest
import torch


def _int_conv_padded(x, w, b, stride, pad):
    """int64 conv2d with explicit zero padding (numpy windows): exact."""
    N, C, H, W = x.shape
    OC, _, kH, kW = w.shape
    sH, sW = stride
    pH, pW = pad
    xp = np.pad(x.astype(np.int64), ((0, 0), (0, 0), (pH, pH), (pW, pW)))
    OH = (H + 2 * pH - kH) // sH + 1
    OW = (W + 2 * pW - kW) // sW + 1
    y = np.zeros((N, OC, OH, OW), np.int64)
    for ky in range(kH):
        for kx in range(kW):
            win = xp[:, :, ky:ky + sH * (OH - 1) + 1:sH, kx:kx + sW * (OW - 1) + 1:sW]
            y += np.einsum("nchw,oc->nohw", win, w[:, :, ky, kx].astype(np.int64))
    if b is not None:
        y += b.astype(np.int64)[None, :, None, None]
    return y


@pytest.mark.parametrize("shape", [
    # N, C, H, W, OC, kH, kW, sH, sW, pH, pW
    (2, 3, 9, 7, 5, 3, 3, 1, 1, 1, 1),
    (1, 4, 10, 11, 6, 3, 2, 2, 3, 1, 0),
    (3, 2, 8, 8, 4, 5, 5, 2, 2, 2, 2),
    (1, 1, 5, 5, 2, 3, 3, 1, 1, 4, 4),     # windows entirely in the padding
    (2, 5, 6, 4, 3, 1, 1, 1, 1, 0, 0),
    (1, 2, 4, 9, 3, 4, 9, 1, 1, 0, 0),     # kernel as wide as the input
])
def test_conv2d_integer_inputs_exact(oracle, shape):
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = shape
    rng = np.random.default_rng(sum(shape))
    x = rng.integers(-8, 9, size=(N, C, H, W)).astype(np.float32)
    w = rng.integers(-8, 9, size=(OC, C, kH, kW)).astype(np.float32)
    b = rng.integers(-8, 9, size=OC).astype(np.float32)
    got = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW))
    want = _int_conv_padded(x, w, b, (sH, sW), (pH, pW))
    np.testing.assert_array_equal(got, want.astype(np.float32))
    # image slabs give the same rows
    part = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW), images=(N - 1, N))
    np.testing.assert_array_equal(part, got[N - 1:N])


def test_conv2d_1x1_is_the_matmul(oracle):
    """A 1 x 1, stride-1 convolution sums over the input channels in
    ascending order, as the pinned matmul does: bit-exact per image."""
    rng = np.random.default_rng(7)
    N, C, H, W, OC = 2, 37, 5, 6, 11
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, C, 1, 1)).astype(np.float32)
    y = oracle.conv2d_fw_f32(x, w)
    for n in range(N):
        ref = oracle.matmul_f32(w[:, :, 0, 0], x[n].reshape(C, H * W))
        np.testing.assert_array_equal(y[n].reshape(OC, H * W), ref)


def test_conv2d_delta_kernels_shift(oracle):
    """w = delta at (dy, dx) on the diagonal of (oc, ic): y is x shifted by
    (dy - pH, dx - pW), zeros where the tap falls in the padding."""
    rng = np.random.default_rng(9)
    N, C, H, W = 2, 3, 7, 6
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    for dy, dx in [(0, 0), (1, 2), (2, 1)]:
        w = np.zeros((C, C, 3, 3), np.float32)
        for c in range(C):
            w[c, c, dy, dx] = 1.0
        y = oracle.conv2d_fw_f32(x, w, None, (1, 1), (1, 1))
        xp = np.pad(x, ((0, 0), (0, 0), (1, 1), (1, 1)))
        np.testing.assert_array_equal(y, xp[:, :, dy:dy + H, dx:dx + W])


def test_conv2d_strict_order_and_clipping(oracle):
    """The float32 loop over the clipped window (ic, ky, kx ascending, one
    rounding per multiply and add, bias last), written out in numpy float32
    on a case whose windows are clipped at every border."""
    rng = np.random.default_rng(11)
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = 1, 3, 5, 4, 2, 3, 3, 2, 1, 1, 2
    x = (rng.standard_normal((N, C, H, W)) * 3).astype(np.float32)
    w = rng.standard_normal((OC, C, kH, kW)).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32)
    y = oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW))
    OH, OW = (H + 2 * pH - kH) // sH + 1, (W + 2 * pW - kW) // sW + 1
    f = np.float32
    for oc in range(OC):
        for oy in range(OH):
            for ox in range(OW):
                s = f(0)
                for ic in range(C):
                    for ky in range(kH):
                        for kx in range(kW):
                            iy, ix = oy * sH - pH + ky, ox * sW - pW + kx
                            if 0 <= iy < H and 0 <= ix < W:
                                s = f(s + f(x[0, ic, iy, ix] * w[oc, ic, ky, kx]))
                s = f(s + b[oc])
                assert y[0, oc, oy, ox] == s, (oc, oy, ox)


def test_conv2d_against_torch_cpu(oracle):
    """torch's CPU conv2d as an independent check, within K * 2^-24 * sum|x||w|."""
    rng = np.random.default_rng(13)
    N, C, H, W, OC, k = 2, 16, 12, 13, 8, 3
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((OC, C, k, k)).astype(np.float32)
    b = rng.standard_normal(OC).astype(np.float32)
    y = oracle.conv2d_fw_f32(x, w, b, (2, 1), (1, 2))
    t = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                   torch.from_numpy(b).double(), stride=(2, 1),
                                   padding=(1, 2)).numpy()
    mag = torch.nn.functional.conv2d(torch.from_numpy(np.abs(x)).double(),
                                     torch.from_numpy(np.abs(w)).double(), stride=(2, 1),
                                     padding=(1, 2)).numpy() + np.abs(b)[None, :, None, None]
    K = C * k * k + 1
    assert y.shape == t.shape
    assert np.all(np.abs(y - t) <= K * 2.0 ** -24 * mag)
