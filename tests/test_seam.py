"""The seam contract of momijo_amd.seam on the CPU (no GPU needed): with no
gfx950 device, or with the device call forced to a non-OK status, each
launcher runs the caller's kernel for every thread id in blocks of
block_size, as the reference's launchers do (tensor/gpu/runtime.mojo:
608-631), and the result is the oracle's; strict mode raises instead.

The kernels below are the test's restatements of the reference's CPU kernels
(learn/nn/layers.mojo:436-475, 624-729): strict ascending order with one
float32 rounding per operation.  The forward is checked bit for bit against
the oracle's _kernel_linear_fw on random inputs; the backward ones on
integer-valued inputs, whose sums are exact in any order.
"""
import numpy as np
import pytest

from momijo_amd import _lib, seam

f32 = np.float32


def k_linear_fw(tid, x, wT, b, y, N, InF, OutF, has_bias):
    if tid >= N * OutF:
        return
    n, o = divmod(tid, OutF)
    acc = f32(0)
    for k in range(InF):
        acc = f32(acc + f32(f32(x[n * InF + k]) * f32(wT[k * OutF + o])))
    if has_bias and len(b) == OutF:
        acc = f32(acc + f32(b[o]))
    y[n * OutF + o] = acc


def k_bw_dx(tid, dy, w, dx, N, InF, OutF):
    if N * InF <= 0 or tid >= N * InF:
        return
    n, i = divmod(tid, InF)
    acc = f32(0)
    for o in range(OutF):
        acc = f32(acc + f32(f32(dy[n * OutF + o]) * f32(w[o * InF + i])))
    dx[n * InF + i] = acc


def k_bw_dw(tid, dy, x, dW, N, InF, OutF):
    if OutF * InF <= 0 or tid >= OutF * InF:
        return
    o, i = divmod(tid, InF)
    acc = f32(0)
    for n in range(N):
        acc = f32(acc + f32(f32(dy[n * OutF + o]) * f32(x[n * InF + i])))
    dW[o * InF + i] = acc


def k_bw_db(tid, dy, db, N, OutF):
    if tid >= OutF:
        return
    acc = f32(0)
    for n in range(N):
        acc = f32(acc + f32(dy[n * OutF + tid]))
    db[tid] = acc


def k_conv2d_fw(tid, x, w, b, y, N, C, H, W, OH, OW, OC, kH, kW, sH, sW, pH, pW, has_bias):
    """The reference's _kernel_conv2d_fwd (learn/nn/conv.mojo:600-681)."""
    if tid >= N * OC * OH * OW:
        return
    n, r = divmod(tid, OC * OH * OW)
    oc, r = divmod(r, OH * OW)
    oy, ox = divmod(r, OW)
    iy0, ix0 = oy * sH - pH, ox * sW - pW
    ky0, ky1 = max(0, -iy0), kH - max(0, iy0 + kH - H)
    kx0, kx1 = max(0, -ix0), kW - max(0, ix0 + kW - W)
    acc = f32(0)
    for ic in range(C):
        for ky in range(ky0, ky1):
            for kx in range(kx0, kx1):
                xv = f32(x[((n * C + ic) * H + iy0 + ky) * W + ix0 + kx])
                wv = f32(w[((oc * C + ic) * kH + ky) * kW + kx])
                acc = f32(acc + f32(xv * wv))
    if has_bias:
        acc = f32(acc + f32(b[oc]))
    y[tid] = acc


class _FailingLib:
    """Stands in for the loaded library: a device is reported, and every
    host-pointer launch returns MJ_ERR_DEVICE."""

    def __init__(self):
        self.calls = []

    def mj_device_available(self):
        return 1

    def mj_last_error(self):
        return b"forced device failure"

    def __getattr__(self, name):
        if name.startswith("mj_launch_"):
            def launch(*args):
                self.calls.append(name)
                return _lib.MJ_ERR_DEVICE
            return launch
        raise AttributeError(name)


@pytest.fixture(params=["forced_error", "no_device"])
def mode(request, monkeypatch):
    if request.param == "forced_error":
        fake = _FailingLib()
        monkeypatch.setattr(_lib, "load", lambda: fake)
        return fake
    lib = _lib.load()
    if lib.mj_device_available():
        pytest.skip("a gfx950 device is present: the no-device path is not reachable here")
    return None


def _counted(kernel, seen):
    def k(tid, *args):
        seen.append(tid)
        kernel(tid, *args)
    return k


def test_linear_fw_falls_back_to_kernel(oracle, mode):
    N, InF, OutF = 3, 21, 5
    x = oracle.randn_f32((N, InF), seed=1).reshape(-1)
    W = oracle.randn_f32((OutF, InF), seed=2)
    wT = np.ascontiguousarray(W.T).reshape(-1)
    b = oracle.randu_f32((OutF,), -1 / 16, 1 / 16, seed=3)
    y = np.zeros(N * OutF, np.float32)
    seen = []
    path = seam.launch_1d_linear_fw(N * OutF, 4, _counted(k_linear_fw, seen), x, wT, b, y,
                                    N, InF, OutF, True)
    assert path == "cpu"
    assert seen == list(range(N * OutF))       # every tid once, in block order
    ref = oracle.kernel_linear_fw_f32(x.reshape(N, InF), wT.reshape(InF, OutF), b)
    np.testing.assert_array_equal(y.reshape(N, OutF), ref)
    if mode is not None:
        assert mode.calls == ["mj_launch_linear_fw_h"]   # the device call was tried first
    # a bias of the wrong length is ignored, as the CPU kernel's guard does
    y2 = np.zeros(N * OutF, np.float32)
    seam.launch_1d_linear_fw(N * OutF, 0, k_linear_fw, x, wT, b[:3], y2, N, InF, OutF, True)
    np.testing.assert_array_equal(
        y2.reshape(N, OutF), oracle.kernel_linear_fw_f32(x.reshape(N, InF), wT.reshape(InF, OutF)))


def test_block_size_and_total_threads(mode):
    seen = []
    y = np.zeros(6, np.float32)
    z = np.zeros(9, np.float32)
    # block_size <= 0 means 256; tids stop at total_threads even inside a block
    seam.launch_1d_linear_fw(5, 0, lambda tid, *a: seen.append(tid), z, z, z, y, 2, 3, 3, False)
    assert seen == [0, 1, 2, 3, 4]
    seen.clear()
    seam.launch_1d_linear_fw(0, 8, lambda tid, *a: seen.append(tid), z, z, z, y, 2, 3, 3, False)
    assert seen == []


def test_backward_seams_fall_back(oracle, mode):
    rng = np.random.default_rng(5)
    N, InF, OutF = 4, 6, 9
    x = rng.integers(-4, 5, size=(N, InF)).astype(np.float32)
    W = rng.integers(-4, 5, size=(OutF, InF)).astype(np.float32)
    dy = rng.integers(-4, 5, size=(N, OutF)).astype(np.float32)
    dW_ref, db_ref, dx_ref = oracle.linear_backward_f32(x, W, dy)
    dx = np.zeros(N * InF, np.float32)
    dW = np.zeros(OutF * InF, np.float32)
    db = np.zeros(OutF, np.float32)
    assert seam.launch_1d_linear_bw_dx(N * InF, 16, k_bw_dx, dy.reshape(-1), W.reshape(-1), dx,
                                       N, InF, OutF) == "cpu"
    assert seam.launch_1d_linear_bw_dw(OutF * InF, 16, k_bw_dw, dy.reshape(-1), x.reshape(-1),
                                       dW, N, InF, OutF) == "cpu"
    assert seam.launch_1d_linear_bw_db(OutF, 16, k_bw_db, dy.reshape(-1), db, N, OutF) == "cpu"
    np.testing.assert_array_equal(dx.reshape(N, InF), dx_ref)
    np.testing.assert_array_equal(dW.reshape(OutF, InF), dW_ref)
    np.testing.assert_array_equal(db, db_ref)


def test_strict_mode_raises(mode):
    z = np.zeros(4, np.float32)
    with pytest.raises(_lib.MomijoHipError) as e:
        seam.launch_1d_linear_fw(4, 4, k_linear_fw, z, z, z, z.copy(), 2, 2, 2, False, strict=True)
    assert e.value.status in (_lib.MJ_ERR_DEVICE, _lib.MJ_ERR_NO_DEVICE)


def test_output_buffer_must_be_writable_float32(mode):
    z = np.zeros(4, np.float32)
    with pytest.raises(TypeError):
        seam.launch_1d_linear_fw(4, 4, k_linear_fw, z, z, z, [0.0] * 4, 2, 2, 2, False)
    with pytest.raises(ValueError):
        seam.launch_1d_linear_fw(4, 4, k_linear_fw, z[:3], z, z, z.copy(), 2, 2, 2, False)


def test_conv2d_fw_falls_back_to_kernel(oracle, mode):
    N, C, H, W, OC, kH, kW, sH, sW, pH, pW = 2, 3, 6, 5, 4, 3, 3, 2, 1, 1, 1
    x = oracle.randn_f32((N, C, H, W), seed=31)
    w = oracle.randn_f32((OC, C, kH, kW), seed=32)
    b = oracle.randu_f32((OC,), -1 / 16, 1 / 16, seed=33)
    OH, OW = oracle.conv_out_size(H, kH, sH, pH), oracle.conv_out_size(W, kW, sW, pW)
    y = np.zeros(N * OC * OH * OW, np.float32)
    seen = []
    path = seam.launch_1d_conv2d_fw(N * OC * OH * OW, 16, _counted(k_conv2d_fw, seen),
                                    x.reshape(-1), w.reshape(-1), b, y, N, C, H, W, OH, OW, OC,
                                    kH, kW, sH, sW, pH, pW, True)
    assert path == "cpu"
    assert seen == list(range(N * OC * OH * OW))
    np.testing.assert_array_equal(y.reshape(N, OC, OH, OW),
                                  oracle.conv2d_fw_f32(x, w, b, (sH, sW), (pH, pW)))
    if mode is not None:
        assert mode.calls == ["mj_launch_conv2d_fw_h"]
