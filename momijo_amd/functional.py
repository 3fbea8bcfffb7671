"""The int8 helpers of momijo's PTQ path (learn/api/functional.mojo:206-302)
and the MinMax observer / convert flow (learn/api/sequential.mojo:217-459),
on the MI355X backend."""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .nn import Linear, QuantLinear, ReLU
from .tensor import Tensor, _ptr, _stream


def quantize_symmetric_int8(x: Tensor, s: float) -> Tensor:
    """quantize_symmetric_int8 (functional.mojo:231-247): q = clamp(trunc(x/s
    +- 0.5)) with a per-tensor scale; s == 0 is replaced by 1."""
    xt = x.torch.contiguous()
    q = torch.empty(xt.shape, dtype=torch.int8, device=xt.device)
    _lib.call("mj_quantize_symmetric_int8", _ptr(xt), xt.numel(), float(np.float32(s)), _ptr(q),
              _stream())
    return Tensor(q)


def matmul_i8_i8_to_i32(a: Tensor, bt: Tensor, legacy_literal: bool = False) -> Tensor:
    """matmul_i8_i8_to_i32 (functional.mojo:249-279).

    ``bt`` is the [K, N] operand.  When it is the transpose view of a
    row-major w_q [N, K] (what QuantLinear passes), the product is
    a @ w_q^T on int8 MFMA.  ``legacy_literal=True`` reproduces the
    reference's read of bt._data[p*N + j] that ignores the view's strides.
    Non-2-D operands or a K mismatch return a [0, 0] tensor as the reference
    does (:253-263)."""
    at, bt_t = a.torch, bt.torch
    if at.dim() != 2 or bt_t.dim() != 2 or at.shape[1] != bt_t.shape[0]:
        return Tensor(torch.zeros((0, 0), dtype=torch.int32, device=at.device))
    M, K = at.shape
    N = bt_t.shape[1]
    at = at.contiguous()
    if legacy_literal:
        # the flat storage of the view's base, read as [K, N]
        w = bt_t.transpose(0, 1).contiguous() if bt_t.stride(0) == 1 else bt_t.contiguous()
    else:
        w = bt_t.transpose(0, 1).contiguous()  # [N, K]
    c = torch.empty((M, N), dtype=torch.int32, device=at.device)
    _lib.call("mj_matmul_i8_i8_to_i32", _ptr(at), _ptr(w), _ptr(c), M, N, K, int(legacy_literal),
              _stream())
    return Tensor(c)


def dequantize_i32_to_f32_add_bias(y_i32: Tensor, sf: float, b: Tensor) -> Tensor:
    """dequantize_i32_to_f32_add_bias (functional.mojo:281-302)."""
    yt = y_i32.torch.contiguous()
    if yt.dim() != 2:
        return Tensor(torch.zeros((0, 0), dtype=torch.float32, device=yt.device))
    M, N = yt.shape
    out = torch.empty((M, N), dtype=torch.float32, device=yt.device)
    _lib.call("mj_dequantize_i32_to_f32_add_bias", _ptr(yt), float(np.float32(sf)),
              _ptr(b.torch.contiguous()), _ptr(out), M, N, _stream())
    return Tensor(out)


def dequantize_i32_scaled(y_i32: Tensor, sw: Tensor, b: Tensor | None = None,
                          sx: Tensor | None = None) -> Tensor:
    """Per-channel form of dequantize_i32_to_f32_add_bias (functional.mojo:
    281-302): y[m, n] = float(acc[m, n]) * (sx[m] * sw[n]) + b[n], rounded
    step by step; sx (per-row scales) and b are optional."""
    yt = y_i32.torch.contiguous()
    if yt.dim() != 2 or yt.dtype != torch.int32:
        raise ValueError(f"acc must be a 2-D int32 tensor, got {yt.dtype} {list(yt.shape)}")
    M, N = yt.shape
    swt = sw.torch.reshape(-1).contiguous()
    if swt.dtype != torch.float32 or swt.numel() != N:
        raise ValueError(f"sw must be float32 with {N} elements")
    bt = None if b is None else b.torch.reshape(-1).contiguous()
    if bt is not None and (bt.dtype != torch.float32 or bt.numel() != N):
        raise ValueError(f"b must be float32 with {N} elements")
    sxt = None if sx is None else sx.torch.reshape(-1).contiguous()
    if sxt is not None and (sxt.dtype != torch.float32 or sxt.numel() != M):
        raise ValueError(f"sx must be float32 with {M} elements")
    out = torch.empty((M, N), dtype=torch.float32, device=yt.device)
    _lib.call("mj_dequantize_i32_scaled_f32", _ptr(yt), _ptr(sxt), _ptr(swt), _ptr(bt),
              _ptr(out), M, N, _stream())
    return Tensor(out)


class MinMaxObserver:
    """MinMaxObserver (sequential.mojo:217-263): running min/max, symmetric
    scale = max(|min|,|max|) / max_q (1.0 without data or for a zero range)."""

    def __init__(self):
        self.has_data = False
        self.min_v = 0.0
        self.max_v = 0.0

    def observe(self, x: Tensor) -> None:
        t = x.torch.contiguous()
        if t.numel() == 0:
            return
        mm = torch.empty((2,), dtype=torch.float32, device=t.device)
        _lib.call("mj_minmax_f32", _ptr(t), t.numel(), _ptr(mm), _stream())
        mn, mx = (float(v) for v in mm.cpu())
        if not self.has_data:
            self.min_v, self.max_v, self.has_data = mn, mx, True
        else:
            self.min_v = min(self.min_v, mn)
            self.max_v = max(self.max_v, mx)

    def scale_symmetric(self, max_q: float = 127.0) -> float:
        if not self.has_data or max_q <= 0.0:
            return 1.0
        f = np.float32
        m = max(abs(f(self.min_v)), abs(f(self.max_v)))
        if m <= 0.0:
            return 1.0
        return float(f(m) / f(max_q))


def scale_symmetric_device(x: Tensor, max_q: float = 127.0) -> float:
    """One-shot MinMax scale of a device tensor, reduced on the GPU."""
    t = x.torch.contiguous()
    out = torch.empty((1,), dtype=torch.float32, device=t.device)
    _lib.call("mj_minmax_scale_symmetric", _ptr(t), t.numel(), float(max_q), _ptr(out), _stream())
    return float(out.item())


class Prepared:
    """Prepared (sequential.mojo:383-411): Linear -> ReLU -> Linear with
    observers on the input, the ReLU output and both weights."""

    def __init__(self, l1: Linear, relu: ReLU, l2: Linear):
        self.l1, self.relu, self.l2 = l1, relu, l2
        self.obs_in, self.obs_relu = MinMaxObserver(), MinMaxObserver()
        self.obs_w1, self.obs_w2 = MinMaxObserver(), MinMaxObserver()

    def forward(self, x: Tensor) -> Tensor:
        self.obs_in.observe(x)
        y1 = self.l1.forward(x)
        y2 = self.relu.forward(y1)
        self.obs_relu.observe(y2)
        self.obs_w1.observe(self.l1.weight)
        self.obs_w2.observe(self.l2.weight)
        return self.l2.forward(y2)


class Converted:
    """Converted (sequential.mojo:413-425): q1 -> float ReLU -> q2."""

    def __init__(self, q1: QuantLinear, q2: QuantLinear):
        self.q1, self.q2 = q1, q2

    def forward(self, x: Tensor) -> Tensor:
        y1 = self.q1.forward(x)
        y2 = y1.maximum_scalar(0.0)
        return self.q2.forward(y2)


def prepare(l1: Linear, relu: ReLU, l2: Linear) -> Prepared:
    """prepare (sequential.mojo:428-433) for the [Linear, ReLU, Linear] pattern."""
    return Prepared(l1, relu, l2)


def convert(p: Prepared, legacy_literal: bool = False) -> Converted:
    """convert (sequential.mojo:436-450): per-tensor symmetric scales from the
    observers, weights quantized with quantize_symmetric_int8."""
    s_in = p.obs_in.scale_symmetric(127.0)
    s_relu = p.obs_relu.scale_symmetric(127.0)
    s_w1 = p.obs_w1.scale_symmetric(127.0)
    s_w2 = p.obs_w2.scale_symmetric(127.0)
    w1_q = quantize_symmetric_int8(p.l1.weight, s_w1)
    w2_q = quantize_symmetric_int8(p.l2.weight, s_w2)
    q1 = QuantLinear(p.l1.in_features, p.l1.out_features, w1_q, p.l1.bias_t, s_w1, s_in,
                     legacy_literal)
    q2 = QuantLinear(p.l2.in_features, p.l2.out_features, w2_q, p.l2.bias_t, s_w2, s_relu,
                     legacy_literal)
    return Converted(q1, q2)
