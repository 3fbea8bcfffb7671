"""Layers of momijo's learn.nn on the MI355X backend: Linear, ReLU and
QuantLinear (learn/nn/layers.mojo), plus the per-channel int8 weight-only
Linear and the Llama-style FFN that the backend adds for bf16 activations.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .tensor import Tensor, _device, _ptr, _stream


class Linear:
    """Linear(in_features, out_features, bias) (learn/nn/layers.mojo:343-794).

    ``weight`` is [OutF, InF] fp32, ``bias_t`` [OutF].  ``forward`` is the
    forward_cpu_parallel contract (:383-433): y = x W^T + b with the bias added
    after the dot; a non-2-D input or a width mismatch returns ``x.copy()``.
    ``forward_act`` fuses the activation layer that follows (ReLU, GELU, SiLU).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        self.in_features = in_features
        self.out_features = out_features
        self.bias = bias
        self.weight = Tensor(torch.zeros((out_features, in_features), dtype=torch.float32))
        self.bias_t = Tensor(torch.zeros((out_features if bias else 0,), dtype=torch.float32))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        """All weights 0.01 / in_features, bias 0 (layers.mojo:361-377)."""
        self.weight.torch.fill_(0.01 / self.in_features)
        if self.bias:
            self.bias_t.torch.zero_()

    def _bias_ptr(self):
        b = self.bias_t.torch
        return _ptr(b) if self.bias and b.numel() == self.out_features else None

    def forward_act(self, x: Tensor, epi: int) -> Tensor:
        xt = x.torch
        if xt.dim() != 2 or xt.shape[1] != self.in_features:
            return x.copy()
        if xt.dtype != torch.float32:
            raise TypeError("Linear takes Float32 inputs")
        xt = xt.contiguous()
        N = xt.shape[0]
        y = torch.empty((N, self.out_features), dtype=torch.float32, device=xt.device)
        _lib.call("mj_linear_f32", _ptr(xt), _ptr(self.weight.torch), self._bias_ptr(), epi,
                  _ptr(y), N, self.in_features, self.out_features, _stream())
        return Tensor(y)

    def forward(self, x: Tensor) -> Tensor:
        """Linear.forward -> forward_auto (layers.mojo:510-516)."""
        return self.forward_act(x, _lib.EPI_NONE)

    forward_auto = forward
    forward_gpu = forward

    def backward(self, x: Tensor, dy: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """Linear.backward -> backward_auto (layers.mojo:519-618, 779-787).

        Returns (dW [OutF, InF], db [OutF], dx [N, InF]) with dW = dy^T x,
        db = column sums of dy, dx = dy W.  Non-2-D operands, a row-count
        mismatch or wrong widths return zeros shaped like (weight, bias_t, x),
        as the reference does."""
        xt, gt = x.torch, dy.torch
        if (xt.dim() != 2 or gt.dim() != 2 or xt.shape[0] != gt.shape[0]
                or xt.shape[1] != self.in_features or gt.shape[1] != self.out_features):
            return (Tensor(torch.zeros_like(self.weight.torch)),
                    Tensor(torch.zeros_like(self.bias_t.torch)), Tensor(torch.zeros_like(xt)))
        if xt.dtype != torch.float32 or gt.dtype != torch.float32:
            raise TypeError("Linear takes Float32 inputs")
        xt, gt = xt.contiguous(), gt.contiguous()
        w = self.weight.torch.contiguous()
        N = xt.shape[0]
        dW = torch.empty((self.out_features, self.in_features), dtype=torch.float32,
                         device=xt.device)
        db = torch.empty(self.out_features, dtype=torch.float32, device=xt.device)
        dx = torch.empty_like(xt)
        _lib.call("mj_linear_backward_f32", _ptr(xt), _ptr(w), _ptr(gt), _ptr(dW), _ptr(db),
                  _ptr(dx), N, self.in_features, self.out_features, _stream())
        return Tensor(dW), Tensor(db), Tensor(dx)

    backward_auto = backward
    backward_gpu = backward


class Conv2d:
    """Conv2d(in_channels, out_channels, kernel, stride, pad, bias)
    (learn/nn/conv.mojo:443-476): weight [OC, C, kH, kW] fp32, bias_t [OC].

    ``forward`` is Conv2d.forward / forward_auto / forward_gpu
    (:494-597, 600-697): NCHW, zero padding, OH = (H + 2 pH - kH) // sH + 1,
    the bias added after the sum, computed as one implicit GEMM per image
    on the fp32 matrix cores (``mj_conv2d_f32``).  The weights are
    initialised as the reference does in distribution (He normal,
    N(0, 1) * sqrt(2 / fan_in), bias zero), from torch's device generator:
    the reference's global RNG stream is not reproduced; callers that need
    given weights assign ``weight`` / ``bias_t``.  An input whose channel
    count differs from the weight's is refused (the reference would read
    past the weight)."""

    def __init__(self, in_channels: int, out_channels: int, kernel, stride=(1, 1),
                 pad=(0, 0), bias: bool = True):
        kH, kW = kernel
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_h, self.kernel_w = int(kH), int(kW)
        self.stride_h, self.stride_w = (int(v) for v in stride)
        self.pad_h, self.pad_w = (int(v) for v in pad)
        if min(self.kernel_h, self.kernel_w, self.stride_h, self.stride_w) < 1 or \
                min(self.pad_h, self.pad_w) < 0:
            raise ValueError("kernel and stride must be >= 1, padding >= 0")
        self.bias = bias
        fan_in = in_channels * self.kernel_h * self.kernel_w
        dev = _device()
        w = torch.randn((out_channels, in_channels, self.kernel_h, self.kernel_w),
                        dtype=torch.float32, device=dev)
        self.weight = Tensor(w * np.float32(np.sqrt(2.0 / max(fan_in, 1))))
        self.bias_t = Tensor(torch.zeros((out_channels if bias else 0,), dtype=torch.float32,
                                         device=dev))

    def out_size(self, H: int, W: int) -> tuple[int, int]:
        """(OH, OW) with floor division (conv.mojo:496-497)."""
        return ((H + 2 * self.pad_h - self.kernel_h) // self.stride_h + 1,
                (W + 2 * self.pad_w - self.kernel_w) // self.stride_w + 1)

    def forward_act(self, x: Tensor, epi: int) -> Tensor:
        xt = x.torch
        if xt.dim() != 4 or xt.shape[1] != self.in_channels:
            raise ValueError(f"Conv2d({self.in_channels}, ...) takes [N, {self.in_channels}, H, W], "
                             f"got {list(xt.shape)}")
        if xt.dtype != torch.float32:
            raise TypeError("Conv2d takes Float32 inputs")
        xt = xt.contiguous()
        N, C, H, W = xt.shape
        OH, OW = self.out_size(H, W)
        w = self.weight.torch.contiguous()
        if tuple(w.shape) != (self.out_channels, C, self.kernel_h, self.kernel_w):
            raise ValueError(f"weight must be [{self.out_channels}, {C}, {self.kernel_h}, "
                             f"{self.kernel_w}], got {list(w.shape)}")
        y = torch.empty((N, self.out_channels, max(OH, 0), max(OW, 0)), dtype=torch.float32,
                        device=xt.device)
        if y.numel() == 0:
            return Tensor(y)
        b = self.bias_t.torch
        bptr = _ptr(b) if self.bias and b.numel() == self.out_channels else None
        _lib.call("mj_conv2d_f32", _ptr(xt), _ptr(w), bptr, epi, _ptr(y), N, C, H, W,
                  self.out_channels, self.kernel_h, self.kernel_w, self.stride_h, self.stride_w,
                  self.pad_h, self.pad_w, _stream())
        return Tensor(y)

    def forward(self, x: Tensor) -> Tensor:
        """Conv2d.forward -> forward_auto (conv.mojo:697-708)."""
        return self.forward_act(x, _lib.EPI_NONE)

    forward_auto = forward
    forward_gpu = forward


class ReLU:
    """ReLU.forward = layers.mojo's own _maximum_scalar(x, 0): v > 0 ? v : 0
    (layers.mojo:117-137), so -0 and NaN give +0 -- unlike
    Tensor.maximum_scalar(0), which keeps -0."""

    def forward(self, x: Tensor) -> Tensor:
        return x._unary(_lib.EPI_RELU)


class QuantLinear:
    """QuantLinear (learn/nn/layers.mojo:1663-1703): per-tensor W8A8.

    forward = quantize_symmetric_int8(x, s_x) -> int8 GEMM against w_q^T ->
    float(acc) * (s_x*s_w) + b, in one quantize launch and one int8-MFMA GEMM
    with the dequantize fused.  ``legacy_literal=True`` reproduces the
    reference's stride-ignoring read of w_q.transpose() (functional.mojo:274).
    """

    def __init__(self, in_features: int, out_features: int, w_q: Tensor, b_f: Tensor,
                 s_w: float, s_x: float, legacy_literal: bool = False):
        self.in_features = in_features
        self.out_features = out_features
        wq, bf = w_q.torch, b_f.torch
        # the kernels read w_q [out, in] and b_f [out] in full: wrong shapes
        # would read past the allocations (the reference indexes them
        # unchecked, layers.mojo:1681-1685, functional.mojo:281-302)
        if wq.dtype != torch.int8 or tuple(wq.shape) != (out_features, in_features):
            raise ValueError(f"w_q must be int8 [{out_features}, {in_features}], "
                             f"got {wq.dtype} {list(wq.shape)}")
        if bf.dtype != torch.float32 or bf.numel() != out_features:
            raise ValueError(f"b_f must be float32 with {out_features} elements, "
                             f"got {bf.dtype} with {bf.numel()}")
        self.w_q = Tensor(wq.contiguous())
        self.b_f = Tensor(bf.reshape(-1).contiguous())
        self.s_w = float(np.float32(s_w))
        self.s_x = float(np.float32(s_x))
        self.legacy_literal = legacy_literal

    def forward(self, x: Tensor) -> Tensor:
        """A non-2-D x or a width other than in_features gives the reference's
        empty [0, 0] result (matmul_i8_i8_to_i32 returns [0, 0] and
        dequantize_i32_to_f32_add_bias keeps it, functional.mojo:253-263,
        291-292)."""
        xt = x.torch
        if xt.dim() != 2 or xt.shape[1] != self.in_features:
            return Tensor(torch.zeros((0, 0), dtype=torch.float32, device=_device()))
        if xt.dtype != torch.float32:
            raise TypeError("QuantLinear takes Float32 inputs")
        xt = xt.contiguous()
        M, K = xt.shape
        N = self.out_features
        y = torch.empty((M, N), dtype=torch.float32, device=xt.device)
        _lib.call("mj_quant_linear_f32", _ptr(xt), _ptr(self.w_q.torch), _ptr(self.b_f.torch),
                  self.s_w, self.s_x, _ptr(y), M, N, K, int(self.legacy_literal), _stream())
        return Tensor(y)


class W8Linear:
    """Weight-only int8 Linear with bf16 activations (per-output-channel,
    round-half-even scales).  No reference counterpart: it is the
    per-channel generalisation of QuantLinear's weights, applied to the
    reference's Linear layout [OutF, InF].

    y = bf16(epi((x . q^T) * scale[n] + bias[n])); M <= 16 rows (M <= 48
    when K is a multiple of 1024 up to 4096) take the GEMV kernels (K-split
    streaming for M <= 2 and for 3-4 rows at other K, skinny MFMA otherwise),
    more rows the MFMA GEMM."""

    def __init__(self, q: torch.Tensor, scales: torch.Tensor, bias: torch.Tensor | None = None,
                 epi: int = _lib.EPI_NONE):
        if q.dtype != torch.int8 or q.dim() != 2:
            raise ValueError(f"q must be a 2-D int8 tensor, got {q.dtype} {list(q.shape)}")
        self.q = q.contiguous()
        self.out_features, self.in_features = self.q.shape
        if scales.dtype != torch.float32 or scales.numel() != self.out_features:
            raise ValueError(f"scales must be float32 with {self.out_features} elements")
        if bias is not None and bias.numel() != self.out_features:
            raise ValueError(f"bias must have {self.out_features} elements")
        self.scales = scales.reshape(-1).contiguous()
        self.bias = None if bias is None else bias.float().reshape(-1).contiguous()
        self.epi = epi

    @classmethod
    def from_float(cls, W: torch.Tensor, bias: torch.Tensor | None = None,
                   epi: int = _lib.EPI_NONE, rounding: int = _lib.ROUND_RHE) -> "W8Linear":
        q, s = quantize_rowwise_int8(W, rounding)
        return cls(q, s, bias, epi)

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        M, K = _check_bf16_rows(x, self.in_features, "x")
        if out is None:
            out = torch.empty((M, self.out_features), dtype=torch.bfloat16, device=x.device)
        _check_bf16_out(out, (M, self.out_features), "out")
        _lib.call("mj_linear_w8a16", _ptr(x), _ptr(self.q), _ptr(self.scales), _ptr(self.bias),
                  self.epi, _ptr(out), M, self.out_features, K, _stream())
        return out


class W8A8Linear(W8Linear):
    """W8Linear's weights with the activations quantized too: each row of x
    gets its own int8 scale (max|row| / 127, round half to even) at call
    time, the product runs on int8 MFMA with exact int32 sums, and the
    epilogue applies both scales:
    y = bf16(epi(float(xq . q^T) * (sx[m] * scale[n]) + bias[n])).
    The per-row / per-channel form of QuantLinear.forward
    (learn/nn/layers.mojo:1681-1685).  For prefill-sized M; decode (M = 1)
    is faster on W8Linear, whose GEMV reads the weights once at HBM rate."""

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        M, K = _check_bf16_rows(x, self.in_features, "x")
        if out is None:
            out = torch.empty((M, self.out_features), dtype=torch.bfloat16, device=x.device)
        _check_bf16_out(out, (M, self.out_features), "out")
        _lib.call("mj_linear_w8a8", _ptr(x), _ptr(self.q), _ptr(self.scales), _ptr(self.bias),
                  self.epi, _ptr(out), M, self.out_features, K, _stream())
        return out


class W8MLP:
    """Llama-style FFN: y = ((silu(x Wg^T) * (x Wu^T)) Wd^T) on W8A16 weights.
    The gate and up projections run as one GEMM whose epilogue forms
    silu(g) * u; the down projection is a second W8A16 GEMM."""

    def __init__(self, gate: W8Linear, up: W8Linear, down: W8Linear):
        # the C ABI reads Wu with Wg's shape and Wd as [H, I]: a mismatch
        # would read past the weights, so it is refused here
        if tuple(gate.q.shape) != tuple(up.q.shape):
            raise ValueError(f"gate and up weights differ in shape: {list(gate.q.shape)} vs "
                             f"{list(up.q.shape)}")
        if down.in_features != gate.out_features:
            raise ValueError(f"down takes {down.in_features} features, gate/up give "
                             f"{gate.out_features}")
        for name, lin in (("gate", gate), ("up", up), ("down", down)):
            if lin.scales.dtype != torch.float32 or lin.scales.numel() != lin.out_features:
                raise ValueError(f"{name} scales must be float32 with {lin.out_features} elements")
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x: torch.Tensor, h: torch.Tensor | None = None,
                out: torch.Tensor | None = None):
        M, K = _check_bf16_rows(x, self.gate.in_features, "x")
        I = self.gate.out_features
        H = self.down.out_features
        if h is None:
            h = torch.empty((M, I), dtype=torch.bfloat16, device=x.device)
        if out is None:
            out = torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
        _check_bf16_out(h, (M, I), "h")
        _check_bf16_out(out, (M, H), "out")
        _lib.call("mj_mlp_w8a16", _ptr(x), _ptr(self.gate.q), _ptr(self.gate.scales),
                  _ptr(self.up.q), _ptr(self.up.scales), _ptr(self.down.q),
                  _ptr(self.down.scales), _ptr(h), _ptr(out), M, K, I, H, _stream())
        return out, h


def _check_bf16_rows(x: torch.Tensor, K: int, name: str) -> tuple[int, int]:
    """x must be a contiguous bfloat16 [M, K] device tensor: the C ABI takes
    its leading dimension as K."""
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {x.dtype}")
    if x.dim() != 2 or x.shape[1] != K:
        raise ValueError(f"{name} must be [M, {K}], got {list(x.shape)}")
    if not x.is_contiguous():
        raise ValueError(f"{name} must be contiguous (row stride == {K})")
    return int(x.shape[0]), K


def _check_bf16_out(t: torch.Tensor, shape: tuple, name: str) -> None:
    if t.dtype != torch.bfloat16 or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bfloat16 {list(shape)} tensor, got "
                         f"{t.dtype} {list(t.shape)}")


def quantize_rowwise_int8(W: torch.Tensor, rounding: int = _lib.ROUND_RHE):
    """Per-output-channel symmetric int8 quantize/pack of W [N,K] fp32 on the
    device; returns (q int8 [N,K], scales fp32 [N])."""
    W = W.float().contiguous()
    N, K = W.shape
    q = torch.empty((N, K), dtype=torch.int8, device=W.device)
    s = torch.empty((N,), dtype=torch.float32, device=W.device)
    _lib.call("mj_quantize_rowwise_i8", _ptr(W), N, K, rounding, _ptr(q), _ptr(s), _stream())
    return q, s


def quantize_rows_bf16_int8(x: torch.Tensor):
    """Per-row dynamic int8 quantize of a contiguous bf16 [M, K] device
    tensor (the activation half of W8A8Linear); returns (xq int8 [M, K],
    sx fp32 [M])."""
    if x.dtype != torch.bfloat16 or x.dim() != 2 or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous 2-D bfloat16 tensor, got {x.dtype} {list(x.shape)}")
    M, K = x.shape
    xq = torch.empty((M, K), dtype=torch.int8, device=x.device)
    sx = torch.empty((M,), dtype=torch.float32, device=x.device)
    _lib.call("mj_quantize_rows_bf16_i8", _ptr(x), M, K, _ptr(xq), _ptr(sx), _stream())
    return xq, sx


__all__ = ["Linear", "Conv2d", "ReLU", "QuantLinear", "W8Linear", "W8A8Linear", "W8MLP",
           "quantize_rowwise_int8", "quantize_rows_bf16_int8", "_device"]
