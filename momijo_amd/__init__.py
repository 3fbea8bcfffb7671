"""momijo_amd: an MI355X (gfx950) backend for momijo's tensor-engine hot path.

Dense matmul / Linear (fp32 and bf16 on MFMA), the int8 weight path
(per-channel quantize/pack, W8A16 GEMV and GEMM, legacy per-tensor W8A8
QuantLinear on int8 MFMA) and the fused bias + activation epilogue, behind
the C ABI declared in include/momijo_hip.h.  The Python classes mirror the
reference's operator surface (Tensor.matmul, Linear, ReLU, QuantLinear, the
int8 helpers of learn/api/functional.mojo).
"""
from ._lib import (EPI_GELU_TANH, EPI_GELU_TANH_APPROX, EPI_NONE, EPI_RELU, EPI_RELU_UNARY,
                   EPI_SILU, EPI_SILU_APPROX, ROUND_LEGACY, ROUND_RHE, MomijoHipError)
from .tensor import (Tensor, empty_f32, empty_f64, gemm_bf16_nt, gpu_available, matmul, matmul2d,
                     matmul_backward, tensordot)
from .nn import (Conv2d, Linear, QuantLinear, ReLU, W8A8Linear, W8Linear, W8MLP, quantize_rowwise_int8,
                 quantize_rows_bf16_int8)
from . import autograd, seam, weights
from .autograd import GradContext, GradTensor
from .functional import (MinMaxObserver, convert, dequantize_i32_scaled, dequantize_i32_to_f32_add_bias,
                         matmul_i8_i8_to_i32, prepare, quantize_symmetric_int8)

__all__ = [
    "Tensor", "matmul", "matmul2d", "matmul_backward", "tensordot", "empty_f32", "empty_f64",
    "gemm_bf16_nt",
    "gpu_available",
    "Linear", "Conv2d", "ReLU", "QuantLinear", "W8Linear", "W8A8Linear", "W8MLP", "quantize_rowwise_int8",
    "quantize_rows_bf16_int8",
    "quantize_symmetric_int8", "matmul_i8_i8_to_i32", "dequantize_i32_to_f32_add_bias",
    "dequantize_i32_scaled",
    "MinMaxObserver", "prepare", "convert", "MomijoHipError", "seam", "weights",
    "autograd", "GradContext", "GradTensor",
    "EPI_NONE", "EPI_RELU", "EPI_GELU_TANH", "EPI_SILU", "EPI_GELU_TANH_APPROX",
    "EPI_SILU_APPROX", "EPI_RELU_UNARY", "ROUND_RHE", "ROUND_LEGACY",
]
