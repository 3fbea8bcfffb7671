"""ctypes binding of ``libmomijo_hip.so`` (the C ABI in include/momijo_hip.h).

The library is loaded from this package directory only; there is no CPU
fallback: if the library or a gfx950 device is missing, the ops raise.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmomijo_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "momijo_hip.h")

# status codes / enums (mirrors of the #defines in the header)
MJ_OK, MJ_ERR_ARG, MJ_ERR_SHAPE, MJ_ERR_UNSUPPORTED, MJ_ERR_DEVICE, MJ_ERR_NO_DEVICE, MJ_ERR_ALLOC = range(7)
EPI_NONE, EPI_RELU, EPI_GELU_TANH, EPI_SILU, EPI_GELU_TANH_APPROX, EPI_SILU_APPROX, EPI_RELU_UNARY = range(7)
ROUND_RHE, ROUND_LEGACY = 0, 1

_STATUS_NAMES = {
    MJ_ERR_ARG: "invalid argument",
    MJ_ERR_SHAPE: "shape mismatch",
    MJ_ERR_UNSUPPORTED: "unsupported layout",
    MJ_ERR_DEVICE: "device error",
    MJ_ERR_NO_DEVICE: "no device",
    MJ_ERR_ALLOC: "allocation failed",
}


class MomijoHipError(RuntimeError):
    def __init__(self, status: int, fn: str, msg: str):
        super().__init__(f"{fn}: {_STATUS_NAMES.get(status, status)} ({msg})")
        self.status = status


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float

# name -> (restype, argtypes); kept in the order of the header
SIGNATURES = {
    "mj_version": (_I32, []),
    "mj_device_available": (_I32, []),
    "mj_last_error": (ctypes.c_char_p, []),
    "mj_stream_synchronize": (_I32, [_P]),
    "mj_matmul_f32": (_I32, [_I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _I64, _P]),
    "mj_matvec_f32": (_I32, [_I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P]),
    "mj_matmul_f64": (_I32, [_I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "mj_matvec_f64": (_I32, [_I64, _I64, _P, _I64, _I64, _P, _I64, _P, _P]),
    "mj_tensordot_f32": (_I32, [_I32, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                _P, _P]),
    "mj_linear_f32": (_I32, [_P, _P, _P, _I32, _P, _I64, _I64, _I64, _P]),
    "mj_launch_linear_fw_h": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I32]),
    "mj_linear_backward_f32": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "mj_launch_linear_bw_dx_h": (_I32, [_P, _P, _P, _I64, _I64, _I64]),
    "mj_launch_linear_bw_dw_h": (_I32, [_P, _P, _P, _I64, _I64, _I64]),
    "mj_launch_linear_bw_db_h": (_I32, [_P, _P, _I64, _I64]),
    "mj_matmul_backward_f64": (_I32, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _I32, _P]),
    "mj_matmul_backward_f32": (_I32, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _I32, _P]),
    "mj_activation_f32": (_I32, [_I32, _P, _P, _I64, _P]),
    "mj_conv2d_f32": (_I32, [_P, _P, _P, _I32, _P] + [_I64] * 11 + [_P]),
    "mj_launch_conv2d_fw_h": (_I32, [_P, _P, _P, _P] + [_I64] * 13 + [_I32]),
    "mj_maximum_scalar_f32": (_I32, [_P, _F, _P, _I64, _P]),
    "mj_cast_i64_f32": (_I32, [_P, _P, _I64, _P]),
    "mj_gemm_bf16_nt": (_I32, [_I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I32, _P, _I64, _P]),
    "mj_quantize_symmetric_int8": (_I32, [_P, _I64, _F, _P, _P]),
    "mj_minmax_f32": (_I32, [_P, _I64, _P, _P]),
    "mj_minmax_scale_symmetric": (_I32, [_P, _I64, _F, _P, _P]),
    "mj_matmul_i8_i8_to_i32": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I32, _P]),
    "mj_dequantize_i32_to_f32_add_bias": (_I32, [_P, _F, _P, _P, _I64, _I64, _P]),
    "mj_dequantize_i32_scaled_f32": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _P]),
    "mj_quant_linear_f32": (_I32, [_P, _P, _P, _F, _F, _P, _I64, _I64, _I64, _I32, _P]),
    "mj_quant_linear_f32_noalloc": (_I32, [_P, _P, _P, _F, _F, _P, _I64, _I64, _I64, _I32, _P]),
    "mj_quantize_rowwise_i8": (_I32, [_P, _I64, _I64, _I32, _P, _P, _P]),
    "mj_linear_w8a16": (_I32, [_P, _P, _P, _P, _I32, _P, _I64, _I64, _I64, _P]),
    "mj_quantize_rows_bf16_i8": (_I32, [_P, _I64, _I64, _P, _P, _P]),
    "mj_linear_w8a8": (_I32, [_P, _P, _P, _P, _I32, _P, _I64, _I64, _I64, _P]),
    "mj_mlp_w8a16": (_I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    # device memory and streams
    "mj_malloc": (_I32, [ctypes.POINTER(_P), _I64]),
    "mj_free": (_I32, [_P]),
    "mj_memcpy_htod": (_I32, [_P, _P, _I64, _P]),
    "mj_memcpy_dtoh": (_I32, [_P, _P, _I64, _P]),
    "mj_memcpy_dtod": (_I32, [_P, _P, _I64, _P]),
    "mj_stream_create": (_I32, [ctypes.POINTER(_P)]),
    "mj_stream_destroy": (_I32, [_P]),
    "mj_device_synchronize": (_I32, []),
    # host-pointer variants
    "mj_matmul_f32_h": (_I32, [_I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _I64]),
    "mj_matvec_f32_h": (_I32, [_I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "mj_matmul_f64_h": (_I32, [_I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64]),
    "mj_matvec_f64_h": (_I32, [_I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "mj_tensordot_f32_h": (_I32, [_I32, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64,
                                  _I64, _P]),
    "mj_linear_f32_h": (_I32, [_P, _P, _P, _I32, _P, _I64, _I64, _I64]),
    "mj_linear_backward_f32_h": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "mj_matmul_backward_f64_h": (_I32, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _I32]),
    "mj_matmul_backward_f32_h": (_I32, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _I32]),
    "mj_activation_f32_h": (_I32, [_I32, _P, _P, _I64]),
    "mj_gemm_bf16_nt_h": (_I32, [_I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I32, _P, _I64]),
    "mj_quantize_symmetric_int8_h": (_I32, [_P, _I64, _F, _P]),
    "mj_minmax_f32_h": (_I32, [_P, _I64, _P]),
    "mj_minmax_scale_symmetric_h": (_I32, [_P, _I64, _F, _P]),
    "mj_matmul_i8_i8_to_i32_h": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I32]),
    "mj_dequantize_i32_to_f32_add_bias_h": (_I32, [_P, _F, _P, _P, _I64, _I64]),
    "mj_dequantize_i32_scaled_f32_h": (_I32, [_P, _P, _P, _P, _P, _I64, _I64]),
    "mj_quant_linear_f32_h": (_I32, [_P, _P, _P, _F, _F, _P, _I64, _I64, _I64, _I32]),
    "mj_quantize_rowwise_i8_h": (_I32, [_P, _I64, _I64, _I32, _P, _P]),
    "mj_linear_w8a16_h": (_I32, [_P, _P, _P, _P, _I32, _P, _I64, _I64, _I64]),
    "mj_linear_w8a8_h": (_I32, [_P, _P, _P, _P, _I32, _P, _I64, _I64, _I64]),
    "mj_mlp_w8a16_h": (_I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/momijo_hip.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(mj_[a-z0-9_]+)\s*\(", text)


def load() -> ctypes.CDLL:
    """Load the in-tree library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m momijo_amd.build` "
                "(there is no CPU fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status: int, fn: str) -> None:
    if status != MJ_OK:
        msg = load().mj_last_error()
        raise MomijoHipError(status, fn, msg.decode() if msg else "")


def call(fn: str, *args) -> None:
    check(getattr(load(), fn)(*args), fn)


def device_available() -> bool:
    return bool(load().mj_device_available())
