"""ctypes binding of include/tinybrain_hip.h (libtinybrain_hip.so).

The library is built in-tree by ``python -m tinybrain_amd.build``.  There is
no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtinybrain_hip.so")

# status codes
OK, E_INVALID, E_UNSUPPORTED, E_NODEVICE, E_OOM, E_HIP = range(6)
# descriptor codes (QuantizationPrecision / QuantizationMode / layout)
PREC_INT8, PREC_INT4 = 1, 2
MODE_SYMMETRIC, MODE_ASYMMETRIC, MODE_PER_CHANNEL, MODE_INT4, MODE_INT4_PER_CHANNEL = range(5)
LAYOUT_KN_FLAT, LAYOUT_NK_FLAT = 0, 1
PATH_INT8_ROW, PATH_INT4_KGROUP, PATH_INT4_NGROUP, PATH_GENERIC = range(4)
PATH_NAMES = {0: "int8_row", 1: "int4_kgroup", 2: "int4_ngroup", 3: "generic"}
# device options (tbh_device_set_option)
OPT_SGEMV_MIN_ROWS, OPT_NOALLOC_SCRATCH_BYTES, OPT_MFMA_MIN_ROWS, OPT_HOST_ENTRY, OPT_HOST_WAIT = 1, 2, 3, 4, 5

# every symbol the header declares
EXPORTS = [
    "tbh_abi_version", "tbh_last_error", "tbh_status_string",
    "tbh_device_open", "tbh_device_close", "tbh_device_get_info", "tbh_device_set_option",
    "tbh_weight_create", "tbh_weight_create_concat", "tbh_weight_destroy", "tbh_weight_get_info",
    "tbh_matmul", "tbh_matmul_device", "tbh_matmul_device_noalloc", "tbh_matmul_bf16_device",
    "tbh_linear_device", "tbh_dequantize", "tbh_dequantize_device",
    "tbh_decoder_create", "tbh_decoder_set_layer", "tbh_decoder_destroy",
    "tbh_decoder_set_position", "tbh_decoder_get_position",
    "tbh_decoder_step_device", "tbh_decoder_step",
    "tbh_tbf_open", "tbh_tbf_close", "tbh_tbf_get_config", "tbh_tbf_tensor_count",
    "tbh_tbf_tensor", "tbh_tbf_find", "tbh_tbf_qtensor", "tbh_tbf_floats", "tbh_tbf_load_decoder",
    "tbh_softmax", "tbh_softmax_device", "tbh_rmsnorm", "tbh_rmsnorm_device",
    "tbh_silu", "tbh_silu_device", "tbh_gelu", "tbh_gelu_device",
    "tbh_attention", "tbh_attention_device",
]


class AttentionShape(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("seq_len", ctypes.c_int64),
        ("kv_len", ctypes.c_int64),
        ("head_dim", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
    ]


class QTensorDesc(ctypes.Structure):
    _fields_ = [
        ("K", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("precision", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("data", ctypes.c_void_p),
        ("data_bytes", ctypes.c_int64),
        ("scales", ctypes.c_void_p),
        ("n_scales", ctypes.c_int64),
        ("zero_points", ctypes.c_void_p),
        ("n_zero_points", ctypes.c_int64),
    ]


class WeightInfo(ctypes.Structure):
    _fields_ = [
        ("K", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("precision", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("path", ctypes.c_int32),
        ("has_zero_points", ctypes.c_int32),
        ("device_bytes", ctypes.c_int64),
        ("stream_bytes", ctypes.c_int64),
    ]


class DecoderConfig(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("intermediate", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("max_seq", ctypes.c_int32),
        ("rms_eps", ctypes.c_float),
        ("rope_base", ctypes.c_float),
    ]


class TBFConfig(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("max_seq", ctypes.c_int32),
        ("intermediate", ctypes.c_int32),
        ("partial_rotary_factor", ctypes.c_float),
        ("architecture", ctypes.c_char * 16),
    ]


class TBFTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("ndim", ctypes.c_int32),
        ("quantized", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 4),
        ("offset", ctypes.c_int64),
        ("bytes", ctypes.c_int64),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """Load libtinybrain_hip.so (raises OSError when it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise OSError(f"{LIB_PATH} is not built; run `python -m tinybrain_amd.build`")
    # One HIP runtime per process: PyTorch ships its own libamdhip64.so.7
    # under the same soname as ROCm's, whichever loads first serves both, and
    # torch cannot initialise its GPU support on a runtime it did not load.
    # When torch is installed, load it first so the library binds to it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    pp = ctypes.POINTER(ctypes.c_void_p)
    L.tbh_abi_version.restype = i32
    L.tbh_last_error.restype = ctypes.c_char_p
    L.tbh_status_string.restype = ctypes.c_char_p
    L.tbh_status_string.argtypes = [i32]
    L.tbh_device_open.argtypes = [i32, pp]
    L.tbh_device_close.argtypes = [vp]
    L.tbh_device_get_info.argtypes = [vp, ctypes.POINTER(i32), ctypes.POINTER(i32)]
    L.tbh_device_set_option.argtypes = [vp, i32, i64]
    L.tbh_weight_create.argtypes = [vp, ctypes.POINTER(QTensorDesc), pp]
    L.tbh_weight_create_concat.argtypes = [vp, i32, ctypes.POINTER(ctypes.POINTER(QTensorDesc)), pp]
    L.tbh_weight_destroy.argtypes = [vp]
    L.tbh_weight_get_info.argtypes = [vp, ctypes.POINTER(WeightInfo)]
    L.tbh_matmul.argtypes = [vp, vp, i64, i64, vp, vp]
    L.tbh_matmul_device.argtypes = [vp, vp, i64, i64, vp, vp]
    L.tbh_matmul_device_noalloc.argtypes = [vp, vp, i64, i64, vp, vp]
    L.tbh_linear_device.argtypes = [vp, vp, i64, i64, vp, vp, vp]
    L.tbh_matmul_bf16_device.argtypes = [vp, vp, i64, i64, vp, vp]
    L.tbh_dequantize.argtypes = [vp, vp, vp]
    L.tbh_dequantize_device.argtypes = [vp, vp, vp]
    dp = ctypes.POINTER(QTensorDesc)
    L.tbh_decoder_create.argtypes = [vp, ctypes.POINTER(DecoderConfig), vp, vp, dp, pp]
    L.tbh_decoder_set_layer.argtypes = [vp, i32, vp, vp, dp, dp, dp, dp, dp, dp, dp]
    L.tbh_decoder_destroy.argtypes = [vp]
    L.tbh_decoder_set_position.argtypes = [vp, i32]
    L.tbh_decoder_get_position.argtypes = [vp, ctypes.POINTER(i32)]
    L.tbh_decoder_step_device.argtypes = [vp, i32, vp, vp]
    L.tbh_decoder_step.argtypes = [vp, i32, vp]
    L.tbh_tbf_open.argtypes = [ctypes.c_char_p, pp]
    L.tbh_tbf_close.argtypes = [vp]
    L.tbh_tbf_get_config.argtypes = [vp, ctypes.POINTER(TBFConfig)]
    L.tbh_tbf_tensor_count.argtypes = [vp]
    L.tbh_tbf_tensor_count.restype = i32
    L.tbh_tbf_tensor.argtypes = [vp, i32, ctypes.POINTER(TBFTensor)]
    L.tbh_tbf_find.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(i32)]
    L.tbh_tbf_qtensor.argtypes = [vp, i32, dp]
    L.tbh_tbf_floats.argtypes = [vp, i32, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(i64)]
    L.tbh_tbf_load_decoder.argtypes = [vp, vp, i32, pp]
    f32 = ctypes.c_float
    L.tbh_softmax.argtypes = [vp, vp, i64, i64, vp]
    L.tbh_softmax_device.argtypes = [vp, vp, i64, i64, vp, vp]
    L.tbh_rmsnorm.argtypes = [vp, vp, i64, i64, vp, f32, vp]
    L.tbh_rmsnorm_device.argtypes = [vp, vp, i64, i64, vp, f32, vp, vp]
    for op in ("silu", "gelu"):
        getattr(L, "tbh_" + op).argtypes = [vp, vp, i64, vp]
        getattr(L, "tbh_" + op + "_device").argtypes = [vp, vp, i64, vp, vp]
    sp = ctypes.POINTER(AttentionShape)
    L.tbh_attention.argtypes = [vp, sp, vp, vp, vp, vp, vp]
    L.tbh_attention_device.argtypes = [vp, sp, vp, vp, vp, vp, vp, vp]
    for name in ("tbh_tbf_open", "tbh_tbf_close", "tbh_tbf_get_config", "tbh_tbf_tensor",
                 "tbh_tbf_find", "tbh_tbf_qtensor", "tbh_tbf_floats", "tbh_tbf_load_decoder"):
        getattr(L, name).restype = i32
    for name in ("tbh_decoder_create", "tbh_decoder_set_layer", "tbh_decoder_destroy",
                 "tbh_decoder_set_position", "tbh_decoder_get_position",
                 "tbh_decoder_step_device", "tbh_decoder_step"):
        getattr(L, name).restype = i32
    for name in ("tbh_device_open", "tbh_device_close", "tbh_device_get_info", "tbh_device_set_option",
                 "tbh_weight_create", "tbh_weight_create_concat", "tbh_weight_destroy", "tbh_weight_get_info",
                 "tbh_matmul", "tbh_matmul_device", "tbh_matmul_device_noalloc", "tbh_matmul_bf16_device",
                 "tbh_linear_device",
                 "tbh_dequantize", "tbh_dequantize_device",
                 "tbh_softmax", "tbh_softmax_device", "tbh_rmsnorm", "tbh_rmsnorm_device",
                 "tbh_silu", "tbh_silu_device", "tbh_gelu", "tbh_gelu_device",
                 "tbh_attention", "tbh_attention_device"):
        getattr(L, name).restype = i32
    _lib = L
    return L


def last_error() -> str:
    return lib().tbh_last_error().decode("utf-8", "replace")


def status_name(st: int) -> str:
    return lib().tbh_status_string(st).decode()
