"""ctypes binding of libgliner_decide_hip.so (include/gliner_decide.h).

There is no fallback: if the library is missing or does not load, every
entry point raises.  Build it with `python gliner-decide-metal_amd/build.py`.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_NAME = "libgliner_decide_hip.so"
_PKG_ROOT = Path(__file__).resolve().parent.parent
DEFAULT_LIB_PATH = _PKG_ROOT / "lib" / LIB_NAME

# gd_status
GD_OK = 0
GD_ERR_INVALID_ARGUMENT = -1
GD_ERR_SHAPE = -2
GD_ERR_UNSUPPORTED = -3
GD_ERR_HIP = -4
GD_ERR_MISSING_WEIGHT = -5
GD_ERR_WEIGHT_SHAPE = -6
GD_ERR_WEIGHT_DTYPE = -7
GD_ERR_IO = -8
GD_ERR_OUT_OF_MEMORY = -9
GD_ERR_DEVICE_INDEX = -10

STATUS_NAMES = {
    GD_ERR_INVALID_ARGUMENT: "invalid argument",
    GD_ERR_SHAPE: "shape",
    GD_ERR_UNSUPPORTED: "unsupported",
    GD_ERR_HIP: "HIP",
    GD_ERR_MISSING_WEIGHT: "missing weight",
    GD_ERR_WEIGHT_SHAPE: "weight shape",
    GD_ERR_WEIGHT_DTYPE: "weight dtype",
    GD_ERR_IO: "I/O",
    GD_ERR_OUT_OF_MEMORY: "out of memory",
    GD_ERR_DEVICE_INDEX: "device index",
}

# gd_dtype
GD_F16, GD_F32, GD_BF16, GD_I32, GD_I64 = 0, 1, 2, 3, 4
# flags / enums
GD_LN_SUM_F16 = 1
GD_EPI_NONE, GD_EPI_BIAS, GD_EPI_BIAS_GELU, GD_EPI_BIAS_RELU = 0, 1, 2, 3
GD_MASK_ATTENTION, GD_MASK_ADDITIVE = 0, 1
GD_ATTN_OUT_PROBS, GD_ATTN_OUT_CONTEXT, GD_ATTN_OUT_BIAS = 0, 1, 2
GD_ATTN_SCORE_DEFAULT, GD_ATTN_SCORE_EXPLICIT, GD_ATTN_SCORE_KERNEL_BIAS = 0x000, 0x100, 0x200
GD_ATTN_SCORE_KERNEL_BIAS_EXPLICIT, GD_ATTN_SCORE_FUSED = 0x300, 0x400
GD_USE_FUSED_KERNELS, GD_USE_COMPILED_GRAPH, GD_USE_GENERIC_ATTENTION, GD_FULL_ROWS = 1, 2, 4, 8
GD_USE_CUSTOM_RELATIVE_KERNEL, GD_USE_FUSED_ATTENTION_KERNEL = 16, 32


class GlinerDecideError(RuntimeError):
    """A non-zero gd_status from the native library."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"[{STATUS_NAMES.get(status, status)}] {message}")


class GdConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32),
        ("num_hidden_layers", C.c_int32),
        ("num_attention_heads", C.c_int32),
        ("layer_norm_eps", C.c_float),
        ("position_buckets", C.c_int32),
        ("max_relative_positions", C.c_int32),
        ("pad_token_id", C.c_int32),
        ("vocab_size", C.c_int32),
        ("classifier_hidden", C.c_int32),
    ]


class GdBhld(C.Structure):
    _fields_ = [("data", C.c_void_p), ("stride_b", C.c_int64), ("stride_h", C.c_int64), ("stride_l", C.c_int64)]


class GdTable(C.Structure):
    _fields_ = [("data", C.c_void_p), ("stride_h", C.c_int64), ("stride_p", C.c_int64)]


class GdProfileEvent(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("milliseconds", C.c_double)]


vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int32
u32 = C.c_uint32
f32 = C.c_float

# name -> (restype, argtypes)
_SIGNATURES = {
    "gd_last_error": (C.c_char_p, []),
    "gd_abi_version": (C.c_int, []),
    "gd_build_info": (C.c_char_p, []),
    "gd_config_default": (None, [C.POINTER(GdConfig)]),
    "gd_residual_layer_norm": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, f32, u32, vp]),
    "gd_embedding_layer_norm": (C.c_int, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, f32, vp, vp]),
    "gd_linear": (C.c_int, [vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, i64, i32, vp]),
    "gd_relative_bias": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, f32, i64, i64, i64, i64, i64, vp, vp]),
    "gd_fused_attention": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, f32, i64, i64, i64, i64, i64, vp, vp]),
    "gd_deberta_attention": (C.c_int, [GdBhld, GdBhld, GdBhld, GdTable, GdTable, vp, i32, i64, i64, i64, i64, i64,
                                       i32, i32, vp, i64, vp]),
    "gd_relative_index_table": (C.c_int, [vp, i32, i32, i32, vp]),
    "gd_stream_probe_add": (C.c_int, [vp, vp, vp, i64, vp]),
    "gd_diag_mfma_forms": (C.c_int, [vp, vp, vp, vp, vp, i64, vp]),
    "gd_weight_store_create": (C.c_int, [C.POINTER(vp)]),
    "gd_weight_store_destroy": (None, [vp]),
    "gd_weight_store_add": (C.c_int, [vp, C.c_char_p, vp, i32, C.POINTER(i64), i32]),
    "gd_weight_store_load_safetensors": (C.c_int, [vp, C.c_char_p]),
    "gd_weight_store_count": (i64, [vp]),
    "gd_weight_store_get": (C.c_int, [vp, C.c_char_p, C.POINTER(i32), C.POINTER(i64), C.POINTER(i32),
                                      C.POINTER(vp), C.POINTER(i64)]),
    "gd_classifier_create": (C.c_int, [C.POINTER(vp), vp, C.POINTER(GdConfig), u32, vp]),
    "gd_classifier_destroy": (None, [vp]),
    "gd_classifier_reserve": (C.c_int, [vp, i64, i64, i64, i64]),
    "gd_classifier_classify": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, i64, i64, vp, vp]),
    "gd_classifier_classify_packed": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp]),
    "gd_classifier_classify_static": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp]),
    "gd_classifier_encode": (C.c_int, [vp, vp, vp, i64, i64, i32, vp, vp]),
    "gd_classifier_layer_forward": (C.c_int, [vp, i32, vp, vp, i64, i64, vp, vp]),
    "gd_classifier_classify_profiled": (C.c_int, [vp, vp, vp, vp, vp, i64, i64, i64, i64, vp,
                                                  C.POINTER(GdProfileEvent), i32, C.POINTER(i32), vp]),
    "gd_classifier_check_device_errors": (C.c_int, [vp, vp]),
    "gd_classifier_device_bytes": (i64, [vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None


def library_path() -> Path:
    env = os.environ.get("GLINER_DECIDE_LIB")
    return Path(env) if env else DEFAULT_LIB_PATH


def lib() -> C.CDLL:
    """Loads the native library once; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built: run `python gliner-decide-metal_amd/build.py` "
            "(the HIP library is required; there is no fallback path)")
    handle = C.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return handle


def last_error() -> str:
    msg = lib().gd_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != GD_OK:
        raise GlinerDecideError(status, last_error())
