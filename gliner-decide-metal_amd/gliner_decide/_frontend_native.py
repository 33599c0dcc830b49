"""ctypes binding of libgliner_decide_frontend.so (include/gliner_decide_frontend.h).

The decision front end (schema, word split, added-token cut, tokenizer.json
pipeline, bucket choice) in C++; no GPU involved.  There is no fallback: if
the library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_NAME = "libgliner_decide_frontend.so"
DEFAULT_LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / LIB_NAME

GD_OK = 0
GD_ERR_SHAPE = -2
GD_ERR_TOKENIZER_FILES = -20
GD_ERR_TOKENIZER_CONFIG = -21
GD_ERR_NO_TASK_LABELS = -22
GD_ERR_INPUT_DOES_NOT_FIT = -23

_vp, _i32p, _i64p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_int64)
_SIGNATURES = {
    "gd_frontend_last_error": (C.c_char_p, []),
    "gd_frontend_open": (C.c_int, [C.POINTER(_vp), C.c_char_p]),
    "gd_frontend_create": (C.c_int, [C.POINTER(_vp), C.c_char_p, C.c_size_t]),
    "gd_frontend_destroy": (None, [_vp]),
    "gd_frontend_pad_id": (C.c_int, [_vp, _i32p]),
    "gd_frontend_clear_cache": (C.c_int, [_vp]),
    "gd_frontend_encode": (C.c_int, [_vp, C.c_char_p, C.c_size_t, _i32p, C.c_int64, _i64p]),
    "gd_frontend_append_tokenized": (C.c_int, [_vp, C.c_char_p, C.c_size_t, _i32p, C.c_int64, _i64p]),
    "gd_frontend_split_words": (C.c_int, [_vp, C.c_char_p, C.c_size_t, C.c_char_p, C.c_int64, _i64p, _i64p]),
    "gd_frontend_make_input": (C.c_int, [_vp, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, _i64p, C.c_int64,
                                         _i32p, C.POINTER(C.c_uint16), C.c_int64, _i32p, C.POINTER(C.c_float),
                                         C.c_int64, _i64p, _i64p, _i64p, _i64p]),
}

_lib = None


class FrontendError(ValueError):
    """A non-zero gd_status from the front-end library."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(message)


def library_path() -> Path:
    env = os.environ.get("GLINER_DECIDE_FRONTEND_LIB")
    return Path(env) if env else DEFAULT_LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run `python gliner-decide-metal_amd/build.py`")
    handle = C.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    _lib = handle
    return handle


def check(status: int) -> None:
    if status != GD_OK:
        msg = lib().gd_frontend_last_error()
        raise FrontendError(status, msg.decode("utf-8", "replace") if msg else f"status {status}")
