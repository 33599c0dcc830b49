"""`WeightStore` (Weights.swift:23-58) over the native store.

Keys follow the fp16 checkpoint written by Tools/prepare_model.py:82-113
(`encoder.*` and `classifier.*`).  The store copies host arrays; the
classifier uploads them to HBM at construction.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import _native as N

_NP_TO_GD = {np.dtype(np.float16): N.GD_F16, np.dtype(np.float32): N.GD_F32, np.dtype(np.int32): N.GD_I32,
             np.dtype(np.int64): N.GD_I64}
_GD_TO_NP = {v: k for k, v in _NP_TO_GD.items()}


class WeightStore:
    def __init__(self, arrays: dict | None = None, url: str | Path | None = None):
        self._lib = N.lib()
        h = C.c_void_p()
        N.check(self._lib.gd_weight_store_create(C.byref(h)))
        self._h = h
        if url is not None:
            self.load_safetensors(url)
        if arrays:
            for k, v in arrays.items():
                self.add(k, v)

    def add(self, key: str, array) -> None:
        a = np.ascontiguousarray(array)
        if a.dtype not in _NP_TO_GD:
            raise TypeError(f"{key}: unsupported dtype {a.dtype}")
        shape = (C.c_int64 * max(a.ndim, 1))(*a.shape)
        N.check(self._lib.gd_weight_store_add(self._h, key.encode(), a.ctypes.data_as(C.c_void_p),
                                              _NP_TO_GD[a.dtype], shape, a.ndim))

    def load_safetensors(self, path: str | Path) -> None:
        N.check(self._lib.gd_weight_store_load_safetensors(self._h, str(path).encode()))

    def array(self, key: str) -> np.ndarray:
        """A copy of the stored tensor `key` (the lookup of WeightStore.array,
        Weights.swift:35-57); BF16 entries come back as raw uint16."""
        dtype, ndim, data, nbytes = C.c_int32(), C.c_int32(), C.c_void_p(), C.c_int64()
        shape = (C.c_int64 * 8)()
        N.check(self._lib.gd_weight_store_get(self._h, key.encode(), C.byref(dtype), shape, C.byref(ndim),
                                              C.byref(data), C.byref(nbytes)))
        np_dtype = _GD_TO_NP.get(dtype.value, np.dtype(np.uint16))
        raw = C.string_at(data, nbytes.value) if nbytes.value else b""
        return np.frombuffer(raw, dtype=np_dtype).reshape(tuple(shape[: ndim.value])).copy()

    def __len__(self) -> int:
        return int(self._lib.gd_weight_store_count(self._h))

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            self._lib.gd_weight_store_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
