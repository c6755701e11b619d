"""GGUF files and device residency through ``libqlin`` (``include/qlin_gguf.h``).

Mirrors the reference engine's container classes so a caller written against them reads the same:

- ``GgufFile`` as ``GgufFile`` (AI/codes/local-llm/src/format/gguf/GgufFile.h): ``version``,
  ``alignment``, ``contain_metadata`` / ``metadata_value``, ``contain_tensor_view`` /
  ``get_tensor_view`` / ``tensor_view_names``;
- ``TensorView`` as ``StorageTensor`` (src/tensor/StorageTensor.h): name, dtype (ggml code), shape
  ``[outermost .. innermost]`` (a weight is ``[out_dim, in_dim]``), nbytes, and the row stride the
  kernels take (``nbytes / shape[0]``, as TensorTool::gemm derives it, TensorTool.cpp:156);
- ``WeightPool`` as ``CudaWeightPool::cached_weight`` (src/backend/cuda/mem/CudaWeightPool.cpp:119-175)
  with the expert views of RoutedExperts.cpp:23-32.

All parsing and copying happen in the C library; this module only binds it and raises
``qlin.QlinError`` where the reference throws.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import qlin

VALUE_INT = (0, 1, 2, 3, 4, 5, 10, 11)
VALUE_F32, VALUE_BOOL, VALUE_STRING, VALUE_ARRAY, VALUE_F64 = 6, 7, 8, 9, 12


@dataclass
class TensorView:
    name: str
    dtype: int
    shape: tuple
    nbytes: int
    offset: int
    host_ptr: int

    @property
    def row_bytes(self) -> int:
        return self.nbytes // self.shape[0] if self.shape and self.shape[0] else self.nbytes

    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def host_bytes(self) -> bytes:
        """The packed bytes as stored in the file."""
        return C.string_at(self.host_ptr, self.nbytes)


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise qlin.QlinError(fn, rc)


class GgufFile:
    def __init__(self, path: str):
        self._lib = qlin.lib()
        h = C.c_void_p()
        _check("qlin_gguf_open", self._lib.qlin_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.path = str(path)

    def close(self) -> None:
        if self._h:
            self._lib.qlin_gguf_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    @property
    def version(self) -> int:
        return self._lib.qlin_gguf_version(self._h)

    @property
    def alignment(self) -> int:
        return self._lib.qlin_gguf_alignment(self._h)

    # ---- tensors ------------------------------------------------------------------------------
    def _view(self, index: int) -> TensorView:
        info = qlin.GgufTensorInfo()
        _check("qlin_gguf_tensor_info", self._lib.qlin_gguf_tensor_info(self._h, index, C.byref(info)))
        return TensorView(info.name.decode(), info.type, tuple(info.shape[:info.n_dims]), info.nbytes, info.offset,
                          info.data or 0)

    def tensor_view_names(self) -> list:
        return [self._view(i).name for i in range(self._lib.qlin_gguf_tensor_count(self._h))]

    def contain_tensor_view(self, name: str) -> bool:
        return self._lib.qlin_gguf_find_tensor(self._h, name.encode()) >= 0

    def get_tensor_view(self, name: str) -> TensorView:
        i = self._lib.qlin_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise qlin.QlinError("qlin_gguf_find_tensor", 10)
        return self._view(i)

    # ---- metadata -----------------------------------------------------------------------------
    def metadata_keys(self) -> list:
        return [self._lib.qlin_gguf_metadata_key(self._h, i).decode()
                for i in range(self._lib.qlin_gguf_metadata_count(self._h))]

    def contain_metadata(self, key: str) -> bool:
        return self._lib.qlin_gguf_metadata_type(self._h, key.encode()) >= 0

    def metadata_value(self, key: str):
        """int (integers), bool, float (f32 / f64), str, or a list for arrays."""
        k = key.encode()
        t = self._lib.qlin_gguf_metadata_type(self._h, k)
        if t < 0:
            raise qlin.QlinError("qlin_gguf_metadata_type", 10)
        if t in VALUE_INT or t == VALUE_BOOL:
            v = C.c_int64()
            _check("qlin_gguf_get_i64", self._lib.qlin_gguf_get_i64(self._h, k, C.byref(v)))
            return bool(v.value) if t == VALUE_BOOL else v.value
        if t in (VALUE_F32, VALUE_F64):
            v = C.c_double()
            _check("qlin_gguf_get_f64", self._lib.qlin_gguf_get_f64(self._h, k, C.byref(v)))
            return v.value
        if t == VALUE_STRING:
            p, n = C.c_void_p(), C.c_size_t()
            _check("qlin_gguf_get_str", self._lib.qlin_gguf_get_str(self._h, k, C.byref(p), C.byref(n)))
            return C.string_at(p.value, n.value).decode("utf-8", "replace") if n.value else ""
        et, cnt = C.c_int(), C.c_int64()
        _check("qlin_gguf_get_array_info", self._lib.qlin_gguf_get_array_info(self._h, k, C.byref(et), C.byref(cnt)))
        out = []
        for i in range(cnt.value):
            if et.value == VALUE_STRING:
                p, n = C.c_void_p(), C.c_size_t()
                _check("qlin_gguf_get_array_str", self._lib.qlin_gguf_get_array_str(self._h, k, i, C.byref(p),
                                                                                    C.byref(n)))
                out.append(C.string_at(p.value, n.value).decode("utf-8", "replace") if n.value else "")
            elif et.value in (VALUE_F32, VALUE_F64):
                v = C.c_double()
                _check("qlin_gguf_get_array_f64", self._lib.qlin_gguf_get_array_f64(self._h, k, i, C.byref(v)))
                out.append(v.value)
            elif et.value in VALUE_INT or et.value == VALUE_BOOL:
                v = C.c_int64()
                _check("qlin_gguf_get_array_i64", self._lib.qlin_gguf_get_array_i64(self._h, k, i, C.byref(v)))
                out.append(v.value)
            else:  # nested arrays: elements are not kept
                out.append(None)
        return out


class WeightPool:
    """One device copy per tensor name (uploaded on first use), freed with the pool."""

    def __init__(self):
        self._lib = qlin.lib()
        h = C.c_void_p()
        _check("qlin_pool_create", self._lib.qlin_pool_create(C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            self._lib.qlin_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def resident_bytes(self) -> int:
        return self._lib.qlin_pool_resident_bytes(self._h)

    def cached_weight(self, f: GgufFile, name: str) -> tuple:
        """(device address, nbytes) of tensor `name` of file `f`."""
        p, n = C.c_void_p(), C.c_uint64()
        _check("qlin_pool_weight", self._lib.qlin_pool_weight(self._h, f.handle, name.encode(), C.byref(p),
                                                              C.byref(n)))
        return p.value, n.value

    def expert_view(self, f: GgufFile, name: str, expert: int) -> tuple:
        """(device address, expert_bytes, rows, cols) of expert `expert` of packed [E, rows, cols] `name`."""
        p, n, r, c = C.c_void_p(), C.c_uint64(), C.c_int64(), C.c_int64()
        _check("qlin_pool_expert_view", self._lib.qlin_pool_expert_view(self._h, f.handle, name.encode(), expert,
                                                                        C.byref(p), C.byref(n), C.byref(r),
                                                                        C.byref(c)))
        return p.value, n.value, r.value, c.value
