"""GgufReader over libjunohip's native GGUF reader.

Mirrors the reference's reader (paths under
/root/reference/node/src/main/java/cab/ml/juno/node/):

* ``GgufReader.open``        GgufReader.open (GgufReader.java:102-183), llamafile ZIPs
                             included (findGgufOffsetInZip, :808-1154)
* ``meta`` / ``meta_*``      meta / metaString / metaLong / metaInt / metaFloat
                             (:185-207) with Java's Number conversions
* ``tensor_*``               hasTensor / tensorAbsoluteOffset / tensorType /
                             tensorDims / tensorNelems / tensorOrder (:209-280)
* ``tensor_raw``             tensorRaw (:329-345) -> QuantizedTensor
* ``tensor``                 tensor (:366-380): F32 / F16 / BF16 converted exactly on
                             the host; packed types dequantized by the device kernels
* ``upload``                 new: tensorRaw + upload in one pass, streamed from the
                             file into HBM without a host copy of the tensor

Parsing runs in the native library; there is no Python parser to fall back to.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .matvec import (F32, DeviceQuantMatrix, IllegalArgumentException, QuantizedTensor, _check)

GGML_TYPE_F16, GGML_TYPE_BF16 = 1, 30

(GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING,
 GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64) = range(13)
_FLOATS = (GGUF_FLOAT32, GGUF_FLOAT64)


@dataclass(frozen=True)
class GgufArray:
    """An array-valued metadata entry (the reference's Object[]): element type
    and length.  The elements themselves are not materialised."""
    elem_type: int
    length: int

    def __len__(self) -> int:
        return self.length


def _java_int(v: int) -> int:
    """(int) of a Java long: the low 32 bits, two's complement."""
    v &= 0xFFFFFFFF
    return v - (1 << 32) if v >= 1 << 31 else v


def _java_f2i(f: float, bits: int) -> int:
    """(int) / (long) of a Java float or double: truncation, NaN -> 0, saturating."""
    if f != f:
        return 0
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    if f >= hi:
        return hi
    if f <= lo:
        return lo
    return int(f)


class GgufReader:
    """An open GGUF (or llamafile) file; use as a context manager or close()."""

    def __init__(self, handle: ctypes.c_void_p, path: str):
        self._h = handle
        self.path = path
        self._L = _lib.load()
        v, nt, nkv, go, do, me = (ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(),
                                  ctypes.c_int64(), ctypes.c_int64())
        _check(self._L.jh_gguf_info(self._h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(go),
                                    ctypes.byref(do), ctypes.byref(me)))
        self.version, self.tensor_count, self.kv_count = v.value, nt.value, nkv.value
        self._gguf_offset, self.data_offset, self._metadata_end = go.value, do.value, me.value
        self._order = [self._info(i)[0] for i in range(self.tensor_count)]

    # ---------------------------------------------------------------- lifecycle
    @classmethod
    def open(cls, path) -> "GgufReader":
        h = ctypes.c_void_p()
        _check(_lib.load().jh_gguf_open(str(path).encode(), ctypes.byref(h)))
        return cls(h, str(path))

    def close(self) -> None:
        if self._h is not None:
            self._L.jh_gguf_close(self._h)
            self._h = None

    def __enter__(self) -> "GgufReader":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise IllegalArgumentException("GgufReader is closed")
        return self._h

    # ---------------------------------------------------------------- metadata
    def _type(self, key: str):
        vt, et, n = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        _check(self._L.jh_gguf_meta_type(self.handle, key.encode(), ctypes.byref(vt), ctypes.byref(et),
                                         ctypes.byref(n)))
        return vt.value, et.value, n.value

    def _number(self, key: str):
        present, lv, dv = ctypes.c_int(), ctypes.c_int64(), ctypes.c_double()
        _check(self._L.jh_gguf_meta_number(self.handle, key.encode(), ctypes.byref(present), ctypes.byref(lv),
                                           ctypes.byref(dv)))
        return bool(present.value), lv.value, dv.value

    def meta(self, key: str):
        """meta(key) (GgufReader.java:185-187): int / long (Python int), float
        (FLOAT32 and FLOAT64 values), bool, str, GgufArray, or None."""
        vt, et, n = self._type(key)
        if vt < 0:
            return None
        if vt == GGUF_STRING:
            return self.meta_string(key)
        if vt == GGUF_ARRAY:
            return GgufArray(et, n)
        if vt == GGUF_BOOL:
            present, val = ctypes.c_int(), ctypes.c_int()
            _check(self._L.jh_gguf_meta_bool(self.handle, key.encode(), ctypes.byref(present), ctypes.byref(val)))
            return bool(val.value)
        _, lv, dv = self._number(key)
        return dv if vt in _FLOATS else lv

    def meta_string(self, key: str):
        """metaString (:189-192): the value if it is a string, else None."""
        n = ctypes.c_size_t()
        _check(self._L.jh_gguf_meta_string(self.handle, key.encode(), None, 0, ctypes.byref(n)))
        if n.value == ctypes.c_size_t(-1).value:
            return None
        buf = ctypes.create_string_buffer(n.value + 1)
        _check(self._L.jh_gguf_meta_string(self.handle, key.encode(), buf, n.value + 1, ctypes.byref(n)))
        return buf.raw[:n.value].decode("utf-8", errors="replace")

    def meta_long(self, key: str, default: int) -> int:
        """metaLong (:194-197): Number.longValue() or default."""
        present, lv, _ = self._number(key)
        return lv if present else default

    def meta_int(self, key: str, default: int) -> int:
        """metaInt (:199-202): Number.intValue() or default."""
        vt, _, _ = self._type(key)
        present, lv, dv = self._number(key)
        if not present:
            return default
        return _java_f2i(dv, 32) if vt in _FLOATS else _java_int(lv)

    def meta_float(self, key: str, default: float) -> float:
        """metaFloat (:204-207): Number.floatValue() (float32) or default."""
        vt, _, _ = self._type(key)
        present, lv, dv = self._number(key)
        if not present:
            return float(np.float32(default))
        return float(np.float32(dv)) if vt in _FLOATS else float(np.float32(lv))

    # ---------------------------------------------------------------- tensors
    def _info(self, i: int):
        name, t, nd, ne, off = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64()
        dims = (ctypes.c_int64 * 8)()
        _check(self._L.jh_gguf_tensor_info(self.handle, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd),
                                           dims, ctypes.byref(ne), ctypes.byref(off)))
        return name.value.decode("utf-8", errors="replace"), t.value, tuple(dims[:nd.value]), ne.value, off.value

    def _index(self, name: str) -> int:
        i = ctypes.c_int64()
        _check(self._L.jh_gguf_tensor_index(self.handle, name.encode(), ctypes.byref(i)))
        return i.value

    def _require(self, name: str) -> int:
        i = self._index(name)
        if i < 0:
            raise IllegalArgumentException(f"Tensor not found: {name}  (available: {len(set(self._order))} tensors)")
        return i

    def has_tensor(self, name: str) -> bool:
        return self._index(name) >= 0

    def tensor_order(self) -> list:
        return list(self._order)

    def tensor_type(self, name: str) -> int:
        return self._info(self._require(name))[1]

    def tensor_dims(self, name: str) -> tuple:
        return self._info(self._require(name))[2]

    def tensor_nelems(self, name: str) -> int:
        return self._info(self._require(name))[3]

    def tensor_absolute_offset(self, name: str) -> int:
        return self._info(self._require(name))[4]

    def metadata_section_end(self) -> int:
        return self._metadata_end

    def gguf_file_offset(self) -> int:
        return self._gguf_offset

    def tensor_raw(self, name: str) -> QuantizedTensor:
        """tensorRaw (:329-345)."""
        i = self._require(name)
        _, t, _, ne, _ = self._info(i)
        n = ctypes.c_size_t()
        _check(self._L.jh_gguf_tensor_read(self.handle, i, None, 0, ctypes.byref(n)))
        buf = np.empty(n.value, dtype=np.uint8)
        _check(self._L.jh_gguf_tensor_read(self.handle, i, buf.ctypes.data, buf.size, ctypes.byref(n)))
        return QuantizedTensor(name, t, ne, buf.tobytes())

    def tensor(self, name: str, backend=None) -> np.ndarray:
        """tensor(name) (:366-380) as float32.  F32, F16 and BF16 widen exactly on
        the host; the packed types are dequantized by the device kernels
        (``backend`` = a MatVec backend, default the shared device 0)."""
        qt = self.tensor_raw(name)
        raw = np.frombuffer(qt.data, dtype=np.uint8)
        if qt.type == F32:
            return raw.view(np.float32).copy()
        if qt.type == GGML_TYPE_F16:
            return raw.view(np.float16).astype(np.float32)
        if qt.type == GGML_TYPE_BF16:
            return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        m = self.upload(name, backend)
        try:
            return (backend or _default_backend()).dequantize(m).reshape(-1)
        finally:
            m.close()

    def upload(self, name: str, backend=None) -> DeviceQuantMatrix:
        """The tensor's packed bytes, streamed from the file into a resident
        matrix: cols = dims[0], rows = nelems / dims[0]."""
        be = backend or _default_backend()
        i = self._require(name)
        _, t, dims, ne, _ = self._info(i)
        h = ctypes.c_void_p()
        _check(self._L.jh_gguf_upload(be.ctx.handle, self.handle, i, ctypes.byref(h)))
        cols = dims[0] if dims else 1
        return DeviceQuantMatrix(h, t, ne // cols, cols)

    @staticmethod
    def raw_byte_count(qtype: int, nelems: int) -> int:
        """rawByteCount (:347-360), every type the reference sizes."""
        per = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 2: (32, 18), 10: (256, 84), 11: (256, 110),
               12: (256, 144), 13: (256, 176), 14: (256, 210)}
        if qtype not in per:
            from .matvec import UnsupportedOperationException
            raise UnsupportedOperationException(f"No byte-size formula for GGML type {qtype}")
        qk, bb = per[qtype]
        return (nelems // qk) * bb


def _default_backend():
    from .matvec import GpuContext
    return GpuContext.shared(0).create_mat_vec()
