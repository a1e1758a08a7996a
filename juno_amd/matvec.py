"""Host-side mirror of Juno's matvec interface over libjunohip.

Names, argument meaning and error behaviour follow the reference (paths under
/root/reference/node/src/main/java/cab/ml/juno/node/):

* ``QuantizedTensor``   GgufReader.QuantizedTensor record (GgufReader.java:319-320)
* ``MatVecBackend``     JFR backend labels (MatVecBackend.java:36-64), plus the
                        resident-quantized labels this library adds
* ``GpuContext``        GpuContext.shared(device) (GpuContext.java:109-120)
* ``DeviceQuantMatrix`` device-resident packed weights, AutoCloseable like
                        DeviceHalfMatrix (DeviceHalfMatrix.java:41-115)
* ``HipMatVec``         the GpuMatVec backend (GpuMatVec.java:38-70, RocmMatVec.java):
                        ``sgemv(A, x, rows, cols)``, ``upload_quant``,
                        ``sgemv_quant(dev, x, row_start, row_end)`` (the device-resident
                        form of LlamaTransformerHandler.matVec(QuantizedTensor, x, rowStart,
                        rowEnd, cols), LlamaTransformerHandler.java:1200-1212),
                        ``sgemv_batched`` and ``dequantize``.

Exceptions: ``IllegalArgumentException`` (ValueError) for dimension errors with
the reference's "rows*cols" / "cols" wording (MatVecBackendContractTest.java:196-212),
``IllegalStateException`` (RuntimeError) for HIP failures "<op> failed: rc=N"
(GpuBindings.java:180-183) and out-of-memory ("hipMalloc ..."), and
``UnsupportedOperationException`` (NotImplementedError) for other ggml types.
"""
from __future__ import annotations

import ctypes
import enum
import threading
from dataclasses import dataclass

import numpy as np

from . import _lib


class IllegalArgumentException(ValueError):
    pass


class IllegalStateException(RuntimeError):
    pass


class UnsupportedOperationException(NotImplementedError):
    pass


class IOException(OSError):
    pass


F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 8, 10, 11, 12, 13, 14
SUPPORTED_TYPES = (F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
_QK = {F32: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
_BLOCK_BYTES = {F32: 4, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def raw_byte_count(qtype: int, nelems: int) -> int:
    """GgufReader.rawByteCount (GgufReader.java:347-360) for the supported types."""
    if qtype not in _QK:
        raise UnsupportedOperationException(f"No byte-size formula for GGML type {qtype}")
    return (nelems // _QK[qtype]) * _BLOCK_BYTES[qtype]


class MatVecBackend(enum.Enum):
    """JFR ``juno.MatVec`` backend labels (MatVecBackend.java:36-64)."""
    CPU = "cpu"
    ROCM = "rocm"
    ROCM_RESIDENT = "rocm-resident"
    ROCM_RESIDENT_FP16 = "rocm-resident-fp16"
    # new: packed weights resident on the device, fused dequant-GEMV
    ROCM_RESIDENT_Q2K = "rocm-resident-q2k"
    ROCM_RESIDENT_Q3K = "rocm-resident-q3k"
    ROCM_RESIDENT_Q4K = "rocm-resident-q4k"
    ROCM_RESIDENT_Q5K = "rocm-resident-q5k"
    ROCM_RESIDENT_Q6K = "rocm-resident-q6k"
    ROCM_RESIDENT_Q8_0 = "rocm-resident-q8_0"

    @property
    def label(self) -> str:
        return self.value

    @staticmethod
    def for_type(qtype: int) -> "MatVecBackend":
        return {F32: MatVecBackend.ROCM_RESIDENT, Q2_K: MatVecBackend.ROCM_RESIDENT_Q2K,
                Q3_K: MatVecBackend.ROCM_RESIDENT_Q3K, Q4_K: MatVecBackend.ROCM_RESIDENT_Q4K, Q5_K: MatVecBackend.ROCM_RESIDENT_Q5K,
                Q6_K: MatVecBackend.ROCM_RESIDENT_Q6K, Q8_0: MatVecBackend.ROCM_RESIDENT_Q8_0}[qtype]


@dataclass(frozen=True)
class QuantizedTensor:
    """GgufReader.QuantizedTensor(name, type, nelems, data) (GgufReader.java:319-320)."""
    name: str
    type: int
    nelems: int
    data: bytes


def _check(rc: int) -> None:
    if rc == _lib.JH_OK:
        return
    msg = _lib.last_error()
    if rc == _lib.JH_EINVAL:
        raise IllegalArgumentException(msg)
    if rc == _lib.JH_EUNSUPPORTED:
        raise UnsupportedOperationException(msg)
    if rc in (_lib.JH_EFORMAT, _lib.JH_EIO):
        raise IOException(msg)
    raise IllegalStateException(msg)


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(_lib.load().jh_device_count(ctypes.byref(n)))
    return n.value


def device_info(device: int = 0) -> dict:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    vram = ctypes.c_uint64(0)
    _check(_lib.load().jh_device_info(device, name, ctypes.byref(vram), arch))
    return {"name": name.value.decode(), "vram_bytes": vram.value, "arch": arch.value.decode()}


class GpuContext:
    """Process-wide shared context per device (GpuContext.shared, GpuContext.java:109-120)."""
    _shared: dict = {}
    _mu = threading.Lock()

    def __init__(self, device: int):
        h = ctypes.c_void_p()
        _check(_lib.load().jh_ctx_create(device, ctypes.byref(h)))
        self.device = device
        self.handle = h

    @classmethod
    def shared(cls, device: int = 0) -> "GpuContext":
        with cls._mu:
            ctx = cls._shared.get(device)
            if ctx is None:
                ctx = cls(device)
                cls._shared[device] = ctx
            return ctx

    def create_mat_vec(self) -> "HipMatVec":
        return HipMatVec(self)


class DeviceQuantMatrix:
    """Packed GGUF weights resident in HBM; close() is idempotent
    (DeviceHalfMatrix.close, DeviceHalfMatrix.java:107-114)."""

    def __init__(self, handle: ctypes.c_void_p, qtype: int, rows: int, cols: int):
        self._h = handle
        self.type = qtype
        self.rows = rows
        self.cols = cols
        self._mu = threading.Lock()

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise IllegalStateException("DeviceQuantMatrix is closed")
        return self._h

    def is_closed(self) -> bool:
        return self._h is None

    def device_pointer(self) -> int:
        p = ctypes.c_void_p()
        _check(_lib.load().jh_qmat_info(self.handle, None, None, None, None, ctypes.byref(p)))
        return p.value

    def nbytes(self) -> int:
        n = ctypes.c_size_t()
        _check(_lib.load().jh_qmat_info(self.handle, None, None, None, ctypes.byref(n), None))
        return n.value

    def packed_bytes(self) -> np.ndarray:
        """The packed GGUF bytes, copied back to the host (the inverse of upload_quant)."""
        import torch  # the HIP runtime torch loaded; device memory plumbing
        n = self.nbytes()
        tmp = torch.empty(n, dtype=torch.uint8, device="cuda")
        hip = ctypes.CDLL("libamdhip64.so.7")  # already loaded by torch (and by libjunohip)
        torch.cuda.synchronize()
        rc = hip.hipMemcpy(ctypes.c_void_p(tmp.data_ptr()), ctypes.c_void_p(self.device_pointer()),
                           ctypes.c_size_t(n), 3)  # hipMemcpyDeviceToDevice
        if rc != 0:
            raise IllegalStateException(f"hipMemcpy failed: rc={rc}")
        return tmp.cpu().numpy()

    def close(self) -> None:
        with self._mu:
            if self._h is not None:
                _lib.load().jh_qmat_free(self._h)
                self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipMatVec:
    """GpuMatVec backend on libjunohip (GpuMatVec.java:38-70)."""

    def __init__(self, ctx: GpuContext):
        if ctx is None:
            raise IllegalArgumentException("ctx must not be null")
        self.ctx = ctx
        self._L = _lib.load()

    def supports_half_resident(self) -> bool:
        # Packed weights are kept resident as-is; the fp16 dequantized copy of
        # the rocBLAS path (RocmMatVec.java:272-329) is not used.
        return False

    # -- MatVec.sgemv(float[] A, float[] x, rows, cols) (MatVec.java:56-66)
    def sgemv(self, A, x, rows: int, cols: int) -> np.ndarray:
        A = np.ascontiguousarray(A, dtype=np.float32).reshape(-1)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if A.size != rows * cols:
            raise IllegalArgumentException(f"A.length={A.size} != rows*cols={rows * cols}")
        if x.size != cols:
            raise IllegalArgumentException(f"x.length={x.size} != cols={cols}")
        y = np.empty(rows, dtype=np.float32)
        if rows == 0:
            return y
        _check(self._L.jh_sgemv(self.ctx.handle, A.ctypes.data, x.ctypes.data, rows, cols, y.ctypes.data))
        return y

    # -- upload of packed bytes, unchanged
    def upload_quant(self, t: QuantizedTensor | int, rows: int, cols: int, data=None) -> DeviceQuantMatrix:
        if isinstance(t, QuantizedTensor):
            qtype, raw = t.type, t.data
            if t.nelems != rows * cols:
                raise IllegalArgumentException(f"nelems={t.nelems} != rows*cols={rows * cols}")
        else:
            qtype, raw = int(t), data
        buf = np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) \
            else np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        h = ctypes.c_void_p()
        _check(self._L.jh_qmat_upload(self.ctx.handle, qtype, buf.ctypes.data, buf.size, rows, cols,
                                      ctypes.byref(h)))
        return DeviceQuantMatrix(h, qtype, rows, cols)

    # -- GpuMatVec.upload(float[] host, rows, cols) (GpuMatVec.java:44-49): fp32 resident
    def upload(self, host, rows: int, cols: int) -> DeviceQuantMatrix:
        host = np.ascontiguousarray(host, dtype=np.float32).reshape(-1)
        if host.size != rows * cols:
            raise IllegalArgumentException(f"host.length={host.size} != rows*cols={rows * cols}")
        return self.upload_quant(F32, rows, cols, host.view(np.uint8))

    def quantize_dev(self, qtype: int, d_src_ptr: int, rows: int, cols: int, stream: int = 0) -> DeviceQuantMatrix:
        """LoraMerge.requantize on the device (LoraMerge.java:226-469)."""
        h = ctypes.c_void_p()
        _check(self._L.jh_qmat_quantize_dev(self.ctx.handle, qtype, d_src_ptr, rows, cols, stream or None,
                                            ctypes.byref(h)))
        return DeviceQuantMatrix(h, qtype, rows, cols)

    def sgemv_quant(self, A: DeviceQuantMatrix, x, row_start: int = 0, row_end: int | None = None) -> np.ndarray:
        if A is None:
            raise IllegalArgumentException("A must not be null")
        if row_end is None:
            row_end = A.rows
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        if x.size != A.cols:
            raise IllegalArgumentException(f"x.length={x.size} != cols={A.cols}")
        y = np.empty(max(row_end - row_start, 0), dtype=np.float32)
        _check(self._L.jh_qmatvec(self.ctx.handle, A.handle, x.ctypes.data, y.ctypes.data, row_start, row_end))
        return y

    def sgemv_batched(self, A: DeviceQuantMatrix, X, row_start: int = 0, row_end: int | None = None) -> np.ndarray:
        if row_end is None:
            row_end = A.rows
        X = np.ascontiguousarray(X, dtype=np.float32)
        if X.ndim != 2 or X.shape[1] != A.cols:
            raise IllegalArgumentException(f"X must be [B][cols={A.cols}], got {X.shape}")
        B = X.shape[0]
        Y = np.empty((B, max(row_end - row_start, 0)), dtype=np.float32)
        _check(self._L.jh_qmatvec_batched(self.ctx.handle, A.handle, X.ctypes.data, B, Y.ctypes.data,
                                          row_start, row_end))
        return Y

    def dequantize(self, A: DeviceQuantMatrix) -> np.ndarray:
        out = np.empty((A.rows, A.cols), dtype=np.float32)
        _check(self._L.jh_qmat_dequant(self.ctx.handle, A.handle, out.ctypes.data))
        return out

    # -- device-pointer forms (operands already in HBM)
    def sgemv_dev(self, A: DeviceQuantMatrix, d_x: int, d_y: int, row_start: int = 0,
                  row_end: int | None = None, stream: int = 0, batch: int = 1) -> None:
        if row_end is None:
            row_end = A.rows
        _check(self._L.jh_qmatvec_batched_dev(A.handle, d_x, batch, d_y, row_start, row_end, stream or None))

    def sgemv_group_dev(self, mats, d_xs, d_ys, stream: int = 0) -> None:
        """Independent full-row GEMVs y_i = W_i x_i in as few launches as possible."""
        n = len(mats)
        if not (len(d_xs) == len(d_ys) == n):
            raise IllegalArgumentException("mats, x and y must have the same length")
        hs = (ctypes.c_void_p * max(n, 1))(*[m.handle for m in mats])
        xs = (ctypes.c_void_p * max(n, 1))(*d_xs)
        ys = (ctypes.c_void_p * max(n, 1))(*d_ys)
        _check(self._L.jh_qmatvec_group_dev(n, hs, xs, ys, stream or None))

    def sgemv_batched_group_dev(self, mats, d_Xs, B: int, d_Ys, stream: int = 0) -> None:
        """Y_i [B][rows_i] = X_i [B][cols] W_i^T for up to 4 matrices sharing cols:
        one launch on the MFMA path (B >= 3), else one batched call per matrix."""
        n = len(mats)
        if not (len(d_Xs) == len(d_Ys) == n):
            raise IllegalArgumentException("mats, X and Y must have the same length")
        hs = (ctypes.c_void_p * max(n, 1))(*[m.handle for m in mats])
        xs = (ctypes.c_void_p * max(n, 1))(*d_Xs)
        ys = (ctypes.c_void_p * max(n, 1))(*d_Ys)
        _check(self._L.jh_qmatvec_batched_group_dev(n, hs, xs, B, ys, stream or None))

    def dequantize_dev(self, A: DeviceQuantMatrix, d_out: int, stream: int = 0) -> None:
        _check(self._L.jh_qmat_dequant_dev(A.handle, d_out, stream or None))


def quantize_dev(qtype: int, d_src: int, n: int, d_dst: int, stream: int = 0) -> None:
    """Raw-pointer quantizer (LoraMerge.requantize on the device)."""
    _check(_lib.load().jh_quantize_dev(qtype, d_src, n, d_dst, stream or None))
