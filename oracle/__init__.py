"""CPU oracle for Juno's quantized matvec path -- TEST INFRASTRUCTURE ONLY.

This package is the checker for the HIP library.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package ``juno_amd`` never does.

It wraps ``oracle/_build/libjuno_oracle.so``, a C restatement of the Java CPU
path (citations per function in ``juno_oracle.c``):

* ``f16_to_f32``      GgufReader.f16ToF32        (GgufReader.java:1248-1271)
* ``f32_to_f16``      LoraMerge.f32ToF16          (LoraMerge.java:589-605)
* ``java_round``      java.lang.Math.round(float)
* ``dequantize``      LlamaTransformerHandler.dequantize* (LlamaTransformerHandler.java:873-1135)
* ``matvec``          LlamaTransformerHandler.matVec(QuantizedTensor, ...)
                      (LlamaTransformerHandler.java:1200-1254, 1428-1638)
* ``quantize``        LoraMerge.requantize        (LoraMerge.java:226-469)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libjuno_oracle.so")

F32, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 8, 10, 11, 12, 13, 14
QK = {F32: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {F32: 4, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}

_lib = None


class LlamaDimsC(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("ffn", ctypes.c_int), ("eps", ctypes.c_float),
                ("theta", ctypes.c_float)]


class LlamaLayerC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "wgate", "wup",
                                                "wdown")] + \
               [(n, ctypes.c_int) for n in ("type_q", "type_k", "type_v", "type_o", "type_gate", "type_up",
                                             "type_down")]


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32_bits.restype = ctypes.c_uint32
        L.or_f16_to_f32_bits.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_java_round.restype = ctypes.c_int32
        L.or_java_round.argtypes = [ctypes.c_float]
        L.or_raw_byte_count.restype = ctypes.c_int64
        L.or_raw_byte_count.argtypes = [ctypes.c_int, ctypes.c_int64]
        L.or_q4k_scale.argtypes = [P, ctypes.c_int]
        L.or_q4k_min.argtypes = [P, ctypes.c_int]
        L.or_q3k_scales.argtypes = [P, P]
        L.or_q3k_scales.restype = None
        L.or_dequantize.argtypes = [ctypes.c_int, P, ctypes.c_int, ctypes.c_int, P]
        L.or_matvec.argtypes = [ctypes.c_int, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                P, ctypes.c_int]
        L.or_quantize.argtypes = [ctypes.c_int, P, ctypes.c_int64, P]
        I, F = ctypes.c_int, ctypes.c_float
        L.or_rmsnorm.argtypes = [P, P, I, F, P]
        L.or_rope.argtypes = [P, I, I, I, F]
        L.or_softmax.argtypes = [P, I]
        L.or_gqa.argtypes = [P, P, P, I, I, I, I, P]
        L.or_silu.argtypes = [F]
        L.or_silu.restype = F
        L.or_silu_mul.argtypes = [P, P, I, P]
        L.or_add.argtypes = [P, P, I, P]
        L.or_lora_forward.argtypes = [P, P, I, I, I, ctypes.c_float, P, P]
        L.or_lora_forward.restype = None
        L.or_llama_layer.argtypes = [ctypes.POINTER(LlamaLayerC), ctypes.POINTER(LlamaDimsC), P, I, P, P, I]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def f16_to_f32(bits: int) -> float:
    return lib().or_f16_to_f32(bits & 0xFFFF)


def f32_to_f16(v: float) -> int:
    return lib().or_f32_to_f16(v)


def java_round(v: float) -> int:
    return lib().or_java_round(v)


def raw_byte_count(qtype: int, nelems: int) -> int:
    return lib().or_raw_byte_count(qtype, nelems)


def q4k_scale(sc: bytes, j: int) -> int:
    b = np.frombuffer(bytes(sc), dtype=np.uint8).copy()
    return lib().or_q4k_scale(_ptr(b), j)


def q4k_min(sc: bytes, j: int) -> int:
    b = np.frombuffer(bytes(sc), dtype=np.uint8).copy()
    return lib().or_q4k_min(_ptr(b), j)


def q3k_scales(sc12: bytes) -> list:
    """The 16 signed Q3_K sub-block scales of a 12-byte field."""
    b = np.frombuffer(bytes(sc12), dtype=np.uint8).copy()
    out = np.zeros(16, dtype=np.int32)
    lib().or_q3k_scales(_ptr(b), _ptr(out))
    return out.tolist()


def _as_u8(raw) -> np.ndarray:
    if isinstance(raw, (bytes, bytearray, memoryview)):
        return np.frombuffer(bytes(raw), dtype=np.uint8)
    return np.ascontiguousarray(raw, dtype=np.uint8)


def dequantize(qtype: int, raw, rows: int, cols: int) -> np.ndarray:
    raw = _as_u8(raw)
    if raw.size != raw_byte_count(qtype, rows * cols):
        raise ValueError("raw size does not match rows*cols")
    out = np.empty(rows * cols, dtype=np.float32)
    if lib().or_dequantize(qtype, _ptr(raw), rows, cols, _ptr(out)) != 0:
        raise ValueError(f"dequantize: unsupported type {qtype} or cols {cols}")
    return out.reshape(rows, cols)


def matvec(qtype: int, raw, x: np.ndarray, row_start: int, row_end: int, cols: int,
           nthreads: int = 0) -> np.ndarray:
    raw = _as_u8(raw)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size != cols:
        raise ValueError("x.length != cols")
    pitch = cols // QK[qtype] * BLOCK_BYTES[qtype]
    if row_end * pitch > raw.size:
        raise ValueError("row range exceeds the tensor")
    y = np.empty(row_end - row_start, dtype=np.float32)
    if lib().or_matvec(qtype, _ptr(raw), _ptr(x), row_start, row_end, cols, _ptr(y), nthreads) != 0:
        raise ValueError(f"matvec: unsupported type {qtype} or cols {cols}")
    return y


def quantize(qtype: int, data: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
    n = data.size
    if n % QK[qtype]:
        raise ValueError("n is not a block multiple")
    out = np.zeros(raw_byte_count(qtype, n), dtype=np.uint8)
    if lib().or_quantize(qtype, _ptr(data), n, _ptr(out)) != 0:
        raise ValueError(f"quantize: unsupported type {qtype}")
    return out


# ---------------------------------------------------------------- decode step (juno_oracle_decode.c)

def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().or_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


def rope(x, pos: int, n_heads: int, head_dim: int, theta: float) -> np.ndarray:
    """Returns a rotated copy (the reference rotates in place)."""
    y = _f32(x).copy()
    lib().or_rope(_ptr(y), pos, n_heads, head_dim, theta)
    return y


def softmax(s) -> np.ndarray:
    y = _f32(s).copy()
    lib().or_softmax(_ptr(y), y.size)
    return y


def gqa(q, k_cache, v_cache, n_heads: int, n_kv_heads: int, head_dim: int, seq_len: int) -> np.ndarray:
    q, k_cache, v_cache = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.empty(n_heads * head_dim, dtype=np.float32)
    lib().or_gqa(_ptr(q), _ptr(k_cache), _ptr(v_cache), n_heads, n_kv_heads, head_dim, seq_len, _ptr(out))
    return out


def silu(x: float) -> float:
    return lib().or_silu(x)


def silu_mul(gate, up) -> np.ndarray:
    gate, up = _f32(gate), _f32(up)
    out = np.empty_like(gate)
    lib().or_silu_mul(_ptr(gate), _ptr(up), gate.size, _ptr(out))
    return out


def lora_forward(a, b, rank: int, in_dim: int, out_dim: int, scale: float, x) -> np.ndarray:
    """LoraAdapter.forward: (B (A x)) * scale in the reference's summation order."""
    a, b, x = _f32(a), _f32(b), _f32(x)
    if a.size != rank * in_dim or b.size != out_dim * rank or x.size != in_dim or rank > 4096:
        raise ValueError("lora_forward: shape mismatch")
    out = np.empty(out_dim, dtype=np.float32)
    lib().or_lora_forward(_ptr(a), _ptr(b), rank, in_dim, out_dim, scale, _ptr(x), _ptr(out))
    return out


def add(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().or_add(_ptr(a), _ptr(b), a.size, _ptr(out))
    return out


def llama_layer(layer: dict, dims: dict, x, pos: int, k_cache: np.ndarray, v_cache: np.ndarray,
                nthreads: int = 0) -> np.ndarray:
    """One transformerLayer; k_cache / v_cache (float32, [>= pos+1, kv_dim]) receive
    this position's k and v in place.  layer holds 'attn_norm', 'ffn_norm' (float32)
    and per matrix m in q,k,v,o,gate,up,down: 'w'+m packed bytes and 'type_'+m."""
    keep = {}
    def buf(a, dt):
        arr = np.ascontiguousarray(a, dtype=dt)
        keep[id(arr)] = arr
        return _ptr(arr)
    L = LlamaLayerC(attn_norm=buf(layer["attn_norm"], np.float32), ffn_norm=buf(layer["ffn_norm"], np.float32),
                    **{"w" + m: buf(layer["w" + m], np.uint8) for m in ("q", "k", "v", "o", "gate", "up", "down")},
                    **{"type_" + m: layer["type_" + m] for m in ("q", "k", "v", "o", "gate", "up", "down")})
    D = LlamaDimsC(**dims)
    y = _f32(x).copy()
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    if lib().or_llama_layer(ctypes.byref(L), ctypes.byref(D), _ptr(y), pos, _ptr(k_cache), _ptr(v_cache),
                            nthreads) != 0:
        raise ValueError("llama_layer: unsupported matrix type")
    return y
