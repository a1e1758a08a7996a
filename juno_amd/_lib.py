"""ctypes binding of libjunohip.so (the C ABI declared in include/junohip.h).

The library is built in-tree (``python -m juno_amd.build``) and loaded from
this package directory.  There is no fallback: if the library is missing,
loading raises ``ImportError``.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# JUNO_LIB_PATH: another build of the library (juno_amd/timeline.py's instrumented variant)
LIB_PATH = os.environ.get("JUNO_LIB_PATH", os.path.join(HERE, "libjunohip.so"))

JH_OK, JH_EINVAL, JH_ENOMEM, JH_EHIP, JH_EUNSUPPORTED, JH_ECLOSED, JH_ENODEV, JH_EFORMAT, JH_EIO = range(9)

# Every symbol include/junohip.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
SIGNATURES = {
    "jh_last_error": (ctypes.c_char_p, []),
    "jh_version": (ctypes.c_char_p, []),
    "jh_device_count": (_I, [ctypes.POINTER(_I)]),
    "jh_device_info": (_I, [_I, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_char_p]),
    "jh_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "jh_ctx_destroy": (_I, [_P]),
    "jh_raw_byte_count": (_I, [_I, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "jh_qmat_upload": (_I, [_P, _I, _P, ctypes.c_size_t, _I, _I, ctypes.POINTER(_P)]),
    "jh_qmat_quantize_dev": (_I, [_P, _I, _P, _I, _I, _P, ctypes.POINTER(_P)]),
    "jh_qmat_free": (_I, [_P]),
    "jh_qmat_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
                          ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(_P)]),
    "jh_qmatvec": (_I, [_P, _P, _P, _P, _I, _I]),
    "jh_qmatvec_batched": (_I, [_P, _P, _P, _I, _P, _I, _I]),
    "jh_qmat_dequant": (_I, [_P, _P, _P]),
    "jh_sgemv": (_I, [_P, _P, _P, _I, _I, _P]),
    "jh_qmatvec_dev": (_I, [_P, _P, _P, _I, _I, _P]),
    "jh_qmatvec_batched_dev": (_I, [_P, _P, _I, _P, _I, _I, _P]),
    "jh_qmat_dequant_dev": (_I, [_P, _P, _P]),
    "jh_qmatvec_batched_noalloc_dev": (_I, [_P, _P, _I, _P, _I, _I, _P]),
    "jh_qmatvec_group_dev": (_I, [_I, _P, _P, _P, _P]),
    "jh_sync_faults": (_I, [_I, _P]),
    "jh_debug_timeline": (_I, [_I, _I, _P, ctypes.c_size_t]),
    "jh_qmatvec_batched_plan_shape": (_I, [_I, _I, _I, _I, _I, _P, _P]),
    "jh_qmatvec_batched_group_dev": (_I, [_I, _P, _P, _I, _P, _P]),
    "jh_qmatvec_swiglu_dev": (_I, [_P, _P, _P, _P, _P]),
    "jh_rmsnorm_qmatvec_swiglu_dev": (_I, [_P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P]),
    "jh_rmsnorm_qmatvec_dev": (_I, [_P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P]),
    "jh_rmsnorm_qmatvec_group_dev": (_I, [_I, _P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _P]),
    "jh_qmatvec_batched_swiglu_dev": (_I, [_P, _P, _P, _I, _P, _P, _P, _P]),
    "jh_qmatvec_batched_plan": (_I, [_I, _P, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "jh_stream_workspace_info": (_I, [_I, _P, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(_P)]),
    "jh_quantize_dev": (_I, [_I, _P, ctypes.c_int64, _P, _P]),
    "jh_rmsnorm_dev": (_I, [_P, _P, _P, _I, ctypes.c_float, _P, _P, _P]),
    "jh_rope_kv_dev": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, ctypes.c_float, _P, _P, _P]),
    "jh_attention_dev": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, _P, _P]),
    "jh_rope_attention_dev": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, ctypes.c_float, _P, _P, _P, _P]),
    "jh_rope_attention_qmatvec_dev": (_I, [_P, _P, _P, _I, _I, _I, _P, _I, ctypes.c_float, _P, _P, _P, _P, _P, _P]),
    "jh_silu_mul_dev": (_I, [_P, _P, _I, _P, _P]),
    "jh_pos_increment_dev": (_I, [_P, _I, _P]),
    "jh_embed_dev": (_I, [_P, _P, _P, _P]),
    "jh_embed_rows_dev": (_I, [_P, _P, _I, _P, _P]),
    "jh_add_rows_dev": (_I, [_P, _P, _I, _I, _P]),
    "jh_lora_apply_dev": (_I, [_P, _P, _I, _I, _I, ctypes.c_float, _P, _I, _P, _P]),
    "jh_rmsnorm_rows_dev": (_I, [_P, _P, _P, _I, _I, ctypes.c_float, _P, _P, _P]),
    "jh_rope_attention_batched_dev": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _I, ctypes.c_float, _P, _P, _P,
                                           _P]),
    "jh_gguf_open": (_I, [ctypes.c_char_p, _P]),
    "jh_gguf_close": (_I, [_P]),
    "jh_gguf_info": (_I, [_P, _P, _P, _P, _P, _P, _P]),
    "jh_gguf_meta_type": (_I, [_P, ctypes.c_char_p, _P, _P, _P]),
    "jh_gguf_meta_number": (_I, [_P, ctypes.c_char_p, _P, _P, _P]),
    "jh_gguf_meta_bool": (_I, [_P, ctypes.c_char_p, _P, _P]),
    "jh_gguf_meta_string": (_I, [_P, ctypes.c_char_p, _P, ctypes.c_size_t, _P]),
    "jh_gguf_tensor_index": (_I, [_P, ctypes.c_char_p, _P]),
    "jh_gguf_tensor_info": (_I, [_P, ctypes.c_int64, _P, _P, _P, _P, _P, _P]),
    "jh_gguf_tensor_read": (_I, [_P, ctypes.c_int64, _P, ctypes.c_size_t, _P]),
    "jh_gguf_upload": (_I, [_P, _P, ctypes.c_int64, _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libjunohip.so and declare its signatures; raise if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run `python -m juno_amd.build` "
                              "(the HIP library has no CPU fallback)")
        # PyTorch-ROCm ships its own libamdhip64.so (soname libamdhip64.so.7)
        # and its libraries request it by the unversioned name.  Loading torch
        # first makes this library bind to that same runtime (same soname), so
        # one process never holds two HIP runtimes.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        check_fresh(L)
        _lib = L
    return _lib


def check_fresh(L) -> None:
    """Refuse a library built from other sources than the tree's (jh_version
    carries the hash build.py computed over csrc/ and include/).
    JUNO_ALLOW_STALE_LIB=1 skips the check (A/B runs of saved builds)."""
    from . import build as _build
    got = L.jh_version().decode()
    want = _build.source_hash()
    if os.environ.get("JUNO_ALLOW_STALE_LIB") == "1" or got.endswith("src:" + want):
        return
    raise ImportError(f"{LIB_PATH} is stale ({got}); the sources hash to {want}: "
                      "rebuild with `python -m juno_amd.build`")


def last_error() -> str:
    return load().jh_last_error().decode("utf-8", "replace")
