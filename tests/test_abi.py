"""CPU-side checks of the C ABI: the library loads, exports every symbol that
include/junohip.h declares, and fails cleanly when no GPU is present.  No
compute calls are made here."""
import ctypes
import os
import re
import subprocess

import pytest

from juno_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "junohip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_the_binding_knows():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    for name in header_functions():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\sT\s(jh_[a-z0-9_]+)", out))
    assert set(header_functions()) <= exported


def test_library_has_gfx950_code_object():
    out = subprocess.run(["readelf", "-S", _lib.LIB_PATH], capture_output=True, text=True)
    assert ".hip_fatbin" in out.stdout
    # the offload bundle id of our own build names the target
    assert b"amdgcn-amd-amdhsa--gfx950" in open(_lib.LIB_PATH, "rb").read()


def test_version_and_last_error_without_gpu():
    L = _lib.load()
    assert L.jh_version().decode().startswith("junohip")
    assert isinstance(L.jh_last_error(), bytes)


def test_library_matches_its_sources(monkeypatch):
    """The loaded library carries the hash of the sources it was built from, and
    a library from other sources is refused (unless JUNO_ALLOW_STALE_LIB=1)."""
    from juno_amd import build
    L = _lib.load()
    assert L.jh_version().decode().endswith("src:" + build.source_hash())

    class Old:
        @staticmethod
        def jh_version():
            return b"junohip 0.1 gfx950 src:0000000000000000"

    monkeypatch.delenv("JUNO_ALLOW_STALE_LIB", raising=False)
    with pytest.raises(ImportError, match="stale"):
        _lib.check_fresh(Old)
    monkeypatch.setenv("JUNO_ALLOW_STALE_LIB", "1")
    _lib.check_fresh(Old)


def test_raw_byte_count_matches_reference_formula():
    L = _lib.load()
    out = ctypes.c_int64()
    # GgufReader.rawByteCount (GgufReader.java:347-360)
    for t, n, want in [(12, 256 * 32, 32 * 144), (14, 256, 210), (8, 32, 34), (0, 10, 40), (10, 256, 84),
                       (11, 512, 220), (13, 256, 176)]:
        assert L.jh_raw_byte_count(t, n, ctypes.byref(out)) == 0
        assert out.value == want
    assert L.jh_raw_byte_count(99, 256, ctypes.byref(out)) == _lib.JH_EUNSUPPORTED
    assert "GGML type 99" in _lib.last_error()


def test_ctx_create_without_device_reports_enodev():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = _lib.load()
    h = ctypes.c_void_p()
    rc = L.jh_ctx_create(0, ctypes.byref(h))
    assert rc in (_lib.JH_ENODEV, _lib.JH_EINVAL)
    assert _lib.last_error()


def test_null_matrix_is_illegal_argument():
    from juno_amd import matvec as mv
    L = _lib.load()
    rc = L.jh_qmatvec_dev(None, None, None, 0, 0, None)
    assert rc == _lib.JH_EINVAL
    assert "must not be null" in _lib.last_error()
    with pytest.raises(mv.IllegalArgumentException):
        mv._check(rc)


def test_batched_group_argument_checks_without_gpu():
    """jh_qmatvec_batched_group_dev rejects a bad group before any device call:
    more than 4 matrices, negative B, null arrays or a null matrix; n = 0 and
    B = 0 are no-ops."""
    L = _lib.load()
    V = ctypes.c_void_p
    arr = (V * 5)()
    assert L.jh_qmatvec_batched_group_dev(5, arr, arr, 32, arr, None) == _lib.JH_EINVAL
    assert "outside [0, 4]" in _lib.last_error()
    assert L.jh_qmatvec_batched_group_dev(1, arr, arr, -1, arr, None) == _lib.JH_EINVAL
    assert L.jh_qmatvec_batched_group_dev(1, None, arr, 32, arr, None) == _lib.JH_EINVAL
    assert L.jh_qmatvec_batched_group_dev(1, arr, arr, 32, arr, None) == _lib.JH_EINVAL  # null matrix
    assert "must not be null" in _lib.last_error()
    assert L.jh_qmatvec_batched_group_dev(0, None, None, 32, None, None) == _lib.JH_OK
    assert L.jh_qmatvec_batched_group_dev(1, arr, arr, 0, arr, None) == _lib.JH_OK


def test_oracle_is_not_imported_by_the_product():
    for dirpath, _, files in os.walk(os.path.join(ROOT, "juno_amd")):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "juno_oracle" not in text, f
