"""jh_qmatvec_batched_noalloc_dev: the batched GEMV with its scratch in a
library-static device array instead of an allocated workspace.

Checked against jh_qmatvec_batched_dev (the same kernels, so bit for bit) and
against the oracle (the GEMV bar, max rel-err 1e-3), on two calls in a row
with the second one smaller, over the split-K, prepared-x and no-scratch
paths; an oversized call is refused with JH_EINVAL; and in a fresh process
whose library allocations are made to fail after the uploads, the entry point
still works while the allocating one reports hipMalloc.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL = 1e-3


def say(*a):
    print(*a, flush=True)


def rel_err(y, ref, deq, x):
    scale = np.abs(deq.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)


def quantized(qtype, rows, cols, seed):
    w = (np.random.default_rng(seed).standard_normal(rows * cols) * 0.02).astype(np.float32)
    return O.quantize(qtype, w)


def plan(L, dev, B):
    hs = (ctypes.c_void_p * 1)(dev.handle)
    kernel, ksplit = ctypes.c_int(), ctypes.c_int()
    assert L.jh_qmatvec_batched_plan(1, hs, B, ctypes.byref(kernel), ctypes.byref(ksplit)) == 0
    return kernel.value, ksplit.value


# (type, rows, cols, B): split-K MFMA, then a smaller prepared-x MFMA call, then
# the scratch-free B = 1 and B = 2 kernels
CASES = [(O.Q4_K, 4096, 4096, 32), (O.Q6_K, 33024, 2048, 16), (O.Q8_0, 512, 2048, 2), (O.Q4_K, 1024, 2048, 1)]


def test_noalloc_matches_allocating_entry_point():
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    s = torch.cuda.Stream()
    S = ctypes.c_void_p(s.cuda_stream)
    for i, (qt, rows, cols, B) in enumerate(CASES):
        raw = quantized(qt, rows, cols, 1600 + i)
        with be.upload_quant(mv.QuantizedTensor("w", qt, rows * cols, raw.tobytes()), rows, cols) as dev:
            say(f"noalloc case {i}: type {qt} {rows}x{cols} B={B} plan {plan(L, dev, B)}")
            X = np.random.default_rng(1700 + i).standard_normal((B, cols)).astype(np.float32)
            dx = torch.from_numpy(X).cuda()
            y0 = torch.full((B, rows), float("nan"), device="cuda")
            y1 = torch.full((B, rows), float("nan"), device="cuda")
            with torch.cuda.stream(s):
                rc = L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B,
                                              ctypes.c_void_p(y0.data_ptr()), 0, rows, S)
                assert rc == 0, _lib.last_error()
                rc = L.jh_qmatvec_batched_noalloc_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B,
                                                      ctypes.c_void_p(y1.data_ptr()), 0, rows, S)
                assert rc == 0, _lib.last_error()
            s.synchronize()
            a, b = y0.cpu().numpy(), y1.cpu().numpy()
            assert np.array_equal(a, b), i
            deq = O.dequantize(qt, raw, rows, cols)
            for j in sorted({0, B - 1}):
                ref = O.matvec(qt, raw, X[j], 0, rows, cols, nthreads=16).astype(np.float64)
                assert rel_err(b[j], ref, deq, X[j]).max() <= TOL, (i, j)


def test_noalloc_refuses_oversized_call():
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    rows, cols, B = 14336, 4096, 64  # split K four ways: 4 * 64 * 14336 * 4 bytes of partials > 8 MiB
    raw = quantized(O.Q4_K, rows, cols, 1650)
    with be.upload_quant(mv.QuantizedTensor("w", O.Q4_K, rows * cols, raw.tobytes()), rows, cols) as dev:
        dx = torch.zeros(B, cols, device="cuda")
        dy = torch.zeros(B, rows, device="cuda")
        rc = L.jh_qmatvec_batched_noalloc_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B,
                                              ctypes.c_void_p(dy.data_ptr()), 0, rows, None)
        msg = _lib.last_error()
        say("oversized:", msg)
        assert rc == _lib.JH_EINVAL
        assert "static scratch" in msg
        torch.cuda.synchronize()


CHILD = r"""
import ctypes, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import torch
import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv
L = _lib.load()
be = mv.GpuContext.shared(0).create_mat_vec()
rows, cols, B = 2048, 4096, 32
w = (np.random.default_rng(5).standard_normal(rows * cols) * 0.02).astype(np.float32)
raw = O.quantize(O.Q4_K, w)
dev = be.upload_quant(mv.QuantizedTensor("w", O.Q4_K, rows * cols, raw.tobytes()), rows, cols)  # allocation 1
X = np.random.default_rng(6).standard_normal((B, cols)).astype(np.float32)
dx = torch.from_numpy(X).cuda()
dy = torch.zeros(B, rows, device="cuda")
s = torch.cuda.Stream()
S = ctypes.c_void_p(s.cuda_stream)
for _ in range(2):
    rc = L.jh_qmatvec_batched_noalloc_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B, ctypes.c_void_p(dy.data_ptr()), 0, rows, S)
    assert rc == 0, _lib.last_error()
s.synchronize()
y = dy.cpu().numpy()
ref = O.matvec(O.Q4_K, raw, X[B - 1], 0, rows, cols).astype(np.float64)
deq = O.dequantize(O.Q4_K, raw, rows, cols).astype(np.float64)
scale = np.abs(deq) @ np.abs(X[B - 1].astype(np.float64))
assert (np.abs(y[B - 1] - ref) / np.maximum(np.abs(ref), 1e-3 * scale)).max() <= 1e-3
rc = L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B, ctypes.c_void_p(dy.data_ptr()), 0, rows, S)
assert rc == _lib.JH_ENOMEM and "hipMalloc" in _lib.last_error(), (rc, _lib.last_error())
print("CHILD_OK", flush=True)
"""


def test_noalloc_makes_no_device_allocation():
    """A fresh process in which every library allocation after the first (the
    matrix upload) fails: the no-allocation entry point still computes the
    right result twice, while the allocating entry point fails with hipMalloc."""
    env = dict(os.environ, JUNO_HIP_FAIL_ALLOC_AFTER="1")
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], env=env, capture_output=True, text=True, timeout=300)
    say(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "CHILD_OK" in r.stdout
