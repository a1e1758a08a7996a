"""Output projections at full size, and the prepared-x MFMA kernel.

outputProjection (LlamaTransformerHandler.java:803-810) multiplies the final
norm output by the vocabulary matrix: the largest GEMV of a step.  At B <= 32
a single matrix with enough 256-row tiles to fill the GPU without splitting K
takes the prepared-x kernel (x_prep + mfma_px); these tests reach it at the
Llama-3-8B lm_head shape (128256 x 4096 Q6_K), at B = 1, 16, 32, and for every
format the kernel supports at 33024 x 2048 (129 row tiles, the smallest count
that keeps K unsplit at 2048 columns) with a row sub-range.  The Phi-3-mini
lm_head (32064 x 3072, Q8_0 and Q6_K) is checked at B = 1 and 32.

Weights are N(0, 0.02) drawn on the device and quantized there with the
LoraMerge quantizers (bit-exact with the oracle's, tests/test_gpu_parity.py);
the packed bytes are read back and the oracle runs on them.  B = 1: every row
against the oracle.  B > 1: for every batch column, 640 sampled rows (the first
and last row tiles and 128 random rows) against the oracle.  Bar: the GEMV
tolerance, max rel-err 1e-3 with eps_r = 1e-3 * sum_c |w_rc x_c|; the plain
relative error (no eps floor) is printed alongside.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    return mv.GpuContext.shared(0).create_mat_vec()


def device_matrix(be, qtype, rows, cols, seed, outliers=False):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
    if outliers:  # 1 % of the entries at 10x (seeded choice)
        idx = torch.randperm(rows * cols, generator=g, device="cuda")[: rows * cols // 100]
        w[idx] *= 10
    m = be.quantize_dev(qtype, w.data_ptr(), rows, cols, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    del w
    return m


def plan(L, dev, B):
    hs = (ctypes.c_void_p * 1)(dev.handle)
    kernel, ksplit = ctypes.c_int(), ctypes.c_int()
    assert L.jh_qmatvec_batched_plan(1, hs, B, ctypes.byref(kernel), ctypes.byref(ksplit)) == 0, _lib.last_error()
    return kernel.value, ksplit.value


def check_rows(qtype, raw, rows, cols, X, Y, row_start, sample, label):
    """Y[j][i] is row row_start + i; compare the rows `sample` (indices into
    Y's row axis) of every batch column against the oracle, 8192 rows at a
    time."""
    pitch = raw.size // rows
    worst, worst_plain = 0.0, 0.0
    for c0 in range(0, len(sample), 8192):
        part = sample[c0:c0 + 8192]
        sub = np.ascontiguousarray(raw.reshape(rows, pitch)[row_start + part]).reshape(-1)
        adeq = np.abs(O.dequantize(qtype, sub, len(part), cols).astype(np.float64))
        for j in range(X.shape[0]):
            ref = O.matvec(qtype, sub, X[j], 0, len(part), cols, nthreads=16).astype(np.float64)
            y = Y[j][part].astype(np.float64)
            scale = adeq @ np.abs(X[j].astype(np.float64))
            err = np.abs(y - ref)
            worst = max(worst, float((err / np.maximum(np.abs(ref), 1e-3 * scale)).max()))
            worst_plain = max(worst_plain, float((err / np.maximum(np.abs(ref), 1e-30)).max()))
    say(f"{label}: max rel-err {worst:.2e} (plain, no eps floor: {worst_plain:.2e})")
    assert worst <= TOL, label


def run(be, dev, qtype, rows, cols, B, row_start, row_end, seed):
    import torch
    L = _lib.load()
    X = np.random.default_rng(seed).standard_normal((B, cols)).astype(np.float32)
    dx = torch.from_numpy(X).cuda()
    dy = torch.full((B, row_end - row_start), float("nan"), device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    rc = L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B, ctypes.c_void_p(dy.data_ptr()),
                                  row_start, row_end, ctypes.c_void_p(s))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return X, dy.cpu().numpy()


def sample_rows(n, seed):
    rng = np.random.default_rng(seed)
    picks = np.concatenate([np.arange(min(256, n)), np.arange(max(0, n - 256), n), rng.integers(0, n, 128)])
    return np.unique(picks)


def test_llama8b_lm_head_q6k(be):
    """128256 x 4096 Q6_K: B = 1 (staged kernel) on every row; B = 16 and 32 on
    the prepared-x kernel, which the plan must choose."""
    L = _lib.load()
    rows, cols, qt = 128256, 4096, O.Q6_K
    say("lm_head 8B: quantize on device")
    dev = device_matrix(be, qt, rows, cols, 1201)
    try:
        raw = dev.packed_bytes()
        say("lm_head 8B: B=1, all rows")
        X, Y = run(be, dev, qt, rows, cols, 1, 0, rows, 1202)
        assert np.isfinite(Y).all()
        check_rows(qt, raw, rows, cols, X, Y, 0, np.arange(rows), "8B lm_head Q6_K B=1 all rows")
        for B in (16, 32):
            kernel, ksplit = plan(L, dev, B)
            assert (kernel, ksplit) == (2, 1), (B, kernel, ksplit)
            say(f"lm_head 8B: B={B} prepared-x kernel")
            X, Y = run(be, dev, qt, rows, cols, B, 0, rows, 1203 + B)
            assert np.isfinite(Y).all()
            check_rows(qt, raw, rows, cols, X, Y, 0, sample_rows(rows, B), f"8B lm_head Q6_K B={B}")
    finally:
        dev.close()


@pytest.mark.parametrize("qt", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0])
def test_prepared_x_kernel_all_formats(be, qt):
    """33024 x 2048 (129 row tiles): the prepared-x kernel at B = 3, 16, 32 for
    every format it supports, over the full rows and over the sub-range
    [100, 32987) (still 129 tiles; the tile rows start mid-matrix)."""
    L = _lib.load()
    rows, cols = 33024, 2048
    dev = device_matrix(be, qt, rows, cols, 1300 + qt, outliers=True)
    try:
        raw = dev.packed_bytes()
        for B in (3, 16, 32):
            kernel, ksplit = plan(L, dev, B)
            assert (kernel, ksplit) == (2, 1), (qt, B, kernel, ksplit)
            for r0, r1 in ((0, rows), (100, rows - 37)):
                say(f"prepared-x type {qt} B={B} rows [{r0}, {r1})")
                X, Y = run(be, dev, qt, rows, cols, B, r0, r1, 1310 + B + r0)
                assert np.isfinite(Y).all()
                check_rows(qt, raw, rows, cols, X, Y, r0, sample_rows(r1 - r0, B + r0),
                           f"type {qt} 33024x2048 B={B} [{r0},{r1})")
    finally:
        dev.close()


@pytest.mark.parametrize("qt", [O.Q8_0, O.Q6_K])
def test_phi3_lm_head(be, qt):
    """Phi-3-mini vocabulary projection 32064 x 3072 with 1 % outliers at 10x:
    B = 1 on every row, B = 32 on sampled rows (whatever kernel the plan takes,
    printed)."""
    L = _lib.load()
    rows, cols = 32064, 3072
    dev = device_matrix(be, qt, rows, cols, 1400 + qt, outliers=True)
    try:
        raw = dev.packed_bytes()
        say(f"phi3 lm_head type {qt} B=1")
        X, Y = run(be, dev, qt, rows, cols, 1, 0, rows, 1401)
        check_rows(qt, raw, rows, cols, X, Y, 0, np.arange(rows), f"Phi-3 lm_head type {qt} B=1 all rows")
        kernel, ksplit = plan(L, dev, 32)
        say(f"phi3 lm_head type {qt} B=32: kernel {kernel}, ksplit {ksplit}")
        assert kernel in (1, 2)
        X, Y = run(be, dev, qt, rows, cols, 32, 0, rows, 1402)
        assert np.isfinite(Y).all()
        check_rows(qt, raw, rows, cols, X, Y, 0, sample_rows(rows, 32), f"Phi-3 lm_head type {qt} B=32")
    finally:
        dev.close()
