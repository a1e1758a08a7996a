"""Seeded random sweep of the GEMV entry points against the CPU oracle: formats
Q4_K / Q5_K / Q6_K / Q8_0 / Q2_K / Q3_K, random shapes (K-quants: 1-40 super-
blocks per row; Q8_0: 1-200 blocks), random row ranges, B drawn from 1-64 (so
the one-shot, staged and MFMA kernels and their K splits all take turns), and
x at random scales with a few spikes.  Grouped launches of 2-4 same-K matrices
with random row counts go through jh_qmatvec_batched_group_dev.  Bar: the
parity suite's per-row metric, max rel-err 1e-3 with eps_r = 1e-3 sum_c |w_rc x_c|.

The staged kernel is taken for large matrices only; a child process with
JUNO_STAGED_R=1 runs the B = 1 cases through it at every size.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle as O
from juno_amd import matvec as mv

pytestmark = pytest.mark.gpu

TOL = 1e-3
QTYPES = [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0, O.Q2_K, O.Q3_K]
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def raw_matrix(qtype, rows, cols, rng):
    if qtype in (O.Q2_K, O.Q3_K):  # no quantizer in the reference for these: random blocks, small d
        from test_oracle_q2q3 import random_blocks
        return random_blocks(qtype, rows, cols, int(rng.integers(1 << 30)))
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    idx = rng.choice(w.size, max(w.size // 200, 1), replace=False)
    w[idx] *= 10
    return O.quantize(qtype, w)


def x_batch(B, cols, rng):
    X = rng.standard_normal((B, cols)).astype(np.float32)
    X *= np.float32(10.0 ** rng.uniform(-3, 2))
    X[:, rng.choice(cols, max(cols // 100, 1), replace=False)] *= 25
    return X


def check(qtype, raw, rows, cols, a, b, X, Y):
    deq = O.dequantize(qtype, raw, rows, cols).astype(np.float64)[a:b]
    worst = 0.0
    for j in range(X.shape[0]):
        ref = O.matvec(qtype, raw, X[j], a, b, cols, nthreads=16).astype(np.float64)
        scale = np.abs(deq) @ np.abs(X[j].astype(np.float64))
        err = np.abs(Y[j].astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)
        worst = max(worst, float(err.max()) if err.size else 0.0)
    return worst


def shape(qtype, rng):
    if qtype == O.Q8_0:
        return int(rng.integers(1, 3000)), 32 * int(rng.integers(1, 201))
    return int(rng.integers(1, 3000)), 256 * int(rng.integers(1, 41))


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_and_batches(seed):
    be = mv.GpuContext.shared(0).create_mat_vec()
    rng = np.random.default_rng(9000 + seed)
    for case in range(8):
        qtype = QTYPES[int(rng.integers(len(QTYPES)))]
        rows, cols = shape(qtype, rng)
        B = int(rng.choice([1, 1, 2, 3, 5, 8, 13, 16, 21, 31, 32, 33, 47, 64]))
        a = int(rng.integers(0, rows))
        b = int(rng.integers(a + 1, rows + 1))
        if rows * cols * B > 40_000_000:  # keep the oracle to seconds
            B = max(1, 40_000_000 // (rows * cols))
        raw = raw_matrix(qtype, rows, cols, rng)
        X = x_batch(B, cols, rng)
        print(f"seed {seed} case {case}: type {qtype} {rows}x{cols} rows [{a},{b}) B={B}", flush=True)
        with be.upload_quant(mv.QuantizedTensor("w", qtype, rows * cols, raw.tobytes()), rows, cols) as dev:
            Y = be.sgemv_batched(dev, X, a, b) if B > 1 else be.sgemv_quant(dev, X[0], a, b)[None, :]
        assert Y.shape == (B, b - a)
        worst = check(qtype, raw, rows, cols, a, b, X, Y)
        assert worst <= TOL, (seed, case, qtype, rows, cols, a, b, B, worst)


@pytest.mark.parametrize("seed", range(4))
def test_random_groups(seed):
    import ctypes

    import torch
    be = mv.GpuContext.shared(0).create_mat_vec()
    rng = np.random.default_rng(9100 + seed)
    for case in range(3):
        qtype = [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0][int(rng.integers(4))]
        cols = 256 * int(rng.integers(1, 17))
        n = int(rng.integers(2, 5))
        rows = [int(rng.integers(1, 2500)) for _ in range(n)]
        B = int(rng.choice([2, 3, 8, 16, 32, 40, 64]))
        print(f"group seed {seed} case {case}: type {qtype} cols {cols} rows {rows} B={B}", flush=True)
        raws = [raw_matrix(qtype, r, cols, rng) for r in rows]
        Xs = [x_batch(B, cols, rng) for _ in range(n)]
        mats = [be.upload_quant(mv.QuantizedTensor("w", qtype, r * cols, raw.tobytes()), r, cols)
                for r, raw in zip(rows, raws)]
        try:
            dX = [torch.from_numpy(X).cuda() for X in Xs]
            dY = [torch.full((B, r), float("nan"), device="cuda") for r in rows]
            be.sgemv_batched_group_dev(mats, [x.data_ptr() for x in dX], B, [y.data_ptr() for y in dY])
            torch.cuda.synchronize()
            for r, raw, X, y in zip(rows, raws, Xs, dY):
                worst = check(qtype, raw, r, cols, 0, r, X, y.cpu().numpy())
                assert worst <= TOL, (seed, case, qtype, r, cols, B, worst)
        finally:
            for m in mats:
                m.close()


STAGED_CHILD = r"""
import sys
sys.path.insert(0, "tests")
import numpy as np
import oracle as O
from juno_amd import matvec as mv
from test_gpu_sweep import QTYPES, check, raw_matrix, shape, x_batch
be = mv.GpuContext.shared(0).create_mat_vec()
rng = np.random.default_rng(9200)
for case in range(24):
    qtype = [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0][int(rng.integers(4))]
    rows, cols = shape(qtype, rng)
    a = int(rng.integers(0, rows))
    b = int(rng.integers(a + 1, rows + 1))
    raw = raw_matrix(qtype, rows, cols, rng)
    X = x_batch(1, cols, rng)
    print("staged case", case, qtype, rows, cols, a, b, flush=True)
    with be.upload_quant(mv.QuantizedTensor("w", qtype, rows * cols, raw.tobytes()), rows, cols) as dev:
        Y = be.sgemv_quant(dev, X[0], a, b)[None, :]
    worst = check(qtype, raw, rows, cols, a, b, X, Y)
    assert worst <= 1e-3, (case, qtype, rows, cols, a, b, worst)
print("staged-sweep-ok", flush=True)
"""


def test_random_shapes_staged_kernel():
    env = dict(os.environ, JUNO_STAGED_R="1")
    r = subprocess.run([sys.executable, "-u", "-c", STAGED_CHILD], env=env, cwd=ROOT, capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0 and "staged-sweep-ok" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
