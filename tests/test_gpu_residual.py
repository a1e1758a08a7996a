"""The staged B = 1 kernel's exact path, held to the GEMV bar.

The staged kernel rounds x * 2^s to an integer below 2^30 with one s per quant
sub-block.  When one element sets the scale of many much smaller ones (the
launch-wide test `residual_matters`: the rounding residual above 2^-20 of the
mean of the sub-block's other elements), every workgroup of the launch
computes sum deq(w) * x in fp32 with the x itself instead of its walk, so such x
are used exactly (LlamaTransformerHandler.java:1457-1460 forms each product of
the fp32 x itself).

Each kernel layout is run in a child process with its environment switches
(they are read once per process): the default (one 16-wave workgroup per CU
claiming row groups; 16 waves sharing x for column-tiled rows), two rows per
group (JUNO_STAGED_R=2), the static split (JUNO_STAGED_DYN=0) and per-lane x
for column tiles (JUNO_STAGED_WIDE=4).  Every case asserts the GEMV bar:
max rel-err 1e-3 with eps_r = 1e-3 * sum_c |w_rc x_c|, and the plain relative
error on rows with |y| >= 1e-2 sum_c |w_rc x_c|.  The x kinds:
  * outlier: one element of every 256 columns at 1e4 among N(0, 1e-2), its own
    weight zero and its sub-block's other weights not, so the small elements of
    that sub-block carry their part of the dot product;
  * every_group: the same with an outlier in every sub-block (the exact path
    over all of them);
  * tiny: N(0, 1) * 1e-37 (shifts capped at 149: the scale 2^-s stays an fp32
    value);
  * normal: N(0, 1) with four channels at 300x (the walk: a control).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r'''
import ctypes, sys
import numpy as np
import torch
import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv

be = mv.GpuContext.shared(0).create_mat_vec()
L = _lib.load()
P = lambda t: ctypes.c_void_p(t.data_ptr())
TOL = 1e-3

def make_x(kind, cols, seed, G):
    rng = np.random.default_rng(seed)
    if kind == "tiny":
        return (rng.standard_normal(cols) * 1e-37).astype(np.float32), []
    if kind == "normal":
        x = rng.standard_normal(cols).astype(np.float32)
        x[rng.choice(cols, 4, replace=False)] *= 300.0
        return x, []
    x = (rng.standard_normal(cols) * 1e-2).astype(np.float32)
    step = G if kind == "every_group" else 256
    big = np.arange(0, cols, step) + rng.integers(0, step, cols // step)
    x[big] = (1e4 * np.sign(rng.standard_normal(len(big)))).astype(np.float32)
    return x, big

def make_w(qtype, rows, cols, big, seed):
    """N(0, 0.02) weights, zero in every row at the columns of big; for Q4_K /
    Q5_K those columns' 32-column sub-blocks are made non-negative (min 0, so a
    zero weight is stored exactly)."""
    w = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    for c in big:
        c0 = c // 32 * 32
        if qtype in (O.Q4_K, O.Q5_K):
            w[:, c0:c0 + 32] = np.abs(w[:, c0:c0 + 32])
        w[:, c] = 0.0
    return O.quantize(qtype, w.reshape(-1))

def check(label, y, ref, absdeq, x):
    y = y.astype(np.float64); ref = ref.astype(np.float64)
    scale = absdeq @ np.abs(x.astype(np.float64))
    err = np.abs(y - ref)
    rel = float((err / np.maximum(np.abs(ref), 1e-3 * scale)).max())
    big = np.abs(ref) >= 1e-2 * scale
    plain = float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0
    print(f"{label}: max rel-err {rel:.2e}, plain {plain:.2e}", flush=True)
    assert np.isfinite(y).all(), label
    assert rel <= TOL and plain <= TOL, (label, rel, plain)

def G_of(qtype):
    return 16 if qtype == O.Q6_K else 32

# single matrices through jh_qmatvec (sizes above the staged thresholds)
SHAPES = [(O.Q4_K, 14336, 4096), (O.Q5_K, 12288, 4096), (O.Q6_K, 12288, 4096), (O.Q8_0, 8192, 4096),
          (O.Q4_K, 4096, 14336), (O.Q6_K, 4096, 14336), (O.Q8_0, 2560, 8192)]
for qtype, rows, cols in SHAPES:
    for kind in ["outlier", "every_group", "tiny", "normal"]:
        x, big = make_x(kind, cols, rows + cols, G_of(qtype))
        raw = make_w(qtype, rows, cols, big, rows * 3 + cols)
        absdeq = np.abs(O.dequantize(qtype, raw, rows, cols).astype(np.float64))
        print(f"case {kind} type {qtype} {rows}x{cols}", flush=True)
        with be.upload_quant(qtype, rows, cols, raw) as dev:
            for a, b in [(0, rows), (rows // 3, rows - rows // 5)]:
                y = be.sgemv_quant(dev, x, a, b)
                ref = O.matvec(qtype, raw, x, a, b, cols, nthreads=16)
                check(f"  {kind} type {qtype} {rows}x{cols} rows [{a},{b})", y, ref, absdeq[a:b], x)

def dsilu(g):
    s = 1.0 / (1.0 + np.exp(-g))
    return s * (1.0 + g * (1.0 - s))

def check_swiglu(label, out, g, u, Sg, Su):
    out = out.astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    bound = TOL * (np.abs(dsilu(g) * u) * np.maximum(np.abs(g), 1e-3 * Sg)
                   + np.abs(g / (1.0 + np.exp(-g))) * np.maximum(np.abs(u), 1e-3 * Su)) + 1e-30
    r = float((np.abs(out - ref) / bound).max())
    print(f"{label}: max error / bound {r:.2e}", flush=True)
    assert np.isfinite(out).all() and r <= 1.0, (label, r)

# the SwiGLU pairing (gate row and up row in one group) and the fused rmsnorm forms
rows, cols, qtype = 14336, 4096, O.Q4_K
eps = 1e-5
for kind in ["outlier", "every_group"]:
    x, big = make_x(kind, cols, 77, 32)
    rg, ru = make_w(qtype, rows, cols, big, 78), make_w(qtype, rows, cols, big, 79)
    ag = np.abs(O.dequantize(qtype, rg, rows, cols).astype(np.float64))
    au = np.abs(O.dequantize(qtype, ru, rows, cols).astype(np.float64))
    gate, up = be.upload_quant(qtype, rows, cols, rg), be.upload_quant(qtype, rows, cols, ru)
    try:
        print(f"case swiglu {kind}", flush=True)
        dx = torch.from_numpy(x).cuda()
        out = torch.full((rows,), float("nan"), device="cuda")
        assert L.jh_qmatvec_swiglu_dev(gate.handle, up.handle, P(dx), P(out), None) == 0, _lib.last_error()
        torch.cuda.synchronize()
        g = O.matvec(qtype, rg, x, 0, rows, cols, nthreads=16).astype(np.float64)
        u = O.matvec(qtype, ru, x, 0, rows, cols, nthreads=16).astype(np.float64)
        ax = np.abs(x.astype(np.float64))
        check_swiglu(f"  swiglu {kind}", out.cpu().numpy(), g, u, ag @ ax, au @ ax)
        # fused residual add + rmsnorm: h = x + res with res small, norm weights near 1
        rng = np.random.default_rng(80)
        res = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
        res[big] = 0.0
        nw = (0.5 + rng.random(cols)).astype(np.float32)
        dres, dnw = torch.from_numpy(res).cuda(), torch.from_numpy(nw).cuda()
        xo, xn = (torch.full((cols,), float("nan"), device="cuda") for _ in range(2))
        assert L.jh_rmsnorm_qmatvec_swiglu_dev(gate.handle, up.handle, P(dx), P(dres), P(dnw), ctypes.c_float(eps),
                                               P(xo), P(xn), P(out), None) == 0, _lib.last_error()
        torch.cuda.synchronize()
        xnr = O.rmsnorm(x + res, nw, eps)
        g = O.matvec(qtype, rg, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
        u = O.matvec(qtype, ru, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
        ax = np.abs(xnr.astype(np.float64))
        check_swiglu(f"  rmsnorm + swiglu {kind}", out.cpu().numpy(), g, u, ag @ ax, au @ ax)
    finally:
        gate.close(); up.close()

# the fused final norm + output projection (Q6_K) and a grouped launch (Q8_0)
for kind in ["outlier", "every_group"]:
    rows, cols, qtype = 32000, 2048, O.Q6_K
    x, big = make_x(kind, cols, 90, 16)
    raw = make_w(qtype, rows, cols, big, 91)
    absdeq = np.abs(O.dequantize(qtype, raw, rows, cols).astype(np.float64))
    rng = np.random.default_rng(92)
    res = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
    res[big] = 0.0
    nw = (0.5 + rng.random(cols)).astype(np.float32)
    with be.upload_quant(qtype, rows, cols, raw) as m:
        print(f"case rmsnorm output projection {kind}", flush=True)
        dx, dres, dnw = (torch.from_numpy(a).cuda() for a in (x, res, nw))
        xo, xn = (torch.full((cols,), float("nan"), device="cuda") for _ in range(2))
        y = torch.full((rows,), float("nan"), device="cuda")
        assert L.jh_rmsnorm_qmatvec_dev(m.handle, P(dx), P(dres), P(dnw), ctypes.c_float(1e-6), P(xo), P(xn), P(y),
                                        None) == 0, _lib.last_error()
        torch.cuda.synchronize()
        xnr = O.rmsnorm(x + res, nw, 1e-6)
        check(f"  rmsnorm output projection {kind}", y.cpu().numpy(), O.matvec(qtype, raw, xnr, 0, rows, cols,
              nthreads=16), absdeq, xnr)
    cols, qtype, rows_list = 3072, O.Q8_0, [9000, 4000]
    x, big = make_x(kind, cols, 93, 32)
    raws = [make_w(qtype, r, cols, big, 94 + i) for i, r in enumerate(rows_list)]
    mats = [be.upload_quant(qtype, r, cols, raw) for r, raw in zip(rows_list, raws)]
    try:
        print(f"case group {kind}", flush=True)
        dx = torch.from_numpy(x).cuda()
        dys = [torch.full((r,), float("nan"), device="cuda") for r in rows_list]
        be.sgemv_group_dev(mats, [dx.data_ptr()] * len(mats), [d.data_ptr() for d in dys])
        torch.cuda.synchronize()
        for r, raw, dy in zip(rows_list, raws, dys):
            absdeq = np.abs(O.dequantize(qtype, raw, r, cols).astype(np.float64))
            check(f"  group {kind} {r}x{cols}", dy.cpu().numpy(), O.matvec(qtype, raw, x, 0, r, cols, nthreads=16),
                  absdeq, x)
    finally:
        for m in mats:
            m.close()
print("residual-ok", flush=True)
'''


@pytest.mark.parametrize("env", [{}, {"JUNO_STAGED_R": "2"}, {"JUNO_STAGED_DYN": "0"}, {"JUNO_STAGED_WIDE": "4"}],
                         ids=["default", "two rows", "static split", "per-lane x"])
def test_exact_path(env):
    print(f"exact path, env {env}", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", CHILD], env=dict(os.environ, **env), cwd=ROOT,
                       capture_output=True, text=True, timeout=600)
    print(r.stdout[-4000:])
    assert r.returncode == 0 and "residual-ok" in r.stdout, r.stdout[-3000:] + r.stderr[-3000:]
