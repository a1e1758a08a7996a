"""The residual add and rmsnorm fused into the staged GEMV launches
(jh_rmsnorm_qmatvec_swiglu_dev, jh_rmsnorm_qmatvec_dev).

transformerLayer computes x2 = x + attnProj, rmsNorm(x2, ffnNorm) and the
SwiGLU of the gate / up projections (LlamaTransformerHandler.java:778-797,
rmsNorm :818-826), and the final norm before the output projection
(:803-810).  Checked, at a shape that takes the fused launch (8B gate / up
14336 x 4096 Q4_K, TinyLlama output 32000 x 2048 Q6_K) and at one that takes the
unfused fallback:
  * x_out = x + res bit for bit;
  * the output against the unfused composition (jh_rmsnorm_dev, then the GEMV
    entry point): they differ only in the summation order of mean(h^2), so the
    norm's scale may differ in its last bit; bar 1e-4 with the eps floor of the
    oracle comparison (measured up to 7e-5 for the SwiGLU product, 0 for the
    output projection);
  * the output against the oracle (rmsnorm, then the quantized matvec): the
    GEMV bar, max rel-err 1e-3;
  * aliasing x_out with x is refused.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from juno_amd import _lib
from juno_amd import matvec as mv

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def device_matrix(be, qtype, rows, cols, seed):
    import torch
    if qtype in (O.Q2_K, O.Q3_K):  # no quantizer for these in the reference: random blocks, small d
        from test_oracle_q2q3 import random_blocks
        return be.upload_quant(qtype, rows, cols, random_blocks(qtype, rows, cols, seed))
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn(rows * cols, generator=g, device="cuda").mul_(0.02)
    m = be.quantize_dev(qtype, w.data_ptr(), rows, cols, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return m


def rel_err(y, ref, absdeq, x):
    scale = absdeq @ np.abs(x.astype(np.float64))
    return np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)


def inputs(cols, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(cols).astype(np.float32)
    res = (rng.standard_normal(cols) * 0.5).astype(np.float32)
    nw = (0.5 + rng.random(cols)).astype(np.float32)
    return x, res, nw


@pytest.mark.parametrize("qt,rows,cols", [(O.Q4_K, 14336, 4096), (O.Q4_K, 1024, 2048)])
def test_rmsnorm_swiglu(qt, rows, cols):
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    eps = 1e-5
    gate, up = device_matrix(be, qt, rows, cols, 1800), device_matrix(be, qt, rows, cols, 1801)
    try:
        x, res, nw = inputs(cols, 1802)
        dx, dres, dnw = (torch.from_numpy(a).cuda() for a in (x, res, nw))
        xo, xn, out = (torch.full((n,), float("nan"), device="cuda") for n in (cols, cols, rows))
        xo2, xn2, out2 = (torch.full((n,), float("nan"), device="cuda") for n in (cols, cols, rows))
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        say(f"fused norm + swiglu {rows}x{cols}")
        rc = L.jh_rmsnorm_qmatvec_swiglu_dev(gate.handle, up.handle, P(dx), P(dres), P(dnw), ctypes.c_float(eps),
                                             P(xo), P(xn), P(out), None)
        assert rc == 0, _lib.last_error()
        # the unfused composition
        assert L.jh_rmsnorm_dev(P(dx), P(dres), P(dnw), cols, ctypes.c_float(eps), P(xo2), P(xn2), None) == 0
        assert L.jh_qmatvec_swiglu_dev(gate.handle, up.handle, P(xn2), P(out2), None) == 0
        torch.cuda.synchronize()
        h = x + res
        assert np.array_equal(xo.cpu().numpy(), h)
        y, y2 = out.cpu().numpy().astype(np.float64), out2.cpu().numpy().astype(np.float64)
        assert np.isfinite(y).all()
        d = np.abs(y - y2) / np.maximum(np.abs(y2), 1e-3 * np.abs(y2).max())
        say(f"  fused vs unfused: max rel diff {d.max():.2e}")
        assert d.max() <= 1e-4
        # the oracle: rmsNorm, gate / up matvecs, silu * up in float64 on the oracle's outputs
        xnr = O.rmsnorm(h, nw, eps)
        rg, ru = gate.packed_bytes(), up.packed_bytes()
        g_ref = O.matvec(qt, rg, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
        u_ref = O.matvec(qt, ru, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
        ref = g_ref / (1.0 + np.exp(-g_ref)) * u_ref
        err = np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3 * np.abs(ref).max())
        say(f"  vs oracle: max rel-err {err.max():.2e}")
        assert err.max() <= 1e-3
        # x_out may not alias x
        rc = L.jh_rmsnorm_qmatvec_swiglu_dev(gate.handle, up.handle, P(dx), P(dres), P(dnw), ctypes.c_float(eps),
                                             P(dx), P(xn), P(out), None)
        assert rc == _lib.JH_EINVAL and "alias" in _lib.last_error()
    finally:
        gate.close()
        up.close()


@pytest.mark.parametrize("qt,rows,cols", [(O.Q6_K, 32000, 2048), (O.Q8_0, 1000, 2048)])
def test_rmsnorm_output_projection(qt, rows, cols):
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    eps = 1e-6
    m = device_matrix(be, qt, rows, cols, 1810)
    try:
        x, res, nw = inputs(cols, 1811)
        dx, dres, dnw = (torch.from_numpy(a).cuda() for a in (x, res, nw))
        xo, xn, y = (torch.full((n,), float("nan"), device="cuda") for n in (cols, cols, rows))
        xn2, y2 = (torch.full((n,), float("nan"), device="cuda") for n in (cols, rows))
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        say(f"fused norm + output projection type {qt} {rows}x{cols}")
        rc = L.jh_rmsnorm_qmatvec_dev(m.handle, P(dx), P(dres), P(dnw), ctypes.c_float(eps), P(xo), P(xn), P(y), None)
        assert rc == 0, _lib.last_error()
        assert L.jh_rmsnorm_dev(P(dx), P(dres), P(dnw), cols, ctypes.c_float(eps), None, P(xn2), None) == 0
        assert L.jh_qmatvec_dev(m.handle, P(xn2), P(y2), 0, rows, None) == 0
        torch.cuda.synchronize()
        h = x + res
        assert np.array_equal(xo.cpu().numpy(), h)
        a, b = y.cpu().numpy().astype(np.float64), y2.cpu().numpy().astype(np.float64)
        raw = m.packed_bytes()
        absdeq = np.abs(O.dequantize(qt, raw, rows, cols).astype(np.float64))
        xnr = O.rmsnorm(h, nw, eps)
        d = np.abs(a - b) / np.maximum(np.abs(b), 1e-3 * (absdeq @ np.abs(xnr.astype(np.float64))))
        say(f"  fused vs unfused: max rel diff {d.max():.2e}")
        assert d.max() <= 1e-4
        ref = O.matvec(qt, raw, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
        err = rel_err(a, ref, absdeq, xnr)
        say(f"  vs oracle: max rel-err {err.max():.2e}")
        assert err.max() <= 1e-3
    finally:
        m.close()


@pytest.mark.parametrize("cols,shapes", [
    (4096, [(O.Q4_K, 4096), (O.Q4_K, 1024), (O.Q6_K, 1024)]),   # Llama-3-8B q / k / v of Q4_K_M
    (2048, [(O.Q4_K, 2048), (O.Q4_K, 256), (O.Q6_K, 256)]),     # TinyLlama
    (3072, [(O.Q8_0, 3072), (O.Q5_K, 768)]),
    (8192, [(O.Q4_K, 512), (O.Q8_0, 256)]),                     # the widest input the LDS image takes
    (14336, [(O.Q6_K, 300)]),                                    # wider: the unfused pair
    (2048, [(O.Q2_K, 1024), (O.Q3_K, 512), (O.Q4_K, 256)]),      # the Q2_K / Q3_K bodies of the fused group kernel
])
def test_rmsnorm_qkv_group(cols, shapes):
    """The attention norm fused into the one-shot grouped q / k / v launch
    (jh_rmsnorm_qmatvec_group_dev): x_out = x + res bit for bit, each output
    against the unfused composition (jh_rmsnorm_dev, then jh_qmatvec_group_dev;
    they differ in where the norm's scale is applied and the summation order of
    mean(h^2): bar 1e-4 with the eps floor) and against the oracle (rmsnorm,
    then the quantized matvec: the GEMV bar 1e-3)."""
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    eps = 1e-5
    mats = [device_matrix(be, qt, rows, cols, 1820 + i) for i, (qt, rows) in enumerate(shapes)]
    try:
        x, res, nw = inputs(cols, 1830)
        dx, dres, dnw = (torch.from_numpy(a).cuda() for a in (x, res, nw))
        n = len(mats)
        xo, xn, xn2 = (torch.full((cols,), float("nan"), device="cuda") for _ in range(3))
        ys = [torch.full((rows,), float("nan"), device="cuda") for _, rows in shapes]
        ys2 = [torch.full((rows,), float("nan"), device="cuda") for _, rows in shapes]
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        V = ctypes.c_void_p
        hs = (V * n)(*[m.handle for m in mats])
        say(f"fused norm + group cols={cols} {shapes}")
        rc = L.jh_rmsnorm_qmatvec_group_dev(n, hs, P(dx), P(dres), P(dnw), ctypes.c_float(eps), P(xo), P(xn),
                                            (V * n)(*[P(y) for y in ys]), None)
        assert rc == 0, _lib.last_error()
        assert L.jh_rmsnorm_dev(P(dx), P(dres), P(dnw), cols, ctypes.c_float(eps), None, P(xn2), None) == 0
        assert L.jh_qmatvec_group_dev(n, hs, (V * n)(*[P(xn2)] * n), (V * n)(*[P(y) for y in ys2]), None) == 0
        torch.cuda.synchronize()
        h = x + res
        assert np.array_equal(xo.cpu().numpy(), h)
        xnr = O.rmsnorm(h, nw, eps)
        for (qt, rows), m, y, y2 in zip(shapes, mats, ys, ys2):
            a, b = y.cpu().numpy().astype(np.float64), y2.cpu().numpy().astype(np.float64)
            raw = m.packed_bytes()
            absdeq = np.abs(O.dequantize(qt, raw, rows, cols).astype(np.float64))
            d = np.abs(a - b) / np.maximum(np.abs(b), 1e-3 * (absdeq @ np.abs(xnr.astype(np.float64))))
            ref = O.matvec(qt, raw, xnr, 0, rows, cols, nthreads=16).astype(np.float64)
            err = rel_err(a, ref, absdeq, xnr)
            say(f"  type {qt} {rows}x{cols}: fused vs unfused {d.max():.2e}, vs oracle {err.max():.2e}")
            assert d.max() <= 1e-4
            assert err.max() <= 1e-3
        # without res the unfused path runs (rmsnorm into xn): same outputs as the composition
        assert L.jh_rmsnorm_qmatvec_group_dev(n, hs, P(dx), None, P(dnw), ctypes.c_float(eps), None, P(xn),
                                              (V * n)(*[P(y) for y in ys]), None) == 0
        assert L.jh_rmsnorm_dev(P(dx), None, P(dnw), cols, ctypes.c_float(eps), None, P(xn2), None) == 0
        assert L.jh_qmatvec_group_dev(n, hs, (V * n)(*[P(xn2)] * n), (V * n)(*[P(y) for y in ys2]), None) == 0
        torch.cuda.synchronize()
        for y, y2 in zip(ys, ys2):
            assert np.array_equal(y.cpu().numpy(), y2.cpu().numpy())
        # x_out may not alias x
        rc = L.jh_rmsnorm_qmatvec_group_dev(n, hs, P(dx), P(dres), P(dnw), ctypes.c_float(eps), P(dx), P(xn),
                                            (V * n)(*[P(y) for y in ys]), None)
        assert rc == _lib.JH_EINVAL and "alias" in _lib.last_error()
    finally:
        for m in mats:
            m.close()


STATIC_CHILD = r'''
import sys
sys.path.insert(0, "tests")
import test_gpu_fused_norm as T
import oracle as O
for qt, rows, cols in [(O.Q4_K, 14336, 4096)]:
    T.test_rmsnorm_swiglu(qt, rows, cols)
for qt, rows, cols in [(O.Q6_K, 32000, 2048)]:
    T.test_rmsnorm_output_projection(qt, rows, cols)
print("static-ok", flush=True)
'''


def test_fused_norm_static_layout():
    """The SwiGLU and output-projection fusions through the static staged layout
    (JUNO_STAGED_DYN=0: 4-wave workgroups with equal shares, the NW = 4 NORM
    kernels), in a child process (the switch is read once per process)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, JUNO_STAGED_DYN="0")
    r = subprocess.run([sys.executable, "-u", "-c", STATIC_CHILD], env=env, cwd=root, capture_output=True,
                       text=True, timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0 and "static-ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
