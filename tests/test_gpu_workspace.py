"""The per-stream library workspace under HIP-graph capture.

A graph captured from *_dev calls keeps the addresses of its stream's
workspace (split-K partials and arrival counters of the batched MFMA path).
When a later eager call on the same stream needs more scratch, the workspace
is replaced by a larger one and the old one stays allocated, so the earlier
graph still replays into valid memory and still matches the oracle.  Growth is
refused inside a capture.
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


def rel_err(y, ref, deq, x):
    scale = np.abs(deq.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)


def quantized(qtype, rows, cols, seed):
    w = (np.random.default_rng(seed).standard_normal(rows * cols) * 0.02).astype(np.float32)
    return O.quantize(qtype, w)


def ws_info(L, stream):
    cap, base = ctypes.c_size_t(), ctypes.c_void_p()
    assert L.jh_stream_workspace_info(0, ctypes.c_void_p(stream.cuda_stream), ctypes.byref(cap),
                                      ctypes.byref(base)) == 0
    return cap.value, base.value


def test_graph_replay_after_workspace_growth():
    """Capture a split-K batched GEMV at B = 16 (2 MB of partials), grow the
    stream's workspace with an eager B = 64 call on a 14336-row matrix (15 MB of
    partials), then replay the first graph between further eager calls: every
    replay equals the eager result bit for bit and the oracle to the GEMV bar."""
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    cols = 4096
    small = (O.Q4_K, 4096, 16)
    large = (O.Q4_K, 14336, 64)
    raws = [quantized(t, r, cols, 900 + i) for i, (t, r, _) in enumerate((small, large))]
    devs = [be.upload_quant(mv.QuantizedTensor("w", t, r * cols, raw.tobytes()), r, cols)
            for (t, r, _), raw in zip((small, large), raws)]
    try:
        s = torch.cuda.Stream()
        S = ctypes.c_void_p(s.cuda_stream)
        rng = np.random.default_rng(901)
        X = [rng.standard_normal((B, cols)).astype(np.float32) for _, _, B in (small, large)]
        dX = [torch.from_numpy(x).cuda() for x in X]
        dY = [torch.zeros(B, r, device="cuda") for _, r, B in (small, large)]

        def launch(i):
            _, rows, B = (small, large)[i]
            rc = L.jh_qmatvec_batched_dev(devs[i].handle, ctypes.c_void_p(dX[i].data_ptr()), B,
                                          ctypes.c_void_p(dY[i].data_ptr()), 0, rows, S)
            assert rc == 0, _lib.last_error()

        say("workspace growth: eager small call, then capture")
        with torch.cuda.stream(s):
            launch(0)
        s.synchronize()
        eager = dY[0].cpu().numpy()
        cap0, base0 = ws_info(L, s)
        assert cap0 > 0 and base0
        deq = O.dequantize(small[0], raws[0], small[1], cols)
        for j in (0, small[2] - 1):
            ref = O.matvec(small[0], raws[0], X[0][j], 0, small[1], cols).astype(np.float64)
            assert rel_err(eager[j], ref, deq, X[0][j]).max() <= TOL, j
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                launch(0)

        say("workspace growth: eager large call grows the workspace")
        with torch.cuda.stream(s):
            launch(1)
        s.synchronize()
        cap1, base1 = ws_info(L, s)
        assert cap1 > cap0 and base1 != base0, (cap0, cap1)
        deq1 = O.dequantize(large[0], raws[1], large[1], cols)
        y1 = dY[1].cpu().numpy()
        for j in (0, large[2] - 1):
            ref = O.matvec(large[0], raws[1], X[1][j], 0, large[1], cols).astype(np.float64)
            assert rel_err(y1[j], ref, deq1, X[1][j]).max() <= TOL, j

        for rep in range(3):
            say("workspace growth: replay of the graph captured before growth", rep)
            dY[0].zero_()
            with torch.cuda.stream(s):
                g.replay()
            s.synchronize()
            assert np.array_equal(dY[0].cpu().numpy(), eager), rep
            with torch.cuda.stream(s):
                launch(1)  # eager work on the grown workspace between replays
                launch(0)
            s.synchronize()
            assert np.array_equal(dY[0].cpu().numpy(), eager), rep
            assert np.array_equal(dY[1].cpu().numpy(), y1), rep
        del g
        torch.cuda.synchronize()
    finally:
        for d in devs:
            d.close()


def test_growth_refused_during_capture():
    """A call that would need a larger workspace inside a capture fails with
    JH_EINVAL and names the eager call to make first; nothing is enqueued."""
    import torch
    L = _lib.load()
    be = mv.GpuContext.shared(0).create_mat_vec()
    rows, cols, B = 14336, 4096, 64
    raw = quantized(O.Q4_K, rows, cols, 950)
    with be.upload_quant(mv.QuantizedTensor("w", O.Q4_K, rows * cols, raw.tobytes()), rows, cols) as dev:
        s = torch.cuda.Stream()  # fresh stream: no workspace yet
        S = ctypes.c_void_p(s.cuda_stream)
        dx = torch.zeros(B, cols, device="cuda")
        dy = torch.zeros(B, rows, device="cuda")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        say("workspace growth refused during capture")
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                rc = L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B,
                                              ctypes.c_void_p(dy.data_ptr()), 0, rows, S)
                msg = _lib.last_error()
                dy.add_(0.0)  # keep the captured graph non-empty
        assert rc == _lib.JH_EINVAL
        assert "graph capture" in msg and "eager" in msg, msg
        assert ws_info(L, s)[0] == 0
        del g
        torch.cuda.synchronize()
