"""Numerics of the integer / fp16-limb x paths against the oracle when x has a
wide dynamic range inside one 256-column super-block.

The B = 1 staged kernel rounds x to a fixed-point integer on a scale set by
the largest |x| of each 256-column block; the batched MFMA kernels split x into
fp16 hi + lo limbs on a power-of-two scale per (batch column, super-block).
Both lose resolution on the small elements of a block that also holds a large
one.  These cases make the small elements carry the whole dot product: the
large element's weight is exactly zero (its 32-column sub-block, or its Q8_0
block, is all zeros, which every quantizer here stores exactly as 0), so a
lost small-element term shows up as a relative error of the output and is not
hidden by the eps floor of the tolerance metric.

Three cases:
  * massive activations: four channels at 300x the typical magnitude (the
    scale of outlier channels in LLM hidden states);
  * extreme: one element of every 256-column block at 1e4, the rest N(0, 1e-2)
    (a dynamic range of 1e6 inside the block);
  * extreme_in_subblock: the same x, with only the large element's own weight
    zero, so the small elements of its sub-block (which share its x scale on
    the staged path) carry their part of the dot product.
Bar, for every case and path: max rel-err 1e-3 with eps_r = 1e-3 * sum_c
|w_rc x_c| (the GEMV bar); the plain relative error (no eps floor) must also
stay within 1e-3 on rows whose |y| is at least 1e-2 of sum_c |w_rc x_c|.  On
the B = 1 staged kernel extreme_in_subblock is the case its exact path
exists for (an element 1e-6 of its sub-block's outlier would keep
only ~2^-11 of itself in the 30-bit integer x alone).
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


def profile_x(kind, B, cols, seed):
    rng = np.random.default_rng(seed)
    if kind == "massive":
        X = rng.standard_normal((B, cols)).astype(np.float32)
        big = rng.choice(cols, 4, replace=False)
        X[:, big] *= 300.0
    else:
        X = (rng.standard_normal((B, cols)) * 1e-2).astype(np.float32)
        big = np.arange(0, cols, 256) + rng.integers(0, 256, cols // 256)
        X[:, big] = 1e4 * np.sign(rng.standard_normal((B, len(big)))).astype(np.float32)
    return X, big


def weights_zero_at(qtype, rows, cols, big, seed, whole_subblock=True):
    """N(0, 0.02) weights that are zero in every row at each column of `big`:
    with whole_subblock, the whole 32-column sub-block (Q8_0: block) around it
    is zero; otherwise only that column, and for Q4_K its sub-block's other
    weights are made non-negative (then the sub-block's min is 0 and a zero
    weight is stored exactly as q = 0)."""
    w = (np.random.default_rng(seed).standard_normal((rows, cols)) * 0.02).astype(np.float32)
    for c in big:
        c0 = c // 32 * 32
        if whole_subblock:
            w[:, c0:c0 + 32] = 0.0
        else:
            if qtype in (O.Q4_K, O.Q5_K):
                w[:, c0:c0 + 32] = np.abs(w[:, c0:c0 + 32])
            w[:, c] = 0.0
    return w.reshape(-1)


def measure(qtype, raw, rows, cols, X, Y, label):
    deq = O.dequantize(qtype, raw, rows, cols).astype(np.float64)
    assert np.all(deq.reshape(rows, cols)[:, [c for c in range(cols) if abs(X[0, c]) >= 1e3]] == 0.0)
    worst = worst_plain = 0.0
    refs = []
    for j in range(X.shape[0]):
        ref = O.matvec(qtype, raw, X[j], 0, rows, cols, nthreads=16).astype(np.float64)
        refs.append(ref)
        scale = np.abs(deq) @ np.abs(X[j].astype(np.float64))
        err = np.abs(Y[j].astype(np.float64) - ref)
        worst = max(worst, float((err / np.maximum(np.abs(ref), 1e-3 * scale)).max()))
        big_rows = np.abs(ref) >= 1e-2 * scale
        if big_rows.any():
            worst_plain = max(worst_plain, float((err[big_rows] / np.abs(ref[big_rows])).max()))
    say(f"{label}: max rel-err {worst:.2e}, plain {worst_plain:.2e}")
    return worst, worst_plain, deq, refs


def run(dev, X, rows, stream=None):
    import torch
    L = _lib.load()
    B = X.shape[0]
    dx = torch.from_numpy(np.ascontiguousarray(X)).cuda()
    dy = torch.empty(B, rows, device="cuda")
    rc = L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B, ctypes.c_void_p(dy.data_ptr()), 0,
                                  rows, None)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return dy.cpu().numpy()


# B = 1 shapes are above the staged kernel's size threshold (28 MB); the
# 14336-column ones take its column-tiled form (each lane converts its own x)
@pytest.mark.parametrize("kind", ["massive", "extreme", "extreme_in_subblock"])
@pytest.mark.parametrize("qtype,rows,cols,B", [
    (O.Q4_K, 16384, 4096, 1), (O.Q5_K, 12288, 4096, 1), (O.Q6_K, 12288, 4096, 1), (O.Q8_0, 8192, 4096, 1),
    (O.Q4_K, 4096, 14336, 1), (O.Q6_K, 4096, 14336, 1),
    (O.Q4_K, 4096, 4096, 16), (O.Q5_K, 4096, 4096, 16), (O.Q6_K, 4096, 4096, 32), (O.Q8_0, 4096, 4096, 32)])
def test_wide_dynamic_range_x(be, kind, qtype, rows, cols, B):
    X, big = profile_x("massive" if kind == "massive" else "extreme", B, cols, 1500 + B)
    w = weights_zero_at(qtype, rows, cols, big, 1501, whole_subblock=kind != "extreme_in_subblock")
    raw = O.quantize(qtype, w)
    with be.upload_quant(mv.QuantizedTensor("w", qtype, rows * cols, raw.tobytes()), rows, cols) as dev:
        say(f"numerics {kind} type {qtype} {rows}x{cols} B={B}")
        Y = run(dev, X, rows)
    worst, worst_plain, _, _ = measure(qtype, raw, rows, cols, X, Y, f"{kind} type {qtype} {rows}x{cols} B={B}")
    assert worst <= TOL
    assert worst_plain <= TOL
