"""GPU parity suite: libjunohip (through its C ABI) against the CPU oracle.

Bars (stated per test): dequantized weights and quantizer bytes bit-exact;
GEMV outputs within max rel-err 1e-3 with the metric
    rel_r = |y_r - ref_r| / max(|ref_r|, 1e-3 * sum_c |w_rc x_c|)
(fp32 accumulation, order-of-summation differences only).

Inputs are seeded numpy draws, quantized with the oracle's restatement of
LoraMerge's quantizers, so both sides see identical packed bytes.
"""
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

import oracle as O
from juno_amd import matvec as mv

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    ctx = mv.GpuContext.shared(0)
    info = mv.device_info(0)
    say("device:", info)
    assert info["arch"].startswith("gfx950")
    return ctx.create_mat_vec()


def weights(n, seed, outliers=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    if outliers:
        idx = rng.choice(n, max(n // 100, 1), replace=False)
        w[idx] *= 10
    return w


def vec(n, seed, batch=None):
    rng = np.random.default_rng(seed)
    shape = (n,) if batch is None else (batch, n)
    return rng.standard_normal(shape).astype(np.float32)


def rel_err(y, ref, deq, x):
    """Per-row relative error with eps_r = 1e-3 * sum_c |w_rc x_c|."""
    scale = np.abs(deq.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)


def upload(be, qtype, raw, rows, cols):
    return be.upload_quant(mv.QuantizedTensor("w", qtype, rows * cols, raw.tobytes()), rows, cols)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K, O.F32])
@pytest.mark.parametrize("outliers", [False, True])
def test_dequant_bit_exact(be, qtype, outliers):
    rows, cols = 96, 1024
    say("dequant", qtype, outliers)
    raw = O.quantize(qtype, weights(rows * cols, 21 + qtype, outliers))
    with upload(be, qtype, raw, rows, cols) as dev:
        got = be.dequantize(dev)
    ref = O.dequantize(qtype, raw, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_random_bytes_bit_exact(be):
    # arbitrary bytes: every scale/min/nibble pattern, subnormal and huge d values
    rng = np.random.default_rng(5)
    for qtype, rows, cols in [(O.Q4_K, 64, 2048), (O.Q6_K, 64, 2048), (O.Q8_0, 64, 2048)]:
        raw = rng.integers(0, 256, O.raw_byte_count(qtype, rows * cols), dtype=np.uint8)
        # keep d / dmin finite so the comparison is on numbers (NaN payloads aside)
        bb, off = O.BLOCK_BYTES[qtype], {O.Q4_K: [0, 2], O.Q6_K: [208], O.Q8_0: [0]}[qtype]
        blocks = raw.reshape(-1, bb)
        for o in off:
            blocks[:, o + 1] &= 0x7B  # exponent < 31
        with upload(be, qtype, raw, rows, cols) as dev:
            got = be.dequantize(dev)
        ref = O.dequantize(qtype, raw, rows, cols)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), qtype


def test_f16_scales_exhaustive_via_q8_0(be):
    # every fp16 bit pattern as a Q8_0 scale with q = 1: dequant == f16ToF32
    halves = np.arange(65536, dtype=np.uint32)
    raw = np.zeros((65536, 34), dtype=np.uint8)
    raw[:, 0] = halves & 0xFF
    raw[:, 1] = halves >> 8
    raw[:, 2:] = 1
    raw = raw.reshape(-1)
    rows, cols = 2048, 1024
    with upload(be, O.Q8_0, raw, rows, cols) as dev:
        got = be.dequantize(dev).reshape(65536, 32)[:, 0]
    ref = halves.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_golden_q6k_block(be, golden):
    g = golden["q6k_golden_block"]
    blk = np.zeros(210, dtype=np.uint8)
    blk[:128] = np.array(g["ql"]).astype(np.int8).view(np.uint8)
    blk[128:192] = np.array(g["qh"]).astype(np.int8).view(np.uint8)
    blk[192:208] = np.array(g["sc"]).astype(np.int8).view(np.uint8)
    blk[208:] = [g["d_f16"] & 0xFF, g["d_f16"] >> 8]
    with upload(be, O.Q6_K, blk, 1, 256) as dev:
        out = be.dequantize(dev)[0]
        y = be.sgemv_quant(dev, np.ones(256, np.float32))
    for idx, val in g["expected"].items():
        assert out[int(idx)] == np.float32(val)
    assert abs(y[0] - float(out.astype(np.float64).sum())) <= 1e-3


# ------------------------------------------------------------------ quantizer

@pytest.mark.parametrize("qtype", [O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
@pytest.mark.parametrize("outliers", [False, True])
def test_device_quantizer_bit_exact(be, qtype, outliers):
    import torch
    n = 256 * 2048
    w = weights(n, 31 + qtype, outliers)
    w[:256] = 0.0                          # zero block
    w[256:512] = np.float32(3e-6) * np.sign(w[256:512])   # tiny values -> subnormal fp16 d
    w[512:768] = 1.0                       # constant block
    say("quantize", qtype, outliers)
    src = torch.from_numpy(w).cuda()
    dst = torch.zeros(O.raw_byte_count(qtype, n), dtype=torch.uint8, device="cuda")
    mv.quantize_dev(qtype, src.data_ptr(), n, dst.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), O.quantize(qtype, w))


# ------------------------------------------------------------------ GEMV

SHAPES = [
    (O.Q4_K, 5632, 2048),    # config 1: TinyLlama FFN up
    (O.Q4_K, 2048, 2048),
    (O.Q4_K, 256, 5632),     # nb = 22, not a multiple of 8
    (O.Q4_K, 1, 256),        # one row, one block
    (O.Q4_K, 37, 768),       # ragged rows, nb = 3
    (O.Q5_K, 3072, 3072),    # Phi-3.5 Q4_K_M uses Q5_K (PhiQuantizedMatVecTest.java:242-248)
    (O.Q5_K, 300, 5632),     # nb = 22
    (O.Q5_K, 1, 256),
    (O.Q6_K, 2048, 5632),    # TinyLlama ffn_down (4620-byte rows)
    (O.Q6_K, 1000, 3072),    # Phi-3 sizes, odd row count
    (O.Q6_K, 3, 256),
    (O.Q8_0, 2304, 3072),    # Phi-3 fused QKV slice
    (O.Q8_0, 129, 8192),
    (O.Q8_0, 5, 32),         # one block per row
    (O.F32, 513, 384),
    (O.F32, 7, 3),
]


@pytest.mark.parametrize("qtype,rows,cols", SHAPES)
def test_gemv_vs_oracle(be, qtype, rows, cols):
    say("gemv", qtype, rows, cols)
    raw = O.quantize(qtype, weights(rows * cols, rows + cols + qtype, outliers=qtype == O.Q8_0))
    x = vec(cols, 7 + cols)
    with upload(be, qtype, raw, rows, cols) as dev:
        y = be.sgemv_quant(dev, x)
    ref = O.matvec(qtype, raw, x, 0, rows, cols)
    deq = O.dequantize(qtype, raw, rows, cols)
    assert rel_err(y, ref.astype(np.float64), deq, x).max() <= TOL


def test_gemv_row_ranges(be):
    rows, cols = 3000, 2048
    for qtype in (O.Q4_K, O.Q6_K, O.Q8_0):
        raw = O.quantize(qtype, weights(rows * cols, 41))
        x = vec(cols, 42)
        deq = O.dequantize(qtype, raw, rows, cols)
        with upload(be, qtype, raw, rows, cols) as dev:
            for a, b in [(0, 1), (1, 2), (0, 2), (1024, 2048), (2048, 3000), (7, 1999), (2999, 3000), (5, 5)]:
                y = be.sgemv_quant(dev, x, a, b)
                assert y.shape == (b - a,)
                if b > a:
                    ref = O.matvec(qtype, raw, x, a, b, cols)
                    assert rel_err(y, ref.astype(np.float64), deq[a:b], x).max() <= TOL, (qtype, a, b)


def test_known_answers(be, golden):
    g = golden["q4k_all_ff_dot_ones"]
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [g["d_f16"] & 0xFF, g["d_f16"] >> 8]
    blk[4] = g["sc0"]
    blk[16:] = g["qs_fill"]
    with upload(be, O.Q4_K, blk, 1, 256) as dev:
        assert be.sgemv_quant(dev, np.ones(256, np.float32))[0] == g["expected_dot_ones"]
    g = golden["q4k_fused_rows"]
    raw = np.zeros((3, 144), dtype=np.uint8)
    for i, r in enumerate(g["rows"]):
        raw[i, 0:2] = [r["d_f16"] & 0xFF, r["d_f16"] >> 8]
        raw[i, 4] = g["sc0"]
        raw[i, 16:] = r["qs_fill"]
    with upload(be, O.Q4_K, raw.reshape(-1), 3, 256) as dev:
        x = np.ones(256, np.float32)
        assert list(be.sgemv_quant(dev, x)) == g["expected_dot_ones"]
        for a, b in g["row_ranges"]:
            assert list(be.sgemv_quant(dev, x, a, b)) == g["expected_dot_ones"][a:b]


def test_known_answer_q5k(be, golden):
    g = golden["q5k_ones"]  # PhiQuantizedMatVecTest.java:255-290
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = [g["d_f16"] & 0xFF, g["d_f16"] >> 8]
    blk[4] = g["sc0"]
    blk[48:] = g["qs_fill"]
    with upload(be, O.Q5_K, blk, 1, 256) as dev:
        assert be.sgemv_quant(dev, np.ones(256, np.float32))[0] == g["expected_dot_ones"]


def test_zero_inputs(be):
    for qtype in (O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0):
        rows, cols = 64, 512
        raw = O.quantize(qtype, weights(rows * cols, 3))
        with upload(be, qtype, raw, rows, cols) as dev:
            assert np.all(be.sgemv_quant(dev, np.zeros(cols, np.float32)) == 0.0)
        zraw = O.quantize(qtype, np.zeros(rows * cols, np.float32))
        with upload(be, qtype, zraw, rows, cols) as dev:
            assert np.all(be.sgemv_quant(dev, vec(cols, 4)) == 0.0)


def test_x_not_mutated(be):
    rows, cols = 128, 1024
    raw = O.quantize(O.Q4_K, weights(rows * cols, 5))
    x = vec(cols, 6)
    x0 = x.copy()
    with upload(be, O.Q4_K, raw, rows, cols) as dev:
        be.sgemv_quant(dev, x)
    assert np.array_equal(x, x0)


@pytest.mark.parametrize("B", [1, 2, 3, 5, 8, 11, 16, 20, 32, 48, 64])
@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0])
def test_batched_vs_independent(be, qtype, B):
    rows, cols = 1024, 2048
    say("batched", qtype, B)
    raw = O.quantize(qtype, weights(rows * cols, 50 + B))
    X = vec(cols, 60 + B, batch=B)
    deq = O.dequantize(qtype, raw, rows, cols)
    with upload(be, qtype, raw, rows, cols) as dev:
        Y = be.sgemv_batched(dev, X)
        y1 = be.sgemv_quant(dev, X[-1])
    assert Y.shape == (B, rows)
    for j in range(B):
        ref = O.matvec(qtype, raw, X[j], 0, rows, cols)
        assert rel_err(Y[j], ref.astype(np.float64), deq, X[j]).max() <= TOL, j
    assert rel_err(y1, Y[-1].astype(np.float64), deq, X[-1]).max() <= TOL


MFMA_SHAPES = [
    (O.Q4_K, 14336, 4096),   # 8B gate/up: one K split per 4 super-blocks
    (O.Q4_K, 1024, 4096),    # 8B k/v: K split 16 ways
    (O.Q5_K, 3072, 3072),    # Phi-3.5 Q4_K_M's Q5_K projections
    (O.Q6_K, 4096, 14336),   # 8B ffn_down (Q4_K_M)
    (O.Q6_K, 1024, 4096),    # 8B attn_v (Q4_K_M)
    (O.Q8_0, 9216, 3072),    # Phi-3 fused QKV
    (O.Q8_0, 3072, 8192),    # Phi-3 down
]


@pytest.mark.parametrize("qtype,rows,cols", MFMA_SHAPES)
def test_batched_mfma_8b_shapes(be, qtype, rows, cols):
    """The batched path at the 8B / Phi-3 shapes, B in {8, 16, 32, 64} (config 4's
    batches: B = 8 takes the MFMA kernel too), against the oracle per column
    (weights with 1 % outliers at 10x, x with spikes)."""
    raw = O.quantize(qtype, weights(rows * cols, 400 + rows + qtype, outliers=True))
    deq = O.dequantize(qtype, raw, rows, cols)
    with upload(be, qtype, raw, rows, cols) as dev:
        for B in (8, 16, 32, 64):
            say("mfma", qtype, rows, cols, B)
            X = vec(cols, 500 + B, batch=B)
            X[:, ::131] *= 30.0
            Y = be.sgemv_batched(dev, X)
            for j in (0, B // 2, B - 1):
                ref = O.matvec(qtype, raw, X[j], 0, rows, cols).astype(np.float64)
                assert rel_err(Y[j], ref, deq, X[j]).max() <= TOL, (rows, B, j)


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0])
def test_batched_mfma_odd_pitch_row_range(be, qtype):
    """Rows whose blocks start at 2 (mod 4) bytes (Q6_K / Q8_0 with 3 super-blocks
    per row), a row range that starts mid-tile, and a batch that is not a multiple of 32."""
    rows, cols, B = 333, 768, 20
    raw = O.quantize(qtype, weights(rows * cols, 80 + qtype))
    deq = O.dequantize(qtype, raw, rows, cols)
    X = vec(cols, 81, batch=B)
    with upload(be, qtype, raw, rows, cols) as dev:
        for a, b in [(0, rows), (37, 300)]:
            say("mfma-range", qtype, a, b)
            Y = be.sgemv_batched(dev, X, a, b)
            for j in range(B):
                ref = O.matvec(qtype, raw, X[j], a, b, cols).astype(np.float64)
                assert rel_err(Y[j], ref, deq[a:b], X[j]).max() <= TOL, (a, b, j)


@pytest.mark.parametrize("qtype,rows,B", [(O.Q4_K, 1024, 32), (O.Q6_K, 4096, 20), (O.Q8_0, 3072, 48)])
def test_batched_mfma_split_graph_replay(be, qtype, rows, B):
    """Split-K tiles hand their partials to the last-arriving split through
    per-tile counters that every launch re-arms: eager launches and HIP-graph
    replays (with other eager work between them) are bit-identical, and match
    the oracle to the GEMV bar."""
    import ctypes
    import torch
    from juno_amd import _lib
    L = _lib.load()
    cols = 4096
    raw = O.quantize(qtype, weights(rows * cols, 600 + rows))
    deq = O.dequantize(qtype, raw, rows, cols)
    X = vec(cols, 601, batch=B)
    with upload(be, qtype, raw, rows, cols) as dev:
        s = torch.cuda.Stream()
        dx = torch.from_numpy(X).cuda()
        dy = torch.zeros(B, rows, device="cuda")
        S = ctypes.c_void_p(s.cuda_stream)

        def launch():
            assert L.jh_qmatvec_batched_dev(dev.handle, ctypes.c_void_p(dx.data_ptr()), B,
                                            ctypes.c_void_p(dy.data_ptr()), 0, rows, S) == 0

        with torch.cuda.stream(s):
            launch()
        s.synchronize()
        eager = dy.cpu().numpy()
        for j in (0, B - 1):
            ref = O.matvec(qtype, raw, X[j], 0, rows, cols).astype(np.float64)
            assert rel_err(eager[j], ref, deq, X[j]).max() <= TOL, j
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                launch()
        for rep in range(3):
            say("mfma graph replay", qtype, rows, B, rep)
            dy.zero_()
            with torch.cuda.stream(s):
                g.replay()
            s.synchronize()
            assert np.array_equal(dy.cpu().numpy(), eager), rep
            with torch.cuda.stream(s):
                launch()  # eager work between replays
            s.synchronize()
            assert np.array_equal(dy.cpu().numpy(), eager), rep


@pytest.mark.parametrize("B", [16, 20, 32, 48])
def test_batched_group_mixed_formats(be, B):
    """jh_qmatvec_batched_group_dev: Q4_K q / k and a Q6_K v sharing cols (a
    Q4_K_M attention group) plus a Q8_0 matrix with its own x, one launch;
    every output against the oracle to the GEMV bar, and a row count that is
    not a multiple of the tile."""
    import torch
    cols = 2048
    spec = [(O.Q4_K, 1024, 0), (O.Q4_K, 256, 0), (O.Q6_K, 333, 0), (O.Q8_0, 512, 1)]
    Xs = [vec(cols, 700 + B, batch=B), vec(cols, 701 + B, batch=B)]
    raws = [O.quantize(t, weights(r * cols, 710 + i)) for i, (t, r, _) in enumerate(spec)]
    devs = [upload(be, t, raw, r, cols) for (t, r, _), raw in zip(spec, raws)]
    try:
        dX = [torch.from_numpy(X).cuda() for X in Xs]
        dY = [torch.full((B, r), float("nan"), device="cuda") for _, r, _ in spec]
        say("batched group", B)
        be.sgemv_batched_group_dev(devs, [dX[xi].data_ptr() for _, _, xi in spec], B, [y.data_ptr() for y in dY])
        torch.cuda.synchronize()
        for (t, r, xi), raw, y in zip(spec, raws, dY):
            Y = y.cpu().numpy()
            deq = O.dequantize(t, raw, r, cols)
            for j in (0, B // 2, B - 1):
                ref = O.matvec(t, raw, Xs[xi][j], 0, r, cols).astype(np.float64)
                assert rel_err(Y[j], ref, deq, Xs[xi][j]).max() <= TOL, (t, r, j)
    finally:
        for d in devs:
            d.close()


def test_batched_row_range(be):
    rows, cols, B = 700, 1024, 16
    raw = O.quantize(O.Q4_K, weights(rows * cols, 70))
    X = vec(cols, 71, batch=B)
    deq = O.dequantize(O.Q4_K, raw, rows, cols)
    with upload(be, O.Q4_K, raw, rows, cols) as dev:
        Y = be.sgemv_batched(dev, X, 100, 333)
    for j in range(B):
        ref = O.matvec(O.Q4_K, raw, X[j], 100, 333, cols)
        assert rel_err(Y[j], ref.astype(np.float64), deq[100:333], X[j]).max() <= TOL


# ------------------------------------------------------------------ contract (MatVecBackendContractTest)

def test_contract_sgemv(be, golden):
    g = golden["contract_identity_2x3"]
    y = be.sgemv(np.array(g["matrix"], np.float32), np.array(g["x"], np.float32), 2, 3)
    assert np.allclose(y, g["expected"], atol=1e-6)
    g = golden["f32_matvec_4x4"]
    assert list(be.sgemv(np.array(g["matrix"], np.float32), np.array(g["x"], np.float32), 4, 4)) == g["expected"]
    rng = np.random.default_rng(20)
    for rows, cols in [(32, 32), (256, 256), (2048, 2048), (5632, 2048), (2048, 5632), (1, 512), (128, 1)]:
        A = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
        x = (rng.standard_normal(cols) * 0.02).astype(np.float32)
        ref = A.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert np.abs(be.sgemv(A, x, rows, cols) - ref).max() < 1e-4  # DELTA of the contract suite
    with pytest.raises(mv.IllegalArgumentException, match=r"rows\*cols"):
        be.sgemv(np.zeros(10, np.float32), np.zeros(4, np.float32), 3, 4)
    with pytest.raises(mv.IllegalArgumentException, match="cols"):
        be.sgemv(np.zeros(12, np.float32), np.zeros(5, np.float32), 3, 4)


def test_argument_errors(be):
    rows, cols = 4, 256
    raw = O.quantize(O.Q4_K, weights(rows * cols, 1))
    with pytest.raises(mv.IllegalArgumentException, match="rawByteCount"):
        be.upload_quant(O.Q4_K, rows, cols, raw[:-1])
    with pytest.raises(mv.IllegalArgumentException, match="cols"):
        be.upload_quant(O.Q4_K, 1, 300, np.zeros(144, np.uint8))
    with pytest.raises(mv.UnsupportedOperationException):
        be.upload_quant(2, 1, 256, np.zeros(144, np.uint8))  # Q4_0: sized by rawByteCount, no matVec
    dev = upload(be, O.Q4_K, raw, rows, cols)
    with pytest.raises(mv.IllegalArgumentException, match="cols"):
        be.sgemv_quant(dev, np.zeros(cols + 1, np.float32))
    with pytest.raises(mv.IllegalArgumentException, match="row range"):
        be.sgemv_quant(dev, np.zeros(cols, np.float32), 2, 5)
    dev.close()
    dev.close()  # idempotent
    with pytest.raises(mv.IllegalStateException, match="closed"):
        be.sgemv_quant(dev, np.zeros(cols, np.float32))


def test_device_pointer_variants(be):
    import torch
    rows, cols, B = 1536, 4096, 4
    raw = O.quantize(O.Q4_K, weights(rows * cols, 80))
    X = vec(cols, 81, batch=B)
    deq = O.dequantize(O.Q4_K, raw, rows, cols)
    dX = torch.from_numpy(X).cuda()
    dY = torch.zeros((B, rows - 100), device="cuda")
    dD = torch.zeros((rows, cols), device="cuda")
    s = torch.cuda.Stream()
    with upload(be, O.Q4_K, raw, rows, cols) as dev:
        with torch.cuda.stream(s):
            be.sgemv_dev(dev, dX.data_ptr(), dY.data_ptr(), 100, rows, stream=s.cuda_stream, batch=B)
            be.dequantize_dev(dev, dD.data_ptr(), stream=s.cuda_stream)
        s.synchronize()
    Y = dY.cpu().numpy()
    for j in range(B):
        ref = O.matvec(O.Q4_K, raw, X[j], 100, rows, cols)
        assert rel_err(Y[j], ref.astype(np.float64), deq[100:], X[j]).max() <= TOL
    assert np.array_equal(dD.cpu().numpy().view(np.uint32), deq.view(np.uint32))


def test_concurrent_threads(be):
    # N host threads x distinct matrices, each compared to the oracle
    rows, cols = 2048, 2048
    mats = []
    for i, qtype in enumerate([O.Q4_K, O.Q6_K, O.Q8_0, O.Q4_K]):
        raw = O.quantize(qtype, weights(rows * cols, 90 + i))
        x = vec(cols, 95 + i)
        mats.append((qtype, raw, x, O.matvec(qtype, raw, x, 0, rows, cols), O.dequantize(qtype, raw, rows, cols)))
    devs = [upload(be, q, raw, rows, cols) for q, raw, *_ in mats]
    errors = []

    def worker(k):
        try:
            q, raw, x, ref, deq = mats[k]
            for _ in range(20):
                y = be.sgemv_quant(devs[k], x)
                if rel_err(y, ref.astype(np.float64), deq, x).max() > TOL:
                    errors.append(k)
        except Exception as e:  # pragma: no cover
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(k,)) for k in range(len(mats))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=60)
    for d in devs:
        d.close()
    assert not errors


def test_alloc_failure_reports_hipmalloc():
    # LlamaTransformerHandler.java:340-357 falls back to the CPU when the
    # upload error names hipMalloc; force it from the host in a child process.
    code = (
        "import numpy as np\n"
        "from juno_amd import matvec as mv\n"
        "be = mv.GpuContext.shared(0).create_mat_vec()\n"
        "a = be.upload_quant(12, 1, 256, np.zeros(144, np.uint8))\n"
        "try:\n"
        "    be.upload_quant(12, 1, 256, np.zeros(144, np.uint8))\n"
        "except mv.IllegalStateException as e:\n"
        "    assert 'hipMalloc' in str(e), str(e)\n"
        "    print('fallback-ok')\n"
        "a.close()\n"
    )
    env = dict(os.environ, JUNO_HIP_FAIL_ALLOC_AFTER="1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=root, capture_output=True, text=True, timeout=120)
    assert "fallback-ok" in r.stdout, r.stdout + r.stderr


# ------------------------------------------------------------------ full sizes, size-independent properties

def test_llama8b_shapes_full_size(be):
    """Full 8B shapes: gate/up Q4_K 14336x4096 and ffn_down Q6_K 4096x14336 vs the
    oracle (multi-threaded), plus linearity W(a x1 + b x2) = a W x1 + b W x2."""
    for qtype, rows, cols in [(O.Q4_K, 14336, 4096), (O.Q6_K, 4096, 14336), (O.Q4_K, 1024, 4096)]:
        say("full", qtype, rows, cols)
        raw = O.quantize(qtype, weights(rows * cols, 100 + rows))
        x1, x2 = vec(cols, 101), vec(cols, 102)
        deq = O.dequantize(qtype, raw, rows, cols)
        with upload(be, qtype, raw, rows, cols) as dev:
            y1 = be.sgemv_quant(dev, x1)
            y2 = be.sgemv_quant(dev, x2)
            y12 = be.sgemv_quant(dev, (np.float32(0.5) * x1 + np.float32(2.0) * x2).astype(np.float32))
        ref = O.matvec(qtype, raw, x1, 0, rows, cols)
        assert rel_err(y1, ref.astype(np.float64), deq, x1).max() <= TOL
        lin = 0.5 * y1.astype(np.float64) + 2.0 * y2.astype(np.float64)
        xs = np.abs(x1) * 0.5 + np.abs(x2) * 2.0
        assert rel_err(y12, lin, deq, xs).max() <= 2 * TOL


def test_group_dev_matches_single_calls(be):
    """jh_qmatvec_group_dev: q, k (Q4_K) + v (Q6_K) sharing x, gate + up (Q4_K,
    >= 28 MB together -> one staged launch), a Q8_0 and an F32 matrix with their
    own x; each output equals the oracle to the GEMV bar."""
    import torch
    specs = [("q", O.Q4_K, 4096, 4096, 0), ("k", O.Q4_K, 1024, 4096, 0), ("v", O.Q6_K, 1024, 4096, 0),
             ("gate", O.Q4_K, 14336, 4096, 1), ("up", O.Q4_K, 14336, 4096, 1),
             ("q8", O.Q8_0, 777, 3072, 2), ("f32", O.F32, 100, 384, 3)]
    xs = {0: vec(4096, 200), 1: vec(4096, 201), 2: vec(3072, 202), 3: vec(384, 203)}
    dxs = {k: torch.from_numpy(v).cuda() for k, v in xs.items()}
    mats, raws, dys = [], [], []
    for name, qt, rows, cols, xi in specs:
        say("group", name)
        raw = O.quantize(qt, weights(rows * cols, 300 + rows + qt))
        raws.append(raw)
        mats.append(upload(be, qt, raw, rows, cols))
        dys.append(torch.full((rows,), float("nan"), device="cuda"))
    be.sgemv_group_dev(mats, [dxs[s[4]].data_ptr() for s in specs], [y.data_ptr() for y in dys])
    torch.cuda.synchronize()
    for (name, qt, rows, cols, xi), raw, dy, m in zip(specs, raws, dys, mats):
        y = dy.cpu().numpy()
        ref = O.matvec(qt, raw, xs[xi], 0, rows, cols).astype(np.float64)
        deq = O.dequantize(qt, raw, rows, cols)
        assert rel_err(y, ref, deq, xs[xi]).max() <= TOL, name
        m.close()


def test_group_dev_arguments(be):
    from juno_amd import _lib
    L = _lib.load()
    assert L.jh_qmatvec_group_dev(9, None, None, None, None) == _lib.JH_EINVAL
    assert "n=9" in _lib.last_error()
    assert L.jh_qmatvec_group_dev(1, None, None, None, None) == _lib.JH_EINVAL
    be.sgemv_group_dev([], [], [])  # n = 0 is a no-op


@pytest.mark.parametrize("qt,rows,cols", [(O.Q4_K, 8192, 4096), (O.Q6_K, 1536, 14336), (O.Q4_K, 256, 1024),
                                          (O.Q8_0, 300, 2048)],
                         ids=["q4k staged", "q6k staged 4 tiles", "q4k small", "q8_0 small"])
def test_swiglu_dev(be, qt, rows, cols):
    """jh_qmatvec_swiglu_dev equals jh_qmatvec_group_dev on [gate, up] followed by
    jh_silu_mul_dev, bit for bit (the paired staged launch forms each row's
    two dot products exactly as the grouped launch does); the projections
    themselves are pinned against the oracle by the group tests."""
    import ctypes
    import torch
    from juno_amd import _lib
    L = _lib.load()
    say("swiglu", qt, rows, cols)
    raw_g = O.quantize(qt, weights(rows * cols, 400 + qt))
    raw_u = O.quantize(qt, weights(rows * cols, 401 + qt))
    g, u = upload(be, qt, raw_g, rows, cols), upload(be, qt, raw_u, rows, cols)
    try:
        x = torch.from_numpy(vec(cols, 402) * 3).cuda()
        yg = torch.full((rows,), float("nan"), device="cuda")
        yu = torch.full((rows,), float("nan"), device="cuda")
        ref = torch.full((rows,), float("nan"), device="cuda")
        out = torch.full((rows,), float("nan"), device="cuda")
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        be.sgemv_group_dev([g, u], [x.data_ptr()] * 2, [yg.data_ptr(), yu.data_ptr()])
        assert L.jh_silu_mul_dev(P(yg), P(yu), rows, P(ref), None) == 0
        assert L.jh_qmatvec_swiglu_dev(g.handle, u.handle, P(x), P(out), None) == 0, L.jh_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref)
        # mismatched shapes are refused
        with upload(be, qt, raw_g[: len(raw_g) // 2], rows // 2, cols) as half:
            assert L.jh_qmatvec_swiglu_dev(g.handle, half.handle, P(x), P(out), None) == 1
    finally:
        g.close()
        u.close()


@pytest.mark.parametrize("qt,rows,cols", [(O.Q4_K, 1000, 4096), (O.Q6_K, 384, 2048), (O.Q5_K, 256, 1024),
                                          (O.Q8_0, 300, 3072), (O.Q4_K, 4096, 14336)],
                         ids=["q4k", "q6k", "q5k", "q8_0", "q4k split K"])
@pytest.mark.parametrize("B", [1, 2, 3, 17, 32, 40])
def test_batched_swiglu_dev(be, qt, rows, cols, B):
    """jh_qmatvec_batched_swiglu_dev equals jh_qmatvec_batched_group_dev on
    [gate, up] followed by jh_silu_mul_dev, bit for bit, at every batch: the
    paired MFMA launch (3 <= B <= 32, a row count that is not a multiple of its
    128-row tiles, split K at 14336 columns), B = 1 and the fallback (B = 2, 40)."""
    import ctypes
    import torch
    from juno_amd import _lib
    L = _lib.load()
    say("batched swiglu", qt, rows, cols, B)
    raw_g = O.quantize(qt, weights(rows * cols, 410 + qt))
    raw_u = O.quantize(qt, weights(rows * cols, 411 + qt))
    g, u = upload(be, qt, raw_g, rows, cols), upload(be, qt, raw_u, rows, cols)
    try:
        X = torch.from_numpy(vec(cols, 412, batch=B) * 3).cuda()
        yg = torch.full((B, rows), float("nan"), device="cuda")
        yu = torch.full((B, rows), float("nan"), device="cuda")
        ref = torch.full((B, rows), float("nan"), device="cuda")
        out = torch.full((B, rows), float("nan"), device="cuda")
        sg = torch.full((B, rows), float("nan"), device="cuda")
        su = torch.full((B, rows), float("nan"), device="cuda")
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        be.sgemv_batched_group_dev([g, u], [X.data_ptr()] * 2, B, [yg.data_ptr(), yu.data_ptr()])
        assert L.jh_silu_mul_dev(P(yg), P(yu), B * rows, P(ref), None) == 0
        rc = L.jh_qmatvec_batched_swiglu_dev(g.handle, u.handle, P(X), B, P(out), P(sg), P(su), None)
        assert rc == 0, L.jh_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref)
    finally:
        g.close()
        u.close()


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_empty_and_edge_ranges(be, qtype):
    """Edge cases of the matVec contract (LlamaTransformerHandler.matVec's row
    range, :1200-1212): an empty row range returns an empty vector, B = 0 an
    empty batch, the first and last single rows match the oracle, a matrix of
    zero rows uploads and multiplies to nothing, and grouped calls with n = 0
    are no-ops."""
    import ctypes

    from juno_amd import _lib
    rows, cols = 300, 512
    raw = O.quantize(qtype, weights(rows * cols, 140 + qtype))
    x = vec(cols, 141)
    deq = O.dequantize(qtype, raw, rows, cols)
    with upload(be, qtype, raw, rows, cols) as dev:
        for k in (0, 17, rows):
            assert be.sgemv_quant(dev, x, k, k).shape == (0,)
            assert be.sgemv_batched(dev, np.zeros((4, cols), np.float32), k, k).shape == (4, 0)
        assert be.sgemv_batched(dev, np.zeros((0, cols), np.float32)).shape == (0, rows)
        for a in (0, rows - 1):
            y = be.sgemv_quant(dev, x, a, a + 1)
            ref = O.matvec(qtype, raw, x, a, a + 1, cols).astype(np.float64)
            assert rel_err(y, ref, deq[a:a + 1], x).max() <= TOL
            Y = be.sgemv_batched(dev, np.stack([x, -x, 2 * x, x]), a, a + 1)
            assert rel_err(Y[1], -ref, deq[a:a + 1], x).max() <= TOL
            assert rel_err(Y[2], 2 * ref, deq[a:a + 1], x).max() <= TOL
        with pytest.raises(mv.IllegalArgumentException, match="row range"):
            be.sgemv_quant(dev, x, 5, 4)
        with pytest.raises(mv.IllegalArgumentException, match="row range"):
            be.sgemv_quant(dev, x, 0, rows + 1)
    with upload(be, qtype, np.zeros(0, np.uint8), 0, cols) as empty:
        assert be.sgemv_quant(empty, x).shape == (0,)
        assert be.sgemv_batched(empty, np.stack([x] * 8)).shape == (8, 0)
    L = _lib.load()
    assert L.jh_qmatvec_group_dev(0, None, None, None, None) == 0
    assert L.jh_qmatvec_batched_group_dev(0, None, None, 32, None, None) == 0
