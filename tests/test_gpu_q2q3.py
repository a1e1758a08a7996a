"""Q2_K and Q3_K on the device against the oracle's restatement of
dequantizeQ2K / dequantizeQ3K and matVecQ2Kraw / matVecQ3Kraw
(LlamaTransformerHandler.java:915-1015, 1293-1425): dequantization bit-exact
(including the reference's known-answer blocks, GgufReaderTest.java:140-287),
GEMVs within the 1e-3 bar (eps_r = 1e-3 * sum |w x|) for B = 1, grouped
launches, row ranges and batches, and the embedding lookup.

Inputs are random blocks with finite fp16 scales: every byte pattern is a
valid Q2_K / Q3_K block (the reference has no quantizer for these formats).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from test_oracle_q2q3 import q2k_block, q3k_block, random_blocks

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from juno_amd import _lib  # noqa: E402
from juno_amd import matvec as mv  # noqa: E402

TYPES = [O.Q2_K, O.Q3_K]


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def be():
    return mv.GpuContext.shared(0).create_mat_vec()


def rel_err(y, ref, deq, x):
    scale = np.abs(deq.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return np.abs(y.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-3 * scale)


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_bit_exact_random_blocks(be, qtype):
    rows, cols = 37, 768
    raw = random_blocks(qtype, rows, cols, 100 + qtype)
    with be.upload_quant(qtype, rows, cols, raw) as m:
        got = be.dequantize(m)
    ref = O.dequantize(qtype, raw, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_reference_known_answers(be, golden):
    for c in golden["q2k_known_answers"]["cases"]:
        blk = q2k_block([c["sc_fill"]] * 16, [c["qs_fill"]] * 64, c["d_f16"], c["dmin_f16"])
        with be.upload_quant(O.Q2_K, 1, 256, blk) as m:
            assert np.all(be.dequantize(m) == np.float32(c["expected_all"])), c
    g = golden["q3k_known_answers"]
    for c in g["cases"]:
        blk = q3k_block([c["hmask_fill"]] * 32, [c["qs_fill"]] * 64, g["scales12"], c["d_f16"])
        with be.upload_quant(O.Q3_K, 1, 256, blk) as m:
            assert np.all(be.dequantize(m) == np.float32(c["expected_all"])), c


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("rows,cols", [(1, 256), (7, 512), (64, 2304), (300, 4096), (4096, 4096), (1000, 14336)])
def test_gemv_vs_oracle(be, qtype, rows, cols):
    say("q2q3 gemv", qtype, rows, cols)
    raw = random_blocks(qtype, rows, cols, rows + cols + qtype)
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    deq = O.dequantize(qtype, raw, rows, cols)
    ref = O.matvec(qtype, raw, x, 0, rows, cols).astype(np.float64)
    with be.upload_quant(qtype, rows, cols, raw) as m:
        y = be.sgemv_quant(m, x)
        lo, hi = rows // 3, rows - rows // 4
        y_rng = be.sgemv_quant(m, x, lo, hi)
    assert rel_err(y, ref, deq, x).max() <= 1e-3
    assert rel_err(y_rng, ref[lo:hi], deq[lo:hi], x).max() <= 1e-3


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("B", [2, 3, 5, 8, 16, 20, 32, 48])
def test_batched_vs_oracle(be, qtype, B):
    rows, cols = 257, 1024
    raw = random_blocks(qtype, rows, cols, 7 * B + qtype)
    X = np.random.default_rng(B).standard_normal((B, cols)).astype(np.float32)
    deq = O.dequantize(qtype, raw, rows, cols)
    with be.upload_quant(qtype, rows, cols, raw) as m:
        Y = be.sgemv_batched(m, X)
    for j in range(B):
        ref = O.matvec(qtype, raw, X[j], 0, rows, cols).astype(np.float64)
        assert rel_err(Y[j], ref, deq, X[j]).max() <= 1e-3, j


@pytest.mark.parametrize("qtype", TYPES)
def test_batched_mfma_split_shapes(be, qtype):
    """The MFMA path (B >= 3) at shapes whose K is split across workgroups
    (the in-kernel hand-off) and at a wide row, B in {3, 32, 64}."""
    for rows, cols in ((1024, 4096), (512, 14336)):
        raw = random_blocks(qtype, rows, cols, 11 + rows + qtype)
        deq = O.dequantize(qtype, raw, rows, cols)
        with be.upload_quant(qtype, rows, cols, raw) as m:
            for B in (3, 32, 64):
                X = np.random.default_rng(B + rows).standard_normal((B, cols)).astype(np.float32)
                Y = be.sgemv_batched(m, X)
                for j in (0, B - 1):
                    ref = O.matvec(qtype, raw, X[j], 0, rows, cols).astype(np.float64)
                    assert rel_err(Y[j], ref, deq, X[j]).max() <= 1e-3, (rows, B, j)


def test_batched_group_all_formats(be):
    """One MFMA launch over Q2_K, Q3_K, Q4_K and Q6_K matrices sharing cols."""
    B, cols = 32, 1024
    shapes = [(O.Q2_K, 300), (O.Q3_K, 257), (O.Q4_K, 128), (O.Q6_K, 200)]
    Xs = np.random.default_rng(5).standard_normal((B, cols)).astype(np.float32)
    dX = torch.from_numpy(Xs).cuda()
    mats, raws, ys = [], [], []
    try:
        for i, (t, r) in enumerate(shapes):
            raw = random_blocks(t, r, cols, 90 + i) if t in TYPES else O.quantize(t, (np.random.default_rng(
                90 + i).standard_normal(r * cols) * 0.02).astype(np.float32))
            raws.append(raw)
            mats.append(be.upload_quant(t, r, cols, raw))
            ys.append(torch.full((B, r), float("nan"), device="cuda"))
        be.sgemv_batched_group_dev(mats, [dX.data_ptr()] * 4, B, [y.data_ptr() for y in ys])
        torch.cuda.synchronize()
        for (t, r), raw, y in zip(shapes, raws, ys):
            Y = y.cpu().numpy()
            deq = O.dequantize(t, raw, r, cols)
            for j in (0, B - 1):
                ref = O.matvec(t, raw, Xs[j], 0, r, cols).astype(np.float64)
                assert rel_err(Y[j], ref, deq, Xs[j]).max() <= 1e-3, (t, j)
    finally:
        for m in mats:
            m.close()


def test_group_dev_mixed_formats(be):
    L = _lib.load()
    shapes = [(O.Q2_K, 512, 2048), (O.Q3_K, 300, 2048), (O.Q4_K, 128, 2048), (O.Q3_K, 2048, 2048)]
    mats, raws, ys = [], [], []
    x = np.random.default_rng(3).standard_normal(2048).astype(np.float32)
    dx = torch.from_numpy(x).cuda()
    for i, (t, r, c) in enumerate(shapes):
        raw = random_blocks(t, r, c, 40 + i) if t != O.Q4_K else O.quantize(
            t, (np.random.default_rng(i).standard_normal(r * c) * 0.02).astype(np.float32))
        raws.append(raw)
        mats.append(be.upload_quant(t, r, c, raw))
        ys.append(torch.empty(r, device="cuda"))
    n = len(mats)
    V = ctypes.c_void_p
    assert L.jh_qmatvec_group_dev(n, (V * n)(*[m.handle for m in mats]), (V * n)(*[dx.data_ptr()] * n),
                                  (V * n)(*[y.data_ptr() for y in ys]), None) == 0
    torch.cuda.synchronize()
    for (t, r, c), raw, y, m in zip(shapes, raws, ys, mats):
        ref = O.matvec(t, raw, x, 0, r, c).astype(np.float64)
        assert rel_err(y.cpu().numpy(), ref, O.dequantize(t, raw, r, c), x).max() <= 1e-3, t
        m.close()


@pytest.mark.parametrize("qtype", TYPES)
def test_embedding_rows(be, qtype):
    L = _lib.load()
    vocab, hidden = 50, 512
    raw = random_blocks(qtype, vocab, hidden, 60 + qtype)
    table = O.dequantize(qtype, raw, vocab, hidden)
    toks = torch.tensor([0, 49, 7, 100, -5], dtype=torch.int32, device="cuda")
    out = torch.full((5, hidden), float("nan"), device="cuda")
    with be.upload_quant(qtype, vocab, hidden, raw) as m:
        assert L.jh_embed_rows_dev(m.handle, ctypes.c_void_p(toks.data_ptr()), 5, ctypes.c_void_p(out.data_ptr()),
                                   None) == 0
        torch.cuda.synchronize()
    want = table[[0, 49, 7, 49, 0]]
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
