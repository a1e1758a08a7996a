"""Pins the oracle's Q2_K and Q3_K restatements (dequantizeQ2K / dequantizeQ3K
and matVecQ2Kraw / matVecQ3Kraw, LlamaTransformerHandler.java:915-1015 and
1293-1425).

* the reference's own known answers (GgufReaderTest.java:140-287), exact;
* the Q3_K 6-bit scale field: unpack(pack(s)) = s for random signed scales,
  with pack written from the field layout (low nibbles in bytes 0..7, the two
  high bits of scale 4k + j in bits 2k of byte 8 + j);
* element order: blocks whose every group carries a distinct min (Q2_K) or
  scale (Q3_K), so each output names its group, and single-field probes (one
  2-bit quant, one hmask bit) that must light exactly one element, at the
  position the block layout puts it;
* the GEMV: within float64 of the dequantized weights, and bitwise equal to
  summing the dequantized weights times x in the reference's order (Q2_K: the
  eight terms l + 16k per l; Q3_K: element order).
"""
import numpy as np
import pytest

import oracle as O

F16_ONE, F16_TWO, F16_HALF = 0x3C00, 0x4000, 0x3800


def q2k_block(sc, qs, d16, dmin16):
    return np.concatenate([np.asarray(sc, np.uint8), np.asarray(qs, np.uint8),
                           np.array([d16 & 0xFF, d16 >> 8, dmin16 & 0xFF, dmin16 >> 8], np.uint8)])


def q3k_block(hm, qs, sc12, d16):
    return np.concatenate([np.asarray(hm, np.uint8), np.asarray(qs, np.uint8), np.asarray(sc12, np.uint8),
                           np.array([d16 & 0xFF, d16 >> 8], np.uint8)])


def q3k_pack(s):
    """12-byte field of 16 signed scales s[i] in [-32, 31] (stored + 32)."""
    u = [int(v) + 32 for v in s]
    b = [0] * 12
    for k in range(4):
        for j in range(4):
            i = 4 * k + j
            lo, hi = u[i] & 0xF, u[i] >> 4
            byte = j + (4 if k in (1, 3) else 0)
            b[byte] |= lo << (4 if k >= 2 else 0)
            b[8 + j] |= hi << (2 * k)
    return b


def test_q2k_reference_known_answers(golden):
    for c in golden["q2k_known_answers"]["cases"]:
        blk = q2k_block([c["sc_fill"]] * 16, [c["qs_fill"]] * 64, c["d_f16"], c["dmin_f16"])
        out = O.dequantize(O.Q2_K, blk, 1, 256)[0]
        assert np.all(out == np.float32(c["expected_all"])), c


def test_q3k_reference_known_answers(golden):
    g = golden["q3k_known_answers"]
    assert O.q3k_scales(bytes(g["scales12"])) == [1] * 16
    for c in g["cases"]:
        blk = q3k_block([c["hmask_fill"]] * 32, [c["qs_fill"]] * 64, g["scales12"], c["d_f16"])
        out = O.dequantize(O.Q3_K, blk, 1, 256)[0]
        assert np.all(out == np.float32(c["expected_all"])), c


def test_q3k_scale_unpack_inverts_pack():
    rng = np.random.default_rng(4)
    for _ in range(200):
        s = rng.integers(-32, 32, 16)
        assert O.q3k_scales(bytes(q3k_pack(s))) == s.tolist()
    assert q3k_pack([1] * 16) == [0x11] * 8 + [0xAA] * 4  # the reference test's encoding


def q2k_group(e):
    half, r = divmod(e, 128)
    return half * 8 + r // 16  # scale byte of element e


def test_q2k_each_element_names_its_scale_byte():
    # min nibble n on scale byte n, scale 1, quants 0, dmin 1: out[e] = -n(e)
    blk = q2k_block([(n << 4) | 1 for n in range(16)], [0] * 64, F16_ONE, F16_ONE)
    out = O.dequantize(O.Q2_K, blk, 1, 256)[0]
    assert out.tolist() == [-float(q2k_group(e)) for e in range(256)]


@pytest.mark.parametrize("shift", [0, 2, 4, 6])
def test_q2k_single_quant_probes(shift):
    for i in range(64):
        qs = [0] * 64
        qs[i] = 3 << shift
        blk = q2k_block([(n << 4) | ((n % 15) + 1) for n in range(16)], qs, F16_ONE, 0)
        out = O.dequantize(O.Q2_K, blk, 1, 256)[0]
        half, li = divmod(i, 32)
        r, l = divmod(li, 16)
        e = half * 128 + 16 * (2 * (shift // 2) + r) + l
        assert np.count_nonzero(out) == 1 and out[e] == 3.0 * ((q2k_group(e) % 15) + 1), (i, shift)


def q3k_group(e):
    half, w = divmod(e, 128)
    j, rl = divmod(w, 32)
    return half * 8 + 2 * j + rl // 16


def test_q3k_each_element_names_its_scale():
    s = [g + 1 for g in range(16)]
    blk = q3k_block([0] * 32, [0] * 64, q3k_pack(s), F16_ONE)
    out = O.dequantize(O.Q3_K, blk, 1, 256)[0]
    assert out.tolist() == [-4.0 * s[q3k_group(e)] for e in range(256)]


def test_q3k_single_field_probes():
    sc = q3k_pack([1] * 16)
    base = O.dequantize(O.Q3_K, q3k_block([0] * 32, [0] * 64, sc, F16_ONE), 1, 256)[0]
    assert np.all(base == -4.0)
    for b in range(32):  # hmask byte b, bit t: element (t // 4, t % 4, b // 16, b % 16) gets q = 0
        for t in range(8):
            hm = [0] * 32
            hm[b] = 1 << t
            out = O.dequantize(O.Q3_K, q3k_block(hm, [0] * 64, sc, F16_ONE), 1, 256)[0]
            e = (t // 4) * 128 + (t % 4) * 32 + b
            assert np.count_nonzero(out != -4.0) == 1 and out[e] == 0.0, (b, t)
    for i in range(64):  # qs byte i, bits at shift 2j: element gets q = 3 - 4 = -1
        for j in range(4):
            qs = [0] * 64
            qs[i] = 3 << (2 * j)
            out = O.dequantize(O.Q3_K, q3k_block([0] * 32, qs, sc, F16_ONE), 1, 256)[0]
            half, li = divmod(i, 32)
            e = half * 128 + 32 * j + li
            assert np.count_nonzero(out != -4.0) == 1 and out[e] == -1.0, (i, j)


def random_blocks(qtype, rows, cols, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, O.raw_byte_count(qtype, rows * cols), dtype=np.uint8)
    bb = O.BLOCK_BYTES[qtype]
    blk = raw.reshape(-1, bb)
    d = (rng.uniform(0.5, 2.0, len(blk)) * 1e-3).astype(np.float16).view(np.uint16)
    if qtype == O.Q2_K:
        m = (rng.uniform(0.5, 2.0, len(blk)) * 1e-3).astype(np.float16).view(np.uint16)
        blk[:, 80], blk[:, 81] = d & 0xFF, d >> 8
        blk[:, 82], blk[:, 83] = m & 0xFF, m >> 8
    else:
        blk[:, 108], blk[:, 109] = d & 0xFF, d >> 8
    return raw


def java_order_sum(qtype, w, x):
    """acc += w * x over the elements in the reference's order, fp32."""
    acc = np.float32(0)
    if qtype == O.Q2_K:
        order = [b * 256 + half * 128 + l + 16 * k for b in range(len(w) // 256) for half in range(2)
                 for l in range(16) for k in range(8)]
    else:
        order = range(len(w))
    for e in order:
        acc = np.float32(acc + np.float32(w[e] * x[e]))
    return acc


@pytest.mark.parametrize("qtype", [O.Q2_K, O.Q3_K])
def test_matvec_against_dequantized_weights(qtype):
    rows, cols = 5, 512
    raw = random_blocks(qtype, rows, cols, qtype)
    x = np.random.default_rng(qtype + 1).standard_normal(cols).astype(np.float32)
    W = O.dequantize(qtype, raw, rows, cols)
    y = O.matvec(qtype, raw, x, 0, rows, cols)
    ref = W.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5 * np.abs(W).sum(1).max() * np.abs(x).max())
    for r in range(rows):
        assert y[r] == java_order_sum(qtype, W[r], x), r
    y_rng = O.matvec(qtype, raw, x, 1, 4, cols)
    assert np.array_equal(y_rng, y[1:4])
