"""Pins the CPU oracle (oracle/juno_oracle.c) before it is trusted as the checker.

What pins each oracle function (none of these retypes the oracle's formula):

* f16_to_f32    -- the reference's spot values (GgufReaderTest.java:35-46) and an
                   exhaustive comparison of all 65,536 halves with numpy's float16.
* f32_to_f16    -- numpy float16 round-to-nearest-even on normal results (exact);
                   on the subnormal branch, the documented Java quirk (rounding after
                   a truncating shift) is characterised: it differs from RNE by at most
                   one ulp and only when the first shift discarded non-zero bits.
* java_round    -- exact rational arithmetic (fractions.Fraction), incl. 0.49999997f.
* dequantize    -- Q6_K: the reference's golden block (bit-exact binary fractions);
                   Q4_K/Q5_K/Q8_0: the reference tests' closed forms; all types:
                   quantize -> dequantize round trips bounded by half a step.
* matvec        -- bitwise equal to the fp32 sequential dot of the oracle's own
                   dequantized weights where the Java sums in column order (Q4_K,
                   Q5_K, Q8_0, F32); Q6_K: bitwise equal to the same dot taken in the
                   interleaved (l, l+32, l+64, l+96) order; all: within 1e-5 of a float64
                   dot; the reference tests' known answers (480; 32/128/288 with row ranges).
* quantize      -- unpack(pack) identity of the 6-bit scales; round-trip error bounds;
                   invariants (zero block, all-equal block, d = max/127 for Q8_0).
"""
import fractions
import math
import struct

import numpy as np
import pytest

import oracle as O


def s8(v):
    return np.array(v, dtype=np.int64).astype(np.int8).view(np.uint8)


# ---------------------------------------------------------------- f16 / f32 / round

def test_f16_spot_values(golden):
    for bits, val in golden["f16_to_f32"]["cases"]:
        assert O.f16_to_f32(bits) == val


def test_f16_exhaustive_vs_numpy():
    L = O.lib()
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = halves.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32_bits(int(h)) for h in halves], dtype=np.uint32).view(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # inf / NaN payload: sign | 0x7F800000 | m << 13
    gb = got[nan].view(np.uint32)
    hb = halves[nan].astype(np.uint32)
    assert np.array_equal(gb, ((hb >> 15) << 31) | 0x7F800000 | ((hb & 0x3FF) << 13))


def _f32_from_bits(b):
    return struct.unpack("<f", struct.pack("<I", b & 0xFFFFFFFF))[0]


def test_f32_to_f16_normal_range_matches_rne():
    rng = np.random.default_rng(1)
    # exponents covering the normal fp16 range and the overflow boundary
    vals = (rng.standard_normal(200000) * np.exp2(rng.integers(-14, 17, 200000))).astype(np.float32)
    vals = np.concatenate([vals, np.float32([65504.0, 65519.99, 65520.0, -65520.0, 6.1035156e-05,
                                             1.0, -2.0, 0.25, 0.0, -0.0])])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    normal = (np.abs(vals) >= np.float32(2.0 ** -14)) | (vals == 0)
    assert np.array_equal(got[normal], ref[normal])


def test_f32_to_f16_quirks():
    assert O.f32_to_f16(float("nan")) == 0x7C00          # NaN -> +inf (reference quirk)
    assert O.f32_to_f16(float("inf")) == 0x7C00
    assert O.f32_to_f16(float("-inf")) == 0xFC00
    assert O.f32_to_f16(1e-9) == 0                      # below half of the smallest subnormal


def test_f32_to_f16_subnormal_branch_characterised():
    rng = np.random.default_rng(2)
    exps = rng.integers(-25, -14, 100000)
    vals = (rng.uniform(1, 2, 100000) * np.exp2(exps)).astype(np.float32)
    vals *= np.where(rng.random(100000) < 0.5, -1, 1).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16).astype(np.int64)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], dtype=np.int64)
    diff = np.abs((got & 0x7FFF) - (ref & 0x7FFF))
    assert diff.max() <= 1
    # differences only where the first (truncating) shift discarded set bits
    bits = vals.view(np.uint32).astype(np.int64)
    e = ((bits >> 23) & 0xFF) - 127 + 15
    shift = 1 - e
    mant = (bits & 0x7FFFFF) | 0x800000
    dropped = (mant & ((1 << np.clip(shift, 0, 31)) - 1)) != 0
    assert not np.any((diff == 1) & ~dropped)


@pytest.mark.parametrize("v", [0.0, 0.5, -0.5, 1.5, 2.5, -2.5, 0.49999997, -0.49999997,
                               8388607.5, -8388608.5, 123.456, -7.5, 3e9, -3e9, 1e-30])
def test_java_round_exact(v):
    f = struct.unpack("<f", struct.pack("<f", v))[0]
    exact = math.floor(fractions.Fraction(f) + fractions.Fraction(1, 2))
    exact = max(min(exact, 2**31 - 1), -2**31)
    assert O.java_round(f) == exact


def test_java_round_nan():
    assert O.java_round(float("nan")) == 0


# ---------------------------------------------------------------- golden blocks

def _q6k_block(ql, qh, sc, d16):
    blk = np.zeros(210, dtype=np.uint8)
    blk[:128] = s8(ql)
    blk[128:192] = s8(qh)
    blk[192:208] = s8(sc)
    blk[208:210] = [d16 & 0xFF, d16 >> 8]
    return blk


def test_q6k_golden_block_bit_exact(golden):
    g = golden["q6k_golden_block"]
    blk = _q6k_block(g["ql"], g["qh"], g["sc"], g["d_f16"])
    out = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    for idx, val in g["expected"].items():
        assert out[int(idx)] == np.float32(val), idx  # exact binary fractions


def test_q6k_all_ff_bounded(golden):
    g = golden["q6k_all_ff_bounded"]
    blk = _q6k_block([g["ql_fill"]] * 128, [g["qh_fill"]] * 64, [g["sc_fill"]] * 16, g["d_f16"])
    out = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    assert np.all(np.abs(out) <= g["max_abs"])
    assert np.all(out == 31.0)  # 0xF | 3<<4 = 63 -> 63 - 32 = 31, times d*sc = 1


def _q4k_block(d16, dmin16, sc, qs):
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [d16 & 0xFF, d16 >> 8]
    blk[2:4] = [dmin16 & 0xFF, dmin16 >> 8]
    blk[4:16] = sc
    blk[16:] = qs
    return blk


def test_q4k_all_zero(golden):
    g = golden["q4k_all_zero"]
    blk = _q4k_block(g["d_f16"], g["dmin_f16"], [0] * 12, [0] * 128)
    assert np.all(O.dequantize(O.Q4_K, blk, 1, 256) == 0.0)


def test_q4k_nibble_split(golden):
    g = golden["q4k_nibble_split"]
    qs = [0] * 128
    qs[0] = g["qs0"]
    sc = [0] * 12
    sc[0] = g["sc0"]
    out = O.dequantize(O.Q4_K, _q4k_block(g["d_f16"], g["dmin_f16"], sc, qs), 1, 256)[0]
    assert out[0] == 0.0
    assert out.shape == (256,)


def test_q4k_all_ff_dot_ones(golden):
    g = golden["q4k_all_ff_dot_ones"]
    sc = [0] * 12
    sc[0] = g["sc0"]
    blk = _q4k_block(g["d_f16"], g["dmin_f16"], sc, [g["qs_fill"]] * 128)
    deq = O.dequantize(O.Q4_K, blk, 1, 256)[0]
    assert np.all(deq[:32] == 15.0) and np.all(deq[32:] == 0.0)
    y = O.matvec(O.Q4_K, blk, np.ones(256, np.float32), 0, 1, 256)
    assert y[0] == g["expected_dot_ones"]


def test_q4k_fused_rows_row_ranges(golden):
    g = golden["q4k_fused_rows"]
    sc = [0] * 12
    sc[0] = g["sc0"]
    raw = np.concatenate([_q4k_block(r["d_f16"], 0, sc, [r["qs_fill"]] * 128) for r in g["rows"]])
    x = np.ones(256, np.float32)
    full = O.matvec(O.Q4_K, raw, x, 0, 3, 256)
    assert list(full) == g["expected_dot_ones"]
    for a, b in g["row_ranges"]:
        assert list(O.matvec(O.Q4_K, raw, x, a, b, 256)) == g["expected_dot_ones"][a:b]


def test_q5k_ones(golden):
    g = golden["q5k_ones"]
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = [g["d_f16"] & 0xFF, g["d_f16"] >> 8]
    blk[4] = g["sc0"]
    blk[48:] = g["qs_fill"]
    assert O.matvec(O.Q5_K, blk, np.ones(256, np.float32), 0, 1, 256)[0] == g["expected_dot_ones"]


def test_q8_0_half_i(golden):
    g = golden["q8_0_llamafile"]
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = [g["scale_f16"] & 0xFF, g["scale_f16"] >> 8]
    blk[2:] = np.arange(32)
    out = O.dequantize(O.Q8_0, blk, 1, 32)[0]
    assert np.array_equal(out, 0.5 * np.arange(32, dtype=np.float32))


def test_f32_known_values(golden):
    g = golden["f32_matvec_4x4"]
    m = np.array(g["matrix"], np.float32)
    assert list(O.matvec(O.F32, m.view(np.uint8), np.array(g["x"], np.float32), 0, 4, 4)) == g["expected"]
    g = golden["contract_identity_2x3"]
    m = np.array(g["matrix"], np.float32)
    assert list(O.matvec(O.F32, m.view(np.uint8), np.array(g["x"], np.float32), 0, 2, 3)) == g["expected"]


# ---------------------------------------------------------------- scale pack/unpack

def test_q4k_scale_pack_unpack_identity():
    rng = np.random.default_rng(3)
    for _ in range(2000):
        ls = rng.integers(0, 64, 8)
        lm = rng.integers(0, 64, 8)
        # LoraMerge.java:340-347 packing layout
        sc = [0] * 12
        for j in range(4):
            sc[j] = (ls[j] & 0x3F) | ((ls[j + 4] & 0x30) << 2)
            sc[j + 4] = (lm[j] & 0x3F) | ((lm[j + 4] & 0x30) << 2)
            sc[j + 8] = (ls[j + 4] & 0x0F) | ((lm[j + 4] & 0x0F) << 4)
        b = bytes(int(v) & 0xFF for v in sc)
        assert [O.q4k_scale(b, j) for j in range(8)] == list(ls)
        assert [O.q4k_min(b, j) for j in range(8)] == list(lm)


# ---------------------------------------------------------------- round trips

def _weights(n, seed, outliers=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    if outliers:
        idx = rng.choice(n, n // 100, replace=False)
        w[idx] *= 10
    return w


@pytest.mark.parametrize("outliers", [False, True])
def test_q8_0_round_trip(outliers):
    w = _weights(32 * 512, 4, outliers)
    raw = O.quantize(O.Q8_0, w)
    deq = O.dequantize(O.Q8_0, raw, 1, w.size)[0]
    for b in range(512):
        v = w[b * 32:(b + 1) * 32]
        d = np.float32(np.abs(v).max()) / np.float32(127)
        d16 = O.f16_to_f32(int(raw[b * 34]) | int(raw[b * 34 + 1]) << 8)
        err = np.abs(deq[b * 32:(b + 1) * 32] - v)
        assert err.max() <= 0.5 * d * 1.0001 + 127 * abs(d16 - d) + 1e-12


@pytest.mark.parametrize("qtype,levels", [(O.Q4_K, 15), (O.Q5_K, 31)])
@pytest.mark.parametrize("outliers", [False, True])
def test_kquant_round_trip(qtype, levels, outliers):
    nb = 256
    w = _weights(256 * nb, 5, outliers)
    raw = O.quantize(qtype, w)
    bb = O.BLOCK_BYTES[qtype]
    deq = O.dequantize(qtype, raw, 1, w.size)[0]
    for b in range(nb):
        blk = raw[b * bb:(b + 1) * bb]
        d16 = O.f16_to_f32(int(blk[0]) | int(blk[1]) << 8)
        dm16 = O.f16_to_f32(int(blk[2]) | int(blk[3]) << 8)
        sc = bytes(blk[4:16])
        for s in range(8):
            v = w[b * 256 + s * 32: b * 256 + (s + 1) * 32]
            ls, lm = O.q4k_scale(sc, s), O.q4k_min(sc, s)
            step = d16 * ls
            dq = deq[b * 256 + s * 32: b * 256 + (s + 1) * 32]
            # the quantizer works with fp32 d/dmin; the stored fp16 ones shift the grid
            slack = levels * ls * abs(d16 * 1.0) * 2 ** -10 + lm * abs(dm16) * 2 ** -10
            # the grid is -lm*dmin + step*q, q in [0, levels]: within half a step of it,
            # or clamped at either end (ls / lm are rounded to nearest)
            lo = -lm * dm16
            hi = lo + levels * step
            bound = (0.5 * step + slack + max(0.0, float(v.max()) - hi)
                     + max(0.0, lo - float(v.min())) + 1e-7)
            assert np.abs(dq - v).max() <= bound + 0.05 * step, (b, s)
    # global quality: relative RMS error well below the 4/5-bit step
    rel = np.sqrt(np.mean((deq - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert rel < (0.12 if qtype == O.Q4_K else 0.06)


@pytest.mark.parametrize("outliers", [False, True])
def test_q6k_round_trip(outliers):
    nb = 256
    w = _weights(256 * nb, 6, outliers)
    raw = O.quantize(O.Q6_K, w)
    deq = O.dequantize(O.Q6_K, raw, 1, w.size)[0]
    for b in range(nb):
        blk = raw[b * 210:(b + 1) * 210]
        d16 = O.f16_to_f32(int(blk[208]) | int(blk[209]) << 8)
        sc = blk[192:208].view(np.int8)
        for s in range(16):
            # sub-block s covers (half, quad, l/16) per LoraMerge.java:455-458
            idx = [p for p in range(256)
                   if (p // 128) * 8 + ((p % 128) % 32) // 16 + ((p % 128) // 32) * 2 == s]
            v = w[b * 256 + np.array(idx)]
            dq = deq[b * 256 + np.array(idx)]
            step = abs(d16 * float(sc[s]))
            # grid step*q, q in [-32, 31]; sc is rounded to nearest so the ends may clamp;
            # the stored fp16 d shifts the grid by at most 32 * step * 2^-11
            bound = (0.5 * step + max(0.0, float(np.abs(v).max()) - 31 * step)
                     + 32 * step * 2 ** -10 + 1e-7)
            assert np.abs(dq - v).max() <= bound, (b, s)
    rel = np.sqrt(np.mean((deq - w) ** 2)) / np.sqrt(np.mean(w ** 2))
    assert rel < 0.05


def test_quantize_zero_block():
    for t in (O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K):
        raw = O.quantize(t, np.zeros(256, np.float32))
        if t != O.Q6_K:  # Q6_K stores q + 32, so its zero block is not all-zero bytes
            assert not raw.any()
        assert np.all(O.dequantize(t, raw, 1, 256) == 0.0)


# ---------------------------------------------------------------- matvec

def _dot_seq(w_row, x):
    acc = np.float32(0)
    for a, b in zip(w_row, x):
        acc = np.float32(acc + np.float32(a * b))
    return acc


@pytest.mark.parametrize("qtype", [O.Q4_K, O.Q5_K, O.Q8_0])
def test_matvec_equals_dequant_dot_bitwise(qtype):
    rows, cols = 6, 512
    w = _weights(rows * cols, 7)
    x = np.random.default_rng(8).standard_normal(cols).astype(np.float32)
    raw = O.quantize(qtype, w)
    deq = O.dequantize(qtype, raw, rows, cols)
    y = O.matvec(qtype, raw, x, 0, rows, cols)
    for r in range(rows):
        assert y[r] == _dot_seq(deq[r], x)


def test_matvec_q6k_interleaved_order_bitwise():
    rows, cols = 4, 512
    w = _weights(rows * cols, 9)
    x = np.random.default_rng(10).standard_normal(cols).astype(np.float32)
    raw = O.quantize(O.Q6_K, w)
    deq = O.dequantize(O.Q6_K, raw, rows, cols)
    order = [b * 256 + h * 128 + l + k * 32 for b in range(cols // 256) for h in range(2)
             for l in range(32) for k in range(4)]
    y = O.matvec(O.Q6_K, raw, x, 0, rows, cols)
    for r in range(rows):
        assert y[r] == _dot_seq(deq[r][order], x[order])


@pytest.mark.parametrize("qtype", [O.F32, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_matvec_vs_float64(qtype):
    rows, cols = 64, 2048
    w = _weights(rows * cols, 11)
    x = np.random.default_rng(12).standard_normal(cols).astype(np.float32)
    raw = O.quantize(qtype, w)
    deq = O.dequantize(qtype, raw, rows, cols).astype(np.float64)
    ref = deq @ x.astype(np.float64)
    y = O.matvec(qtype, raw, x, 0, rows, cols)
    scale = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - ref) <= 1e-5 * scale)


def test_matvec_thread_count_invariant():
    rows, cols = 300, 1024
    raw = O.quantize(O.Q4_K, _weights(rows * cols, 13))
    x = np.random.default_rng(14).standard_normal(cols).astype(np.float32)
    a = O.matvec(O.Q4_K, raw, x, 0, rows, cols, nthreads=1)
    b = O.matvec(O.Q4_K, raw, x, 0, rows, cols, nthreads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_raw_byte_count():
    # GgufReader.rawByteCount (GgufReader.java:347-360); PhiQuantizedMatVecTest.java:174-189
    assert O.raw_byte_count(O.Q4_K, 256 * 32) == 32 * 144
    assert O.raw_byte_count(O.Q6_K, 256) == 210
    assert O.raw_byte_count(O.Q8_0, 32) == 34
    assert O.raw_byte_count(O.Q5_K, 256) == 176
    assert O.raw_byte_count(O.F32, 10) == 40
