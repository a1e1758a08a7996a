"""The kernels' address arithmetic replayed on the CPU (no GPU): every global
load and store and every LDS window access of the batched MFMA kernel
(jh_mfma.hip gemm_body / mfma_px), the staged B = 1 kernel
(jh_gemv_staged.hip) and the one-shot kernels (jh_gemv.hip), for every
BASELINE shape, batch and row range, must stay inside the buffer it targets.

Each model below restates one kernel's index formulas with its file:line, per
lane, wave, workgroup and step (numpy over all of them at once, at the extreme
steps), and asserts the byte range it touches against the allocation: a packed
matrix is rows x pitch bytes plus kTailPad (256) bytes of zeros
(jh_kernels.hpp:12); x is B x cols floats; y, the split-K partials, the
counters and the prepared-x slabs are sized by the planner's own formulas.
The MFMA model's plan (K split, prepared x or not) is checked against the
library's planner (jh_qmatvec_batched_plan), so the model walks the same
launches the library makes.

It was written for an unexplained hipErrorIllegalAddress seen once on the
first eager B = 32 MFMA launch of a bench run: it finds every access of the
current kernels in bounds at every benchmark configuration.
"""
import ctypes

import numpy as np
import pytest

from juno_amd import _lib

TAIL = 256  # kTailPad, jh_kernels.hpp:12
Q4_K, Q5_K, Q6_K, Q8_0, Q2_K, Q3_K = 12, 13, 14, 8, 10, 11
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110)}


def pitch(t, cols):
    qk, bb = BLOCK[t]
    return cols // qk * bb


# TinyLlama (config 1 and 2), Llama-3-8B (3 and 4), Phi-3-mini (5)
SHAPES = sorted({
    (Q4_K, 5632, 2048), (Q4_K, 2048, 2048), (Q4_K, 256, 2048), (Q6_K, 256, 2048), (Q6_K, 2048, 5632),
    (Q6_K, 32000, 2048),
    (Q4_K, 4096, 4096), (Q4_K, 1024, 4096), (Q6_K, 1024, 4096), (Q4_K, 14336, 4096), (Q6_K, 4096, 14336),
    (Q6_K, 128256, 4096),
    (Q8_0, 9216, 3072), (Q8_0, 3072, 3072), (Q8_0, 16384, 3072), (Q8_0, 3072, 8192), (Q8_0, 32064, 3072),
    (Q6_K, 9216, 3072), (Q6_K, 3072, 3072), (Q6_K, 16384, 3072), (Q6_K, 3072, 8192), (Q6_K, 32064, 3072),
    (Q5_K, 3072, 3072), (Q2_K, 2048, 2048), (Q3_K, 2048, 2048), (Q4_K, 333, 768), (Q6_K, 333, 768),
})


def ranges(rows):
    out = {(0, rows), (1, rows), (0, rows - 1), (rows // 3, rows - rows // 5)}
    return sorted((a, b) for a, b in out if 0 <= a < b <= rows)


def within(lo, hi, size, what):
    lo, hi = int(np.min(lo)), int(np.max(hi))
    assert lo >= 0 and hi <= size, f"{what}: bytes [{lo}, {hi}) outside [0, {size})"


# ------------------------------------------------------------------ batched MFMA kernel (jh_mfma.hip)
# Format constants: kBytes / kChunks / kRowChunks (jh_mfma.hip:293-295, 391-395, 451-453, 499-501, 561-563)
MF = {Q4_K: (144, 9, 9), Q5_K: (176, 11, 11), Q6_K: (210, 14, 15), Q8_0: (272, 19, 20), Q2_K: (84, 6, 7),
      Q3_K: (110, 8, 9)}
ROWS_PER_WAVE, WAVES, ROWS_PER_WG, MIN_WG, COUNTER_SLOTS = 32, 8, 256, 256, 1024  # jh_mfma.hip:52-56, jh_kernels.hpp:149
XPAD = 8
COLH = 256 + XPAD
SLAB_BYTES, SLAB_ROWS = 34 * 1024, 34
WIN_PAD = 16


def plan(tiles_list, nsb, B, types):
    """plan_group (jh_mfma.hip:1206-1241): the K split by its cost model."""
    tiles = sum(tiles_list)
    best, ksb, ksplit = 1 << 30, nsb, 1
    for ks in range(1, nsb + 1):
        kb = (nsb + ks - 1) // ks
        kse = (nsb + kb - 1) // kb
        if kse > 1 and tiles > COUNTER_SLOTS:
            break
        rounds = (tiles * kse + MIN_WG - 1) // MIN_WG
        cost = 4 * (rounds * (kb + 5) + (1 if kse > 1 else 0)) + (kse if kse > 1 else 0)
        if cost < best:
            best, ksb, ksplit = cost, kb, kse
    prepared = len(tiles_list) == 1 and ksplit == 1 and B <= 32 and types[0] not in (Q2_K, Q3_K)
    return ksb, ksplit, prepared


def lds_w_offset(nt):  # jh_mfma.hip:748
    return (2 * 32 * nt * COLH + 32 * nt * 16 + 32 * nt * 32) * 2 + 32 * nt * 8


def lds_bytes(nt, types):  # jh_mfma.hip:750-753
    return (2 if nt == 1 else 1) * lds_w_offset(nt) + WAVES * ROWS_PER_WAVE * max(MF[t][2] for t in types) * 16 + WIN_PAD


def win_chunk(j, ch, rc):  # jh_mfma.hip:278-279
    return j + (rc - ch) * (j // ch)


def check_mfma_weights(t, rows_alloc, p, row0, nrows, tiles, sb_ranges, nt, lds_total, prepared):
    """Weight chunk loads (JH_LOAD_W, jh_mfma.hip:874-879 / 1136-1140) and the
    window writes and field reads (:939-945, 964-969)."""
    kbytes, ch, rc_fmt = MF[t]
    rc = rc_fmt if (nt == 1) else ch  # RC: padded window rows at NT = 1 (jh_mfma.hip:867)
    if prepared:
        rc = rc_fmt                      # mfma_px always uses the padded rows (:1106)
    cl = (ROWS_PER_WAVE * ch + 63) // 64
    lane = np.arange(64)
    k = np.arange(cl)
    j = np.minimum(lane[:, None] + 64 * k[None, :], ROWS_PER_WAVE * ch - 1)           # (64, CL)
    tile = np.arange(tiles)[:, None, None, None]
    wave = np.arange(WAVES)[None, :, None, None]
    rbase = tile * ROWS_PER_WG + wave * ROWS_PER_WAVE
    row = row0 + np.minimum(rbase + j[None, None] // ch, nrows - 1)                   # row_off (:858)
    coff = row * p + 16 * (j[None, None] % ch)
    alloc = rows_alloc * p + TAIL
    for sb0, sb1 in sb_ranges:
        for sb in {sb0, sb1 - 1}:
            a = (coff + sb * kbytes) & ~15
            within(a, a + 16, alloc, f"mfma weights type {t} sb {sb}")
            # the lane's own block inside its window: myoff + sb*kBytes, misalignment 0..15,
            # fields read up to kBytes plus one dword of realignment (lds_read_u, :255-263)
            myoff = (row0 + np.minimum(rbase[:, :, 0, 0][..., None] + (lane & 31)[None, None, :], nrows - 1)) * p
            mis = (myoff + sb * kbytes) & 15
            lr = lane & 31
            start = lds_w_offset(nt) * (1 if (nt == 2 or prepared) else 2) \
                + wave[:, :, 0, 0][..., None] * (ROWS_PER_WAVE * rc * 16) + lr[None, None, :] * rc * 16 + mis
            if prepared:  # mfma_px: the windows are an array of their own (sh_w, jh_mfma.hip:1106)
                start = start - lds_w_offset(nt)
                within(start, start + kbytes + 4, WAVES * ROWS_PER_WAVE * rc * 16 + WIN_PAD, f"px window type {t}")
            else:
                within(start, start + kbytes + 4, lds_total, f"mfma window read type {t}")
    wpos = win_chunk(j, ch, rc)
    if not prepared:
        base = lds_w_offset(nt) * (2 if nt == 1 else 1)
        w = base + WAVES * 0 + (np.arange(WAVES)[:, None, None] * ROWS_PER_WAVE * rc * 16) + 16 * wpos[None]
        live = (lane[:, None] + 64 * k[None, :]) < ROWS_PER_WAVE * ch
        within(w[:, live], w[:, live] + 16, lds_total, f"mfma window write type {t}")


@pytest.mark.parametrize("t,rows,cols", [s for s in SHAPES if s[2] % 256 == 0])
def test_mfma_addresses(t, rows, cols):
    L = _lib.load()
    p = pitch(t, cols)
    nsb = cols // 256
    for B in (3, 8, 16, 20, 31, 32, 33, 48, 64):
        nt = 1 if B <= 32 else 2
        for r0, r1 in ranges(rows):
            nrows = r1 - r0
            tiles = (nrows + ROWS_PER_WG - 1) // ROWS_PER_WG
            ksb, ksplit, prepared = plan([tiles], nsb, B, [t])
            # the library plans the same launch (jh_qmatvec_batched_plan: kernel 2 = prepared x, 1 = grouped)
            kern, ks = ctypes.c_int(), ctypes.c_int()
            assert L.jh_qmatvec_batched_plan_shape(t, cols, r0, r1, B, ctypes.byref(kern), ctypes.byref(ks)) == 0
            assert (kern.value, ks.value) == (2 if prepared else 1, ksplit), (t, rows, cols, B, r0, r1)
            sb_ranges = [(sp * ksb, min(nsb, sp * ksb + ksb)) for sp in range(ksplit)]
            sb_ranges = [r for r in sb_ranges if r[0] < r[1]]
            lds_total = lds_bytes(nt, [t])
            assert lds_total <= 160 * 1024
            check_mfma_weights(t, rows, p, r0, nrows, tiles, sb_ranges, nt, lds_total, prepared)
            # x: X + min(b, B-1)*cols + SB*256 + 16*xq + 4k (JH_LOAD_X, :880-890): in [0, B*cols)
            bmax = min(32 * nt - 1, B - 1)
            within(0, (bmax * cols + (nsb - 1) * 256 + 16 * 15 + 16) * 4, B * cols * 4, "x")
            # y and the split-K partials (store_tile, :626-700): b < B, r < nrows, splits < ksplit
            within(0, ((B - 1) * nrows + nrows) * 4, B * nrows * 4, "y")
            if ksplit > 1:
                plane = B * nrows
                within(0, ((ksplit - 1) * plane + (B - 1) * nrows + nrows) * 4, ksplit * B * nrows * 4, "partials")
                assert tiles <= COUNTER_SLOTS  # a counter per tile (:1228)
            if prepared:  # x_prep slabs and the DMA rows (:1040-1054, :1119-1128)
                r = np.minimum(np.arange(WAVES)[:, None] + WAVES * np.arange((SLAB_ROWS + WAVES - 1) // WAVES), SLAB_ROWS - 1)
                src = (nsb - 1) * SLAB_BYTES + 16 * 63 + 1024 * r
                within(src, src + 16, nsb * SLAB_BYTES, "prepared x slab DMA source")
                within(1024 * r, 1024 * r + 16 * 64, SLAB_BYTES, "prepared x slab DMA target")


# ------------------------------------------------------------------ staged B = 1 kernel (jh_gemv_staged.hip)
# Fmt (jh_gemv_staged.hip:256-259): QK, BB, LPB, TBMAX, CH (16-byte chunks per row tile)
SF = {Q4_K: (256, 144, 4, 16, 145), Q5_K: (256, 176, 4, 16, 177), Q6_K: (256, 210, 4, 16, 212), Q8_0: (32, 34, 1, 64, 138)}


def staged_layouts(t, cols):
    qk, bb, lpb, tbmax, ch = SF[t]
    nb = cols // qk
    gw = 1 if nb <= tbmax else 2 if nb <= 2 * tbmax else 4  # launch_staged_t
    tb = (nb + gw - 1) // gw
    return nb, gw, tb


@pytest.mark.parametrize("t,rows,cols", [s for s in SHAPES if s[0] in SF])
def test_staged_addresses(t, rows, cols):
    qk, bb, lpb, tbmax, ch = SF[t]
    p = pitch(t, cols)
    nb, gw, tb = staged_layouts(t, cols)
    if nb > 4 * tbmax:
        pytest.skip("wider than the staged kernel takes (staged_supported)")
    K = (ch + 63) // 64                                     # loads per lane per row (:639)
    lane = np.arange(64)
    for r0, r1 in ranges(rows):
        nrows = r1 - r0
        for tile in range(gw):
            b0 = tile * tb
            ntile = min(tb, nb - b0)
            tile_bytes = ntile * bb
            nch = (15 + tile_bytes + 15) >> 4               # :672
            ld = 16 * np.minimum(lane[:, None] + 64 * np.arange(K)[None, :], nch - 1)
            assert nch <= ch, (t, cols, tile)  # every loaded chunk is parked (park: chunks < CH, :767-772)
            for vr in {0, nrows - 1}:                        # issue(): rows clamped to nrows - 1 (:743-752)
                off = (r0 + vr) * p + b0 * bb
                base = off & ~15
                within(base + ld, base + ld + 16, rows * p + TAIL, f"staged weights type {t} tile {tile}")
            # block_dot reads a block's fields from the parked row at lane_blk + cstart (cstart =
            # the row's misalignment mod 16); the last byte read past the block's start:
            # Q4_K / Q5_K the block, Q6_K dwords 0..53 of the dword-aligned start (lds_word reads
            # w[k + 1], :78-80; d at word 52), Q8_0 dwords up to 9 (:540-545)
            act_blk = (lane // lpb) < ntile
            lane_blk = np.where(act_blk, lane // lpb, 0) * bb
            field_end = {Q4_K: 144, Q5_K: 176, Q6_K: 216, Q8_0: 40}[t]
            cstart = 15 if t in (Q6_K, Q8_0) else 0  # K-quant rows are 16-byte aligned (pitch 144 / 176 x n)
            within(lane_blk, lane_blk + cstart + field_end, 16 * ch, f"staged block fields type {t}")
        # x (x_load4, :104-106): c clamped to cols - 4, so [0, cols) floats
        within(0, cols * 4, cols * 4, "staged x")


# ------------------------------------------------------------------ one-shot kernels (jh_gemv.hip)
@pytest.mark.parametrize("t,rows,cols", SHAPES)
def test_one_shot_addresses(t, rows, cols):
    """gemv_q4k_body and its siblings: row pointers clamped to nrows - 1
    (jh_gemv.hip:56-57), blocks b < nb, each field read inside its block except
    the dword realignment of 2-byte-aligned Q6_K / Q8_0 / Q3_K fields, which reads
    at most 6 bytes past a block (covered by the tail padding)."""
    qk, bb = BLOCK[t]
    p = pitch(t, cols)
    nb = cols // qk
    over = {Q4_K: 0, Q5_K: 0, Q6_K: 6, Q8_0: 6, Q2_K: 0, Q3_K: 6}[t]
    for r0, r1 in ranges(rows):
        last = (r1 - 1) * p + (nb - 1) * bb
        within(r0 * p, last + bb + over, rows * p + TAIL, f"one-shot type {t}")
