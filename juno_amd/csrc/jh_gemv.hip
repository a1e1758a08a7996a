// jh_gemv.hip -- fused dequant-GEMV kernels for gfx950 on packed GGUF blocks.
//
// y[j][r] = sum_c deq(W[r][c]) * x[j][c] for a small batch of B vectors
// (B = 1 is the decode GEMV).  The weights are streamed from HBM exactly once
// in their packed layout; dequantization happens in registers.
//
// Work split (all quantized kernels): a workgroup is 4 wavefronts, a
// wavefront owns R consecutive rows, and its 64 lanes sweep the row's blocks
// as 8 blocks x 8 lanes per step.  All R rows share each lane's x values, so
// x is read R times less than the weights would require.  Per-lane partial
// sums are reduced with DPP (jh::wave_sum).
//
// Numerics.  The Java path (LlamaTransformerHandler.java:1428-1468,
// 1486-1508, 1587-1638) sums (scale*q - min)*x per element in fp32.  Here
// each sub-block is folded as  scale * sum(q*x) - min * sum(x)  (fp32 FMAs),
// which is the same sum in another order; the difference is order-of-
// summation rounding only (bar: max rel-err 1e-3 against the Java path).
// Quants with an offset (Q6_K u - 32, Q3_K q - 4) or a sign (Q8_0) enter as signed values
// (a signed bit-field extract of the offset-flipped field), never as
// sum(u*x) - 32 * sum(x): that difference cancels in fp32 when x has an
// outlier over a zero weight.
#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {

// The signed W-bit field of w at bit off, by shifts (the compiler treated the
// result of __builtin_amdgcn_sbfe as non-negative and converted it to float
// as unsigned).
template <int W>
__device__ __forceinline__ int sfield(uint32_t w, int off) {
    return (int)(w << (32 - W - off)) >> (32 - W);
}

// ---------------------------------------------------------------- Q4_K / Q5_K
// Lane (kb, ch): block b = step*8 + kb, 16-byte qs chunk ch of that block.
// Chunk ch covers group g = ch/2, elements 16*(ch&1) .. +16 of sub-block 2g
// (low nibbles) and of sub-block 2g+1 (high nibbles).  Q5_K (Q5 = true,
// matVecQ5Kraw, LlamaTransformerHandler.java:1525-1576) adds the 5th bits:
// bit 2g / 2g+1 of qh[l] for the same 16 elements l.
template <int R, int B, bool Q5 = false>
__device__ __forceinline__ void gemv_q4k_body(int wg, const uint8_t *__restrict__ W, size_t pitch, int nb,
                                                int nrows, const float *__restrict__ X, int ldx,
                                                float *__restrict__ Y, int ldy, float ysc = 1.f) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (wg * 4 + wave) * R;
    if (r0 >= nrows) return;
    const int kb = lane >> 3, ch = lane & 7, g = ch >> 1, hf = ch & 1;

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) acc[i][j] = 0.f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int i = 0; i < R; i++) rowp[i] = W + (size_t)min(r0 + i, nrows - 1) * pitch;

    constexpr int kBB = Q5 ? 176 : 144, kQs = Q5 ? 48 : 16;
    for (int b = kb; b < nb; b += 8) {
        uint4 hdr[R], qs[R], qh[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t *bp = rowp[i] + (size_t)b * kBB;
            hdr[i] = *reinterpret_cast<const uint4 *>(bp);
            qs[i] = load_stream16(bp + kQs + ch * 16);
            if (Q5) qh[i] = *reinterpret_cast<const uint4 *>(bp + 16 + hf * 16);
        }
        const int xo = b * 256 + g * 64 + hf * 16;
        float xl[B][16], xh[B][16], sl[B], sh[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const float *xp = X + (size_t)j * ldx + xo;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float4 a = load_f4(xp + 4 * k), c = load_f4(xp + 32 + 4 * k);
                xl[j][4 * k] = a.x; xl[j][4 * k + 1] = a.y; xl[j][4 * k + 2] = a.z; xl[j][4 * k + 3] = a.w;
                xh[j][4 * k] = c.x; xh[j][4 * k + 1] = c.y; xh[j][4 * k + 2] = c.z; xh[j][4 * k + 3] = c.w;
            }
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int k = 0; k < 16; k++) { s0 += xl[j][k]; s1 += xh[j][k]; }
            sl[j] = s0;
            sh[j] = s1;
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float d = half_bits_to_float(hdr[i].x), dmin = half_bits_to_float(hdr[i].x >> 16);
            int ls0, lm0, ls1, lm1;
            q4k_scale_min(hdr[i].y, hdr[i].z, hdr[i].w, 2 * g, ls0, lm0);
            q4k_scale_min(hdr[i].y, hdr[i].z, hdr[i].w, 2 * g + 1, ls1, lm1);
            const float sc0 = d * (float)ls0, mn0 = dmin * (float)lm0;
            const float sc1 = d * (float)ls1, mn1 = dmin * (float)lm1;
            const uint32_t w[4] = {qs[i].x, qs[i].y, qs[i].z, qs[i].w};
            const uint32_t h5[4] = {qh[i].x, qh[i].y, qh[i].z, qh[i].w};
#pragma unroll
            for (int j = 0; j < B; j++) {
                float dl = 0.f, dh = 0.f;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t lo = w[k] & 0x0F0F0F0Fu, hi = (w[k] >> 4) & 0x0F0F0F0Fu;
                    if (Q5) {
                        lo |= ((h5[k] >> (2 * g)) & 0x01010101u) << 4;
                        hi |= ((h5[k] >> (2 * g + 1)) & 0x01010101u) << 4;
                    }
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        dl = fmaf((float)byte_of(lo, e), xl[j][4 * k + e], dl);
                        dh = fmaf((float)byte_of(hi, e), xh[j][4 * k + e], dh);
                    }
                }
                float a = acc[i][j];
                a = fmaf(sc0, dl, a);
                a = fmaf(-mn0, sl[j], a);
                a = fmaf(sc1, dh, a);
                a = fmaf(-mn1, sh[j], a);
                acc[i][j] = a;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) {
            float s = wave_sum(acc[i][j]);
            if (lane == 0 && r0 + i < nrows) Y[(size_t)j * ldy + r0 + i] = s * ysc;
        }
}

// ---------------------------------------------------------------- Q6_K
// Lane (kb, ch): block b = step*8 + kb; half h = ch/4, l0 = 8*(ch&3).  The lane
// covers l in [l0, l0+8) of that half for all four quads (elements l, l+32,
// l+64, l+96), i.e. 32 weights, reading 8 bytes each of ql[l], ql[l+32], qh[l].
template <int R, int B>
__device__ __forceinline__ void gemv_q6k_body(int wg, const uint8_t *__restrict__ W, size_t pitch, int nb,
                                                int nrows, const float *__restrict__ X, int ldx,
                                                float *__restrict__ Y, int ldy, float ysc = 1.f) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (wg * 4 + wave) * R;
    if (r0 >= nrows) return;
    const int kb = lane >> 3, ch = lane & 7, h = ch >> 2, l0 = (ch & 3) * 8, is = l0 >> 4;

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) acc[i][j] = 0.f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int i = 0; i < R; i++) rowp[i] = W + (size_t)min(r0 + i, nrows - 1) * pitch;

    // One step's loads and arithmetic.  A row of 16 blocks is two steps per lane;
    // both steps' loads go out before either is computed, so the row is one
    // memory round trip (8B-shaped Q6_K 4096 x 4096: 8.9 -> 7.4 us).
    struct Step {
        uint2 qa[R], qb[R], qh[R], scw[R];
        uint32_t dw[R];
        float xv[B][4][8];
    };
    auto load = [&](int b, Step &t) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t *bp = rowp[i] + (size_t)b * 210;
            t.qa[i] = load8_a2(bp + h * 64 + l0);
            t.qb[i] = load8_a2(bp + h * 64 + 32 + l0);
            t.qh[i] = load8_a2(bp + 128 + h * 32 + l0);
            t.scw[i] = load8_a2(bp + 192 + h * 8);
            const uint8_t *dp = bp + 208;
            uintptr_t a = reinterpret_cast<uintptr_t>(dp);
            uint32_t w = *reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
            t.dw[i] = w >> (8 * (a & 3u));
        }
        // x runs for quads k = 0..3: x[b*256 + h*128 + k*32 + l0 .. +8]
#pragma unroll
        for (int j = 0; j < B; j++) {
            const float *xp = X + (size_t)j * ldx + b * 256 + h * 128 + l0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float4 a = load_f4(xp + 32 * k), c = load_f4(xp + 32 * k + 4);
                t.xv[j][k][0] = a.x; t.xv[j][k][1] = a.y; t.xv[j][k][2] = a.z; t.xv[j][k][3] = a.w;
                t.xv[j][k][4] = c.x; t.xv[j][k][5] = c.y; t.xv[j][k][6] = c.z; t.xv[j][k][7] = c.w;
            }
        }
    };
    auto compute = [&](const Step &t) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float d = half_bits_to_float(t.dw[i]);
            // scales sc[h*8 + is + 2k], k = 0..3 (signed bytes)
            float dk[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int idx = is + 2 * k;
                const uint32_t word = idx < 4 ? t.scw[i].x : t.scw[i].y;
                const int s8 = (int)(int8_t)byte_of(word, idx & 3);
                dk[k] = d * (float)s8;
            }
            uint32_t u[4][2];
#pragma unroll
            for (int tt = 0; tt < 2; tt++) {
                const uint32_t a = tt ? t.qa[i].y : t.qa[i].x, c = tt ? t.qb[i].y : t.qb[i].x,
                               e = tt ? t.qh[i].y : t.qh[i].x;
                // 6-bit u with bit 5 flipped: as a signed 6-bit field it is u - 32
                u[0][tt] = ((a & 0x0F0F0F0Fu) | ((e << 4) & 0x30303030u)) ^ 0x20202020u;
                u[1][tt] = ((c & 0x0F0F0F0Fu) | ((e << 2) & 0x30303030u)) ^ 0x20202020u;
                u[2][tt] = (((a >> 4) & 0x0F0F0F0Fu) | (e & 0x30303030u)) ^ 0x20202020u;
                u[3][tt] = (((c >> 4) & 0x0F0F0F0Fu) | ((e >> 2) & 0x30303030u)) ^ 0x20202020u;
            }
#pragma unroll
            for (int j = 0; j < B; j++) {
                float a = acc[i][j];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float dot = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++)  // q = u - 32
                        dot = fmaf((float)sfield<6>(u[k][e >> 2], 8 * (e & 3)), t.xv[j][k][e], dot);
                    a = fmaf(dk[k], dot, a);
                }
                acc[i][j] = a;
            }
        }
    };
    if (nb <= 8) {  // one step per lane-block
        for (int b = kb; b < nb; b += 8) {
            Step t;
            load(b, t);
            compute(t);
        }
    } else {
        for (int b = kb; b < nb; b += 16) {
            const bool two = b + 8 < nb;  // the second step's loads are clamped, its arithmetic skipped
            Step t0, t1;
            load(b, t0);
            load(two ? b + 8 : b, t1);
            compute(t0);
            if (two) compute(t1);
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) {
            float s = wave_sum(acc[i][j]);
            if (lane == 0 && r0 + i < nrows) Y[(size_t)j * ldy + r0 + i] = s * ysc;
        }
}

// ---------------------------------------------------------------- Q2_K
// matVecQ2Kraw (LlamaTransformerHandler.java:1303-1346), block [sc 16][qs 64][d][dmin].
// Lane (kb, ch): block b = step*8 + kb; half h = ch/4, r = (ch/2)&1, l0 = 8*(ch&1).
// The 8 qs bytes [32h + 16r + l0, +8) at shift 2j (j = 0..3) are the elements
// h*128 + 16(2j + r) + l, l in [l0, l0+8), with scale byte sc[8h + 2j + r]
// (low nibble scale, high nibble min): w = (d*scale)*q - dmin*min.  Folded per
// run as d*scale*sum(q*x) - dmin*min*sum(x).
template <int R, int B>
__device__ __forceinline__ void gemv_q2k_body(int wg, const uint8_t *__restrict__ W, size_t pitch, int nb,
                                                int nrows, const float *__restrict__ X, int ldx,
                                                float *__restrict__ Y, int ldy, float ysc = 1.f) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (wg * 4 + wave) * R;
    if (r0 >= nrows) return;
    const int kb = lane >> 3, ch = lane & 7, h = ch >> 2, r = (ch >> 1) & 1, l0 = (ch & 1) * 8;

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) acc[i][j] = 0.f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int i = 0; i < R; i++) rowp[i] = W + (size_t)min(r0 + i, nrows - 1) * pitch;

    for (int b = kb; b < nb; b += 8) {
        uint2 q[R], sc[R];
        uint32_t dm[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t *bp = rowp[i] + (size_t)b * 84;  // 4-byte aligned: 84 = 4 * 21
            q[i] = load8_a2(bp + 16 + 32 * h + 16 * r + l0);
            sc[i] = load8_a2(bp + 8 * h);
            dm[i] = *reinterpret_cast<const uint32_t *>(bp + 80);
        }
        float xv[B][4][8], sx[B][4];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const float *xp = X + (size_t)j * ldx + b * 256 + h * 128 + 16 * r + l0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float4 a = load_f4(xp + 32 * k), c = load_f4(xp + 32 * k + 4);
                xv[j][k][0] = a.x; xv[j][k][1] = a.y; xv[j][k][2] = a.z; xv[j][k][3] = a.w;
                xv[j][k][4] = c.x; xv[j][k][5] = c.y; xv[j][k][6] = c.z; xv[j][k][7] = c.w;
                float s = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) s += xv[j][k][e];
                sx[j][k] = s;
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float d = half_bits_to_float(dm[i]), dmin = half_bits_to_float(dm[i] >> 16);
            float dsc[4], dmn[4];
            uint32_t u[4][2];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int idx = 2 * k + r;  // scale byte within the half
                const uint32_t sb = byte_of(idx < 4 ? sc[i].x : sc[i].y, idx & 3);
                dsc[k] = d * (float)(sb & 15u);
                dmn[k] = dmin * (float)(sb >> 4);
                u[k][0] = (q[i].x >> (2 * k)) & 0x03030303u;
                u[k][1] = (q[i].y >> (2 * k)) & 0x03030303u;
            }
#pragma unroll
            for (int j = 0; j < B; j++) {
                float a = acc[i][j];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float dot = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        dot = fmaf((float)byte_of(u[k][e >> 2], e & 3), xv[j][k][e], dot);
                    a = fmaf(dsc[k], dot, a);
                    a = fmaf(-dmn[k], sx[j][k], a);
                }
                acc[i][j] = a;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) {
            float s = wave_sum(acc[i][j]);
            if (lane == 0 && r0 + i < nrows) Y[(size_t)j * ldy + r0 + i] = s * ysc;
        }
}

// ---------------------------------------------------------------- Q3_K
// matVecQ3Kraw (LlamaTransformerHandler.java:1358-1425), block [hmask 32][qs 64][scales 12][d].
// Lane (kb, ch): block b = step*8 + kb; half h = ch/4, r = (ch/2)&1, l0 = 8*(ch&1).
// Elements h*128 + 32j + 16r + l (j = 0..3, l in [l0, l0+8)) take the 2 bits at
// shift 2j of qs[32h + 16r + l], bit 4h + j of hmask[16r + l] and the signed
// scale sc[8h + 2j + r]: w = (d*sc) * (q - 4), folded as d*sc*sum((q - 4)*x).
// Blocks are 2-byte aligned (110 bytes).
template <int R, int B>
__device__ __forceinline__ void gemv_q3k_body(int wg, const uint8_t *__restrict__ W, size_t pitch, int nb,
                                                int nrows, const float *__restrict__ X, int ldx,
                                                float *__restrict__ Y, int ldy, float ysc = 1.f) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (wg * 4 + wave) * R;
    if (r0 >= nrows) return;
    const int kb = lane >> 3, ch = lane & 7, h = ch >> 2, r = (ch >> 1) & 1, l0 = (ch & 1) * 8;

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) acc[i][j] = 0.f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int i = 0; i < R; i++) rowp[i] = W + (size_t)min(r0 + i, nrows - 1) * pitch;

    for (int b = kb; b < nb; b += 8) {
        uint2 q[R], hm[R], a01[R], a2d[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t *bp = rowp[i] + (size_t)b * 110;
            q[i] = load8_a2(bp + 32 + 32 * h + 16 * r + l0);
            hm[i] = load8_a2(bp + 16 * r + l0);
            a01[i] = load8_a2(bp + 96);   // scale words aux0, aux1
            a2d[i] = load8_a2(bp + 104);  // aux2, then d in the low half of .y
        }
        float xv[B][4][8];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const float *xp = X + (size_t)j * ldx + b * 256 + h * 128 + 16 * r + l0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float4 a = load_f4(xp + 32 * k), c = load_f4(xp + 32 * k + 4);
                xv[j][k][0] = a.x; xv[j][k][1] = a.y; xv[j][k][2] = a.z; xv[j][k][3] = a.w;
                xv[j][k][4] = c.x; xv[j][k][5] = c.y; xv[j][k][6] = c.z; xv[j][k][7] = c.w;
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            const float d = half_bits_to_float(a2d[i].y);
            // the scale words of this half (dequantizeQ3K's utmp[2h], utmp[2h+1], :969-985)
            const uint32_t aux2 = a2d[i].x;
            const uint32_t ua = ((a01[i].x >> (4 * h)) & 0x0f0f0f0fu) | (((aux2 >> (4 * h)) & 0x03030303u) << 4);
            const uint32_t ub = ((a01[i].y >> (4 * h)) & 0x0f0f0f0fu) | (((aux2 >> (4 * h + 2)) & 0x03030303u) << 4);
            float dsc[4];
            uint32_t u[4][2];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int s6 = (int)byte_of(k < 2 ? ua : ub, 2 * (k & 1) + r) - 32;
                dsc[k] = d * (float)s6;
                const int hb = 4 * h + k;
                // 3-bit q with bit 2 flipped: as a signed 3-bit field it is q - 4
                u[k][0] = (((q[i].x >> (2 * k)) & 0x03030303u) | (((hm[i].x >> hb) & 0x01010101u) << 2)) ^ 0x04040404u;
                u[k][1] = (((q[i].y >> (2 * k)) & 0x03030303u) | (((hm[i].y >> hb) & 0x01010101u) << 2)) ^ 0x04040404u;
            }
#pragma unroll
            for (int j = 0; j < B; j++) {
                float a = acc[i][j];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float dot = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        dot = fmaf((float)sfield<3>(u[k][e >> 2], 8 * (e & 3)), xv[j][k][e], dot);
                    a = fmaf(dsc[k], dot, a);
                }
                acc[i][j] = a;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) {
            float s = wave_sum(acc[i][j]);
            if (lane == 0 && r0 + i < nrows) Y[(size_t)j * ldy + r0 + i] = s * ysc;
        }
}

// ---------------------------------------------------------------- Q8_0
// One lane per 34-byte block (32 weights); a wavefront step covers 64 blocks.
// The block start is 2-byte aligned: ten aligned dwords cover it.
template <int R, int B>
__device__ __forceinline__ void gemv_q8_0_body(int wg, const uint8_t *__restrict__ W, size_t pitch, int nb,
                                                 int nrows, const float *__restrict__ X, int ldx,
                                                 float *__restrict__ Y, int ldy, float ysc = 1.f) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = (wg * 4 + wave) * R;
    if (r0 >= nrows) return;

    float acc[R][B];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) acc[i][j] = 0.f;

    const uint8_t *rowp[R];
#pragma unroll
    for (int i = 0; i < R; i++) rowp[i] = W + (size_t)min(r0 + i, nrows - 1) * pitch;

    for (int b = lane; b < nb; b += 64) {
        uint32_t q[R][8];
        float dsc[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(rowp[i] + (size_t)b * 34);
            const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
            const uint32_t mis = (uint32_t)(a & 3u);  // 0 or 2
            uint32_t v[10];
            u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(w);
            u32x4a4 v1 = *reinterpret_cast<const u32x4a4 *>(w + 4);
            u32x2a4 v2 = *reinterpret_cast<const u32x2a4 *>(w + 8);
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
            v[8] = v2.x; v[9] = v2.y;
            dsc[i] = half_bits_to_float(mis ? (v[0] >> 16) : v[0]);
            // q bytes start at byte offset mis + 2 of the window
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t lo = mis ? v[k + 1] : v[k], hi = mis ? v[k + 2] : v[k + 1];
                q[i][k] = __builtin_amdgcn_alignbyte(hi, lo, mis ? 0u : 2u);
            }
        }
#pragma unroll
        for (int j = 0; j < B; j++) {
            const float *xp = X + (size_t)j * ldx + b * 32;
            float xv[32];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                float4 a = load_f4(xp + 4 * k);
                xv[4 * k] = a.x; xv[4 * k + 1] = a.y; xv[4 * k + 2] = a.z; xv[4 * k + 3] = a.w;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                float dot = 0.f;  // q as signed bytes (sign-extending byte selects of the convert)
#pragma unroll
                for (int k = 0; k < 32; k++) dot = fmaf((float)sfield<8>(q[i][k >> 2], 8 * (k & 3)), xv[k], dot);
                acc[i][j] = fmaf(dsc[i], dot, acc[i][j]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < B; j++) {
            float s = wave_sum(acc[i][j]);
            if (lane == 0 && r0 + i < nrows) Y[(size_t)j * ldy + r0 + i] = s * ysc;
        }
}


template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q4k(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q4k_body<R, B>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}
template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q5k(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q4k_body<R, B, true>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}
template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q2k(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q2k_body<R, B>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}
template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q3k(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q3k_body<R, B>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}
template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q6k(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q6k_body<R, B>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}
template <int R, int B>
__global__ __launch_bounds__(256) void gemv_q8_0(const uint8_t *__restrict__ W, size_t pitch, int nb, int nrows,
                                                 const float *__restrict__ X, int ldx, float *__restrict__ Y, int ldy) {
    gemv_q8_0_body<R, B>(blockIdx.x, W, pitch, nb, nrows, X, ldx, Y, ldy);
}

// Several independent B = 1 GEMVs of any of the three formats in one launch:
// workgroups [wg_begin[p], wg_begin[p+1]) belong to problem p.  One launch
// instead of n removes the per-launch ramp and drain that dominate small
// matrices (a Llama-3-8B k projection streams 2.4 MB, ~0.4 us at HBM speed).
//
// NORM: every problem's x is w_n * h * scale with h = x + res (the first
// problem's x) and scale = 1 / sqrt(mean(h^2) + eps) (rmsNorm,
// LlamaTransformerHandler.java:818-826).  Each workgroup forms w_n * h for all
// columns in LDS and sums h^2 in the same pass; the bodies read x from there and
// multiply their sums by the scale, so the norm costs one pass over three
// vectors instead of a launch.  Workgroup 0 stores h to x_out.
// MASK: the formats compiled in (1 Q4_K, 2 Q5_K, 4 Q6_K, 8 Q8_0, 16 Q2_K, 32 Q3_K):
// the kernel's registers are the most any compiled-in body needs, so a group of
// one or two formats does not pay for the others.
template <bool NORM, int MASK>
__global__ __launch_bounds__(256) void gemv_group(GroupArgs g) {
    const int bid = blockIdx.x;
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroup; i++)
        if (i < g.n && bid >= g.p[i].wg_begin) p = i;
    const GroupProblem &q = g.p[p];
    const int wg = bid - q.wg_begin;
    const int nb = q.type == 8 ? q.cols / 32 : q.cols / 256;
    const float *X = q.x;
    float ysc = 1.f;
    if constexpr (NORM) {
        extern __shared__ __align__(16) float xs[];
        __shared__ float part[4];
        const int cols = q.cols;
        float4 hv[kNormGroupMaxCols / 1024], wv[kNormGroupMaxCols / 1024];
        // every load first (addresses clamped in range), then the arithmetic
#pragma unroll
        for (int k = 0; k < kNormGroupMaxCols / 1024; k++) {
            const int c = min((int)threadIdx.x * 4 + 1024 * k, cols - 4);
            const float4 a = load_f4(X + c), r = load_f4(g.res + c);
            hv[k] = make_float4(a.x + r.x, a.y + r.y, a.z + r.z, a.w + r.w);
            wv[k] = load_f4(g.norm_w + c);
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < kNormGroupMaxCols / 1024; k++) {
            const int c = (int)threadIdx.x * 4 + 1024 * k;
            if (c < cols) {
                const float4 h = hv[k], w = wv[k];
                if (bid == 0 && g.x_out) *reinterpret_cast<float4 *>(g.x_out + c) = h;
                *reinterpret_cast<float4 *>(xs + c) = make_float4(w.x * h.x, w.y * h.y, w.z * h.z, w.w * h.w);
                ss += (h.x * h.x + h.y * h.y) + (h.z * h.z + h.w * h.w);
            }
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
        __syncthreads();
        const float tot = (part[0] + part[1]) + (part[2] + part[3]);
        ysc = 1.f / (float)sqrt((double)(tot / (float)cols + g.eps));
        X = xs;
    }
    if (q.rows_per_wave == 2) {
        switch (q.type) {
        case 12: if constexpr ((MASK & 1) != 0) gemv_q4k_body<2, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 13: if constexpr ((MASK & 2) != 0) gemv_q4k_body<2, 1, true>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 14: if constexpr ((MASK & 4) != 0) gemv_q6k_body<2, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 10: if constexpr ((MASK & 16) != 0) gemv_q2k_body<2, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 11: if constexpr ((MASK & 32) != 0) gemv_q3k_body<2, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        default: if constexpr ((MASK & 8) != 0) gemv_q8_0_body<2, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        }
    } else {
        switch (q.type) {
        case 12: if constexpr ((MASK & 1) != 0) gemv_q4k_body<1, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 13: if constexpr ((MASK & 2) != 0) gemv_q4k_body<1, 1, true>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 14: if constexpr ((MASK & 4) != 0) gemv_q6k_body<1, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 10: if constexpr ((MASK & 16) != 0) gemv_q2k_body<1, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        case 11: if constexpr ((MASK & 32) != 0) gemv_q3k_body<1, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        default: if constexpr ((MASK & 8) != 0) gemv_q8_0_body<1, 1>(wg, q.w, q.pitch, nb, q.nrows, X, q.cols, q.y, q.nrows, ysc); break;
        }
    }
}

static int format_bit(int type) {
    switch (type) {
    case 12: return 1;
    case 13: return 2;
    case 14: return 4;
    case 8: return 8;
    case 10: return 16;
    default: return 32;
    }
}
// the formats of the group picked from a few compiled combinations (a Q4_K_M
// layer's [q, k, v] is Q4_K + Q6_K); anything else takes the kernel with all six
template <bool NORM>
static void launch_group_mask(const GroupArgs &g, int total, size_t lds, hipStream_t s) {
    int mask = 0;
    for (int i = 0; i < g.n; i++) mask |= format_bit(g.p[i].type);
    switch (mask) {
    case 1: gemv_group<NORM, 1><<<total, 256, lds, s>>>(g); break;
    case 4: gemv_group<NORM, 4><<<total, 256, lds, s>>>(g); break;
    case 5: gemv_group<NORM, 5><<<total, 256, lds, s>>>(g); break;
    case 8: gemv_group<NORM, 8><<<total, 256, lds, s>>>(g); break;
    default: gemv_group<NORM, 63><<<total, 256, lds, s>>>(g); break;
    }
}

hipError_t launch_gemv_group(GroupArgs g, hipStream_t s) {
    int total = 0;
    for (int i = 0; i < g.n; i++) {
        GroupProblem &q = g.p[i];
        if (q.type != 12 && q.type != 13 && q.type != 14 && q.type != 8 && q.type != 10 && q.type != 11)
            return hipErrorInvalidValue;
        q.rows_per_wave = q.nrows >= 2048 ? 2 : 1;
        q.wg_begin = total;
        total += (q.nrows + 4 * q.rows_per_wave - 1) / (4 * q.rows_per_wave);
    }
    if (total == 0) return hipSuccess;
    if (g.norm_w) {
        // one input for all problems, its columns a multiple of 4 and within the LDS image
        for (int i = 0; i < g.n; i++)
            if (g.p[i].x != g.p[0].x || g.p[i].cols != g.p[0].cols) return hipErrorNotSupported;
        const int cols = g.p[0].cols;
        if (!g.res || cols % 4 || cols > kNormGroupMaxCols) return hipErrorNotSupported;
        launch_group_mask<true>(g, total, (size_t)cols * sizeof(float), s);
    } else {
        launch_group_mask<false>(g, total, 0, s);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- F32
// One wavefront per row; lanes stride along the row.
template <int B>
__global__ __launch_bounds__(256) void gemv_f32(const float *__restrict__ W, size_t ld, int cols, int nrows,
                                                const float *__restrict__ X, int ldx, float *__restrict__ Y,
                                                int ldy) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + wave;
    if (r >= nrows) return;
    const float *wr = W + (size_t)r * ld;
    float acc[B];
#pragma unroll
    for (int j = 0; j < B; j++) acc[j] = 0.f;
    for (int c = lane; c < cols; c += 64) {
        const float w = __builtin_nontemporal_load(wr + c);
#pragma unroll
        for (int j = 0; j < B; j++) acc[j] = fmaf(w, X[(size_t)j * ldx + c], acc[j]);
    }
#pragma unroll
    for (int j = 0; j < B; j++) {
        float s = wave_sum(acc[j]);
        if (lane == 0) Y[(size_t)j * ldy + r] = s;
    }
}

// ---------------------------------------------------------------- launchers

template <int R, int B>
static hipError_t launch_q(int type, const uint8_t *W, size_t pitch, int nb, int nrows, const float *X, int ldx,
                           float *Y, int ldy, hipStream_t s) {
    const int rows_per_wg = 4 * R;
    dim3 grid((nrows + rows_per_wg - 1) / rows_per_wg), block(256);
    switch (type) {
    case 12: gemv_q4k<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    case 13: gemv_q5k<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    case 14: gemv_q6k<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    case 8: gemv_q8_0<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    case 10: gemv_q2k<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    case 11: gemv_q3k<R, B><<<grid, block, 0, s>>>(W, pitch, nb, nrows, X, ldx, Y, ldy); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int B>
static hipError_t launch_b(const GemvArgs &a, hipStream_t s) {
    const uint8_t *W = a.w + (size_t)a.row_start * a.pitch;
    const int nrows = a.row_end - a.row_start;
    if (a.type == 0) {
        dim3 grid((nrows + 3) / 4), block(256);
        gemv_f32<B><<<grid, block, 0, s>>>(reinterpret_cast<const float *>(W), a.pitch / 4, a.cols, nrows, a.x,
                                          a.ldx, a.y, a.ldy);
        return hipGetLastError();
    }
    const int nb = a.type == 8 ? a.cols / 32 : a.cols / 256;
    // Two rows per wavefront share x; one row when that leaves too few waves.
    if (B <= 2 && nrows >= 2048)
        return launch_q<2, B>(a.type, W, a.pitch, nb, nrows, a.x, a.ldx, a.y, a.ldy, s);
    return launch_q<1, B>(a.type, W, a.pitch, nb, nrows, a.x, a.ldx, a.y, a.ldy, s);
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s) {
    switch (a.batch) {
    case 1: return launch_b<1>(a, s);
    case 2: return launch_b<2>(a, s);
    case 4: return launch_b<4>(a, s);
    case 8: return launch_b<8>(a, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace jh
