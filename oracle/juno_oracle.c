/*
 * juno_oracle.c -- CPU restatement of Juno's Java quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libjunohip.so, never part of the
 * product path.  Built with -O2 -ffp-contract=off and without fast-math so
 * that every fp32 operation is one IEEE-rounded Java operation.
 *
 * Reference files (under /root/reference/node/src/main/java/cab/ml/juno/node/):
 *   LlamaTransformerHandler.java  dequantizers 873-1135, matVec dispatch 1200-1254,
 *                                 matVecQ4Kraw 1428-1468, q4kScaleRaw/q4kMinRaw 1471-1482,
 *                                 matVecQ8_0raw 1486-1508, readLE16 1511-1513,
 *                                 matVecQ5Kraw 1526-1578, matVecQ6Kraw 1587-1638,
 *                                 matVecF32raw 1258-1280
 *   GgufReader.java               rawByteCount 347-360, f16ToF32 1248-1271
 *   LoraMerge.java                quantizeQ8_0 265-277, quantizeQ4_K 311-366,
 *                                 quantizeQ5_K 376-430, quantizeQ6_K 437-469,
 *                                 f32ToF16 589-605, clamp 607-609
 *
 * Pinning (what checks each function): see the header of tests/test_oracle.py.
 */
#include "juno_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---------------------------------------------------------------------------
 * Scalar helpers
 * ------------------------------------------------------------------------- */

/* GgufReader.f16ToF32 (GgufReader.java:1248-1271): exact half -> single,
 * subnormals normalised, inf/NaN keep the payload shifted by 13. */
float or_f16_to_f32(uint16_t h) {
    uint32_t s = (h >> 15) & 1u;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = s << 31;
        } else {
            int exp = -14;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                exp--;
            }
            m &= 0x3FFu;
            f = (s << 31) | ((uint32_t)(exp + 127) << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = (s << 31) | 0x7F800000u | (m << 13);
    } else {
        f = (s << 31) | ((e - 15 + 127) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

/* Bit pattern of or_f16_to_f32 (a float return through a Python float would
 * quieten signalling NaNs). */
uint32_t or_f16_to_f32_bits(uint16_t h) {
    float f = or_f16_to_f32(h);
    uint32_t b;
    memcpy(&b, &f, 4);
    return b;
}

/* LoraMerge.f32ToF16 (LoraMerge.java:589-605), quirks kept: NaN maps to inf,
 * the subnormal branch rounds after a truncating shift. */
uint16_t or_f32_to_f16(float value) {
    int32_t bits;
    memcpy(&bits, &value, 4);
    int32_t sign = (int32_t)(((uint32_t)bits >> 31) & 1u);
    int32_t exp = (int32_t)(((uint32_t)bits >> 23) & 0xFFu) - 127 + 15;
    int32_t mant = bits & 0x7FFFFF;
    if (exp <= 0) {
        if (exp < -10) return (uint16_t)(sign << 15);
        mant = (mant | 0x800000) >> (1 - exp);
        mant = (mant + 0x0FFF + ((mant >> 13) & 1)) >> 13;
        return (uint16_t)((sign << 15) | mant);
    }
    if (exp >= 31) return (uint16_t)((sign << 15) | 0x7C00);
    int32_t round = mant & 0x1FFF;
    mant >>= 13;
    if (round > 0x1000 || (round == 0x1000 && (mant & 1) == 1)) {
        mant++;
        if (mant == 0x400) {
            mant = 0;
            exp++;
        }
    }
    if (exp >= 31) return (uint16_t)((sign << 15) | 0x7C00);
    return (uint16_t)((sign << 15) | (exp << 10) | mant);
}

/* java.lang.Math.round(float): the closest int, ties toward +inf, i.e.
 * floor(a + 0.5) in exact arithmetic; NaN -> 0; saturating like (int) casts.
 * (float)a + 0.5 is exact in double for every float with |a| < 2^52. */
int32_t or_java_round(float a) {
    if (a != a) return 0;
    double r = floor((double)a + 0.5);
    if (r >= 2147483647.0) return INT32_MAX;
    if (r <= -2147483648.0) return INT32_MIN;
    return (int32_t)r;
}

static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { /* LoraMerge.java:607 */
    return v < lo ? lo : (v > hi ? hi : v);
}

/* GgufReader.rawByteCount (GgufReader.java:347-360), the types of this path. */
int64_t or_raw_byte_count(int type, int64_t nelems) {
    switch (type) {
    case OR_TYPE_F32: return nelems * 4;
    case OR_TYPE_Q8_0: return (nelems / 32) * 34;
    case OR_TYPE_Q2_K: return (nelems / 256) * 84;
    case OR_TYPE_Q3_K: return (nelems / 256) * 110;
    case OR_TYPE_Q4_K: return (nelems / 256) * 144;
    case OR_TYPE_Q5_K: return (nelems / 256) * 176;
    case OR_TYPE_Q6_K: return (nelems / 256) * 210;
    default: return -1;
    }
}

static inline uint16_t le16(const uint8_t *p) { /* readLE16 (LlamaTransformerHandler.java:1511-1513) */
    return (uint16_t)(p[0] | (p[1] << 8));
}

/* q4kScaleRaw / q4kMinRaw (LlamaTransformerHandler.java:1471-1482);
 * twins getScale4K / getMin4K (GgufReader.java:708-721). */
int or_q4k_scale(const uint8_t *sc, int j) {
    if (j < 4) return sc[j] & 0x3F;
    return ((sc[j + 4] & 0x0F) | ((sc[j - 4] & 0xC0) >> 2)) & 0x3F;
}

int or_q4k_min(const uint8_t *sc, int j) {
    if (j < 4) return sc[j + 4] & 0x3F;
    return ((sc[j + 4] >> 4) | ((sc[j] & 0xC0) >> 2)) & 0x3F;
}

static int block_geometry(int type, int *qk, int *bytes) {
    switch (type) {
    case OR_TYPE_F32: *qk = 1; *bytes = 4; return 0;
    case OR_TYPE_Q8_0: *qk = 32; *bytes = 34; return 0;
    case OR_TYPE_Q2_K: *qk = 256; *bytes = 84; return 0;
    case OR_TYPE_Q3_K: *qk = 256; *bytes = 110; return 0;
    case OR_TYPE_Q4_K: *qk = 256; *bytes = 144; return 0;
    case OR_TYPE_Q5_K: *qk = 256; *bytes = 176; return 0;
    case OR_TYPE_Q6_K: *qk = 256; *bytes = 210; return 0;
    default: return -1;
    }
}

/* ---------------------------------------------------------------------------
 * Dequantizers: one block -> 256 (or 32) fp32 values.
 * ------------------------------------------------------------------------- */

/* dequantizeQ8_0 (LlamaTransformerHandler.java:895-913): out = scale * q. */
static void deq_q8_0(const uint8_t *bo, float *out) {
    float scale = or_f16_to_f32(le16(bo));
    for (int i = 0; i < 32; i++) out[i] = scale * (float)(int8_t)bo[2 + i];
}

/* dequantizeQ4K (LlamaTransformerHandler.java:1017-1050):
 * out = (d*sc)*q - dmin*m, two separately rounded operations. */
static void deq_q4_k(const uint8_t *bo, float *out) {
    const uint8_t *sc = bo + 4, *qs = bo + 16;
    float d = or_f16_to_f32(le16(bo));
    float dmin = or_f16_to_f32(le16(bo + 2));
    int qi = 0;
    for (int g = 0; g < 256; g += 64) {
        int s0 = g / 32, s1 = s0 + 1;
        float scale0 = d * (float)or_q4k_scale(sc, s0);
        float min0 = dmin * (float)or_q4k_min(sc, s0);
        float scale1 = d * (float)or_q4k_scale(sc, s1);
        float min1 = dmin * (float)or_q4k_min(sc, s1);
        for (int i = 0; i < 32; i++) out[g + i] = scale0 * (float)(qs[qi + i] & 0x0F) - min0;
        for (int i = 0; i < 32; i++) out[g + 32 + i] = scale1 * (float)((qs[qi + i] >> 4) & 0x0F) - min1;
        qi += 32;
    }
}

/* dequantizeQ5K (LlamaTransformerHandler.java:1052-1093). */
static void deq_q5_k(const uint8_t *bo, float *out) {
    const uint8_t *sc = bo + 4, *qh = bo + 16, *qs = bo + 48;
    float d = or_f16_to_f32(le16(bo));
    float dmin = or_f16_to_f32(le16(bo + 2));
    int qi = 0;
    for (int g = 0; g < 4; g++) {
        int s0 = g * 2, s1 = s0 + 1;
        float scale0 = d * (float)or_q4k_scale(sc, s0);
        float min0 = dmin * (float)or_q4k_min(sc, s0);
        float scale1 = d * (float)or_q4k_scale(sc, s1);
        float min1 = dmin * (float)or_q4k_min(sc, s1);
        for (int l = 0; l < 32; l++) {
            int lo = qs[qi + l] & 0x0F, hi = (qh[l] >> s0) & 1;
            out[g * 64 + l] = scale0 * (float)(lo | (hi << 4)) - min0;
        }
        for (int l = 0; l < 32; l++) {
            int lo = (qs[qi + l] >> 4) & 0x0F, hi = (qh[l] >> s1) & 1;
            out[g * 64 + 32 + l] = scale1 * (float)(lo | (hi << 4)) - min1;
        }
        qi += 32;
    }
}

/* dequantizeQ6K (LlamaTransformerHandler.java:1095-1135): out = (d*sc) * q. */
static void deq_q6_k(const uint8_t *bo, float *out) {
    float d = or_f16_to_f32(le16(bo + 208));
    for (int half = 0; half < 2; half++) {
        const uint8_t *ql = bo + half * 64, *qh = bo + 128 + half * 32;
        const int8_t *sc = (const int8_t *)(bo + 192 + half * 8);
        float *o = out + half * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int qlL = ql[l], qlL2 = ql[l + 32], qhL = qh[l];
            int q1 = ((qlL & 0x0F) | (((qhL >> 0) & 3) << 4)) - 32;
            int q2 = ((qlL2 & 0x0F) | (((qhL >> 2) & 3) << 4)) - 32;
            int q3 = ((qlL >> 4) | (((qhL >> 4) & 3) << 4)) - 32;
            int q4 = ((qlL2 >> 4) | (((qhL >> 6) & 3) << 4)) - 32;
            float d1 = d * (float)sc[is], d2 = d * (float)sc[is + 2];
            float d3 = d * (float)sc[is + 4], d4 = d * (float)sc[is + 6];
            o[l] = d1 * (float)q1;
            o[l + 32] = d2 * (float)q2;
            o[l + 64] = d3 * (float)q3;
            o[l + 96] = d4 * (float)q4;
        }
    }
}

/* dequantizeQ2K (LlamaTransformerHandler.java:915-952): [scales 16][qs 64][d][dmin];
 * per half of 128, element l + 16k (k = 0..7) uses scale byte 8*half + k (low
 * nibble scale, high nibble min) and the 2 bits at shift 2*(k/2) of
 * qs[32*half + l + 16*(k&1)]: out = (d*sc)*q - dmin*m. */
static void deq_q2_k(const uint8_t *bo, float *out) {
    float d = or_f16_to_f32(le16(bo + 80)), dmin = or_f16_to_f32(le16(bo + 82));
    for (int half = 0; half < 2; half++) {
        const uint8_t *sh = bo + half * 8, *qh = bo + 16 + half * 32;
        float *o = out + half * 128;
        for (int l = 0; l < 16; l++) {
            int q0 = qh[l], q1 = qh[l + 16];
            for (int k = 0; k < 8; k++) {
                int q = ((k & 1) ? q1 : q0) >> (2 * (k / 2)) & 3;
                o[l + 16 * k] = d * (float)(sh[k] & 0x0F) * (float)q - dmin * (float)(sh[k] >> 4);
            }
        }
    }
}

/* The 16 signed 6-bit scales of a Q3_K block (biased by 32), unpacked from 12
 * bytes as dequantizeQ3K does (LlamaTransformerHandler.java:969-985). */
void or_q3k_scales(const uint8_t *sc12, int sc[16]) {
    uint32_t aux0 = sc12[0] | (sc12[1] << 8) | (sc12[2] << 16) | ((uint32_t)sc12[3] << 24);
    uint32_t aux1 = sc12[4] | (sc12[5] << 8) | (sc12[6] << 16) | ((uint32_t)sc12[7] << 24);
    uint32_t aux2 = sc12[8] | (sc12[9] << 8) | (sc12[10] << 16) | ((uint32_t)sc12[11] << 24);
    uint32_t utmp[4] = {(aux0 & 0x0f0f0f0fu) | ((aux2 & 0x03030303u) << 4),
                        (aux1 & 0x0f0f0f0fu) | (((aux2 >> 2) & 0x03030303u) << 4),
                        ((aux0 >> 4) & 0x0f0f0f0fu) | (((aux2 >> 4) & 0x03030303u) << 4),
                        ((aux1 >> 4) & 0x0f0f0f0fu) | (((aux2 >> 6) & 0x03030303u) << 4)};
    for (int k = 0; k < 4; k++)
        for (int j = 0; j < 4; j++) sc[4 * k + j] = (int)((utmp[k] >> (8 * j)) & 0xFF) - 32;
}

/* dequantizeQ3K (LlamaTransformerHandler.java:954-1015): [hmask 32][qs 64][scales 12][d];
 * group is = 2j + r of half h (16 elements l) takes the 2 bits at shift 2j of
 * qs[32h + 16r + l] and bit (4h + j) of hmask[16r + l] as q = (low2 | hi<<2) - 4;
 * out = (d*sc[is]) * q (exact). */
static void deq_q3_k(const uint8_t *bo, float *out) {
    const uint8_t *hm = bo, *qs = bo + 32;
    float d = or_f16_to_f32(le16(bo + 108));
    int sc[16];
    or_q3k_scales(bo + 96, sc);
    int is = 0, m = 1, oi = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t *qh = qs + half * 32;
        for (int j = 0, shift = 0; j < 4; j++, shift += 2, m <<= 1)
            for (int r = 0; r < 2; r++) {
                float dl = d * (float)sc[is++];
                for (int l = 0; l < 16; l++) {
                    int low2 = (qh[16 * r + l] >> shift) & 3, hi = (hm[16 * r + l] & m) ? 4 : 0;
                    out[oi++] = dl * (float)((low2 | hi) - 4);
                }
            }
    }
}

static void deq_f32(const uint8_t *bo, float *out) { memcpy(out, bo, 4); } /* dequantizeF32 :887-893 */

typedef void (*deq_fn)(const uint8_t *, float *);

static deq_fn deq_for(int type) {
    switch (type) {
    case OR_TYPE_F32: return deq_f32;
    case OR_TYPE_Q8_0: return deq_q8_0;
    case OR_TYPE_Q2_K: return deq_q2_k;
    case OR_TYPE_Q3_K: return deq_q3_k;
    case OR_TYPE_Q4_K: return deq_q4_k;
    case OR_TYPE_Q5_K: return deq_q5_k;
    case OR_TYPE_Q6_K: return deq_q6_k;
    default: return NULL;
    }
}

/* dequantize switch (LlamaTransformerHandler.java:873-885). */
int or_dequantize(int type, const uint8_t *raw, int rows, int cols, float *out) {
    int qk, bb;
    deq_fn fn = deq_for(type);
    if (!fn || block_geometry(type, &qk, &bb) || rows < 0 || cols <= 0 || cols % qk) return -1;
    size_t nb = (size_t)cols / qk;
    for (size_t r = 0; r < (size_t)rows; r++)
        for (size_t b = 0; b < nb; b++)
            fn(raw + (r * nb + b) * bb, out + r * (size_t)cols + b * qk);
    return 0;
}

/* ---------------------------------------------------------------------------
 * Per-row dot products, Java summation order.
 * ------------------------------------------------------------------------- */

/* matVecF32raw (LlamaTransformerHandler.java:1258-1280): acc += w * x. */
static float row_f32(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    for (int c = 0; c < cols; c++) {
        float w;
        memcpy(&w, row + 4 * (size_t)c, 4);
        acc += w * x[c];
    }
    return acc;
}

/* matVecQ8_0raw (LlamaTransformerHandler.java:1486-1508): acc += (scale*q)*x. */
static float row_q8_0(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 32;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 34;
        float scale = or_f16_to_f32(le16(bo));
        const float *xb = x + b * 32;
        for (int i = 0; i < 32; i++) acc += scale * (float)(int8_t)bo[2 + i] * xb[i];
    }
    return acc;
}

/* matVecQ4Kraw (LlamaTransformerHandler.java:1428-1468):
 * acc += ((scale*q) - min) * x, low nibbles then high nibbles per group. */
static float row_q4_k(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 256;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 144;
        const uint8_t *sc = bo + 4, *qs = bo + 16;
        float d = or_f16_to_f32(le16(bo));
        float dmin = or_f16_to_f32(le16(bo + 2));
        const float *xb = x + b * 256;
        int qi = 0;
        for (int g = 0; g < 256; g += 64) {
            int s0 = g / 32, s1 = s0 + 1;
            float scale0 = d * (float)or_q4k_scale(sc, s0);
            float min0 = dmin * (float)or_q4k_min(sc, s0);
            float scale1 = d * (float)or_q4k_scale(sc, s1);
            float min1 = dmin * (float)or_q4k_min(sc, s1);
            for (int i = 0; i < 32; i++)
                acc += (scale0 * (float)(qs[qi + i] & 0x0F) - min0) * xb[g + i];
            for (int i = 0; i < 32; i++)
                acc += (scale1 * (float)((qs[qi + i] >> 4) & 0x0F) - min1) * xb[g + 32 + i];
            qi += 32;
        }
    }
    return acc;
}

/* matVecQ5Kraw (LlamaTransformerHandler.java:1526-1578). */
static float row_q5_k(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 256;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 176;
        const uint8_t *sc = bo + 4, *qh = bo + 16, *qs = bo + 48;
        float d = or_f16_to_f32(le16(bo));
        float dmin = or_f16_to_f32(le16(bo + 2));
        const float *xb = x + b * 256;
        int qi = 0;
        for (int g = 0; g < 4; g++) {
            int s0 = g * 2, s1 = s0 + 1;
            float scale0 = d * (float)or_q4k_scale(sc, s0);
            float min0 = dmin * (float)or_q4k_min(sc, s0);
            float scale1 = d * (float)or_q4k_scale(sc, s1);
            float min1 = dmin * (float)or_q4k_min(sc, s1);
            for (int l = 0; l < 32; l++) {
                int lo = qs[qi + l] & 0x0F, hi = (qh[l] >> s0) & 1;
                acc += (scale0 * (float)(lo | (hi << 4)) - min0) * xb[g * 64 + l];
            }
            for (int l = 0; l < 32; l++) {
                int lo = (qs[qi + l] >> 4) & 0x0F, hi = (qh[l] >> s1) & 1;
                acc += (scale1 * (float)(lo | (hi << 4)) - min1) * xb[g * 64 + 32 + l];
            }
            qi += 32;
        }
    }
    return acc;
}

/* matVecQ6Kraw (LlamaTransformerHandler.java:1587-1638): for each l the four
 * terms l, l+32, l+64, l+96 are accumulated in that order as (dN*qN)*x. */
static float row_q6_k(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 256;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 210;
        float d = or_f16_to_f32(le16(bo + 208));
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = bo + half * 64, *qh = bo + 128 + half * 32;
            const int8_t *sc = (const int8_t *)(bo + 192 + half * 8);
            const float *xo = x + b * 256 + half * 128;
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int qlL = ql[l], qlL2 = ql[l + 32], qhL = qh[l];
                int q1 = ((qlL & 0x0F) | (((qhL >> 0) & 3) << 4)) - 32;
                int q2 = ((qlL2 & 0x0F) | (((qhL >> 2) & 3) << 4)) - 32;
                int q3 = ((qlL >> 4) | (((qhL >> 4) & 3) << 4)) - 32;
                int q4 = ((qlL2 >> 4) | (((qhL >> 6) & 3) << 4)) - 32;
                float d1 = d * (float)sc[is], d2 = d * (float)sc[is + 2];
                float d3 = d * (float)sc[is + 4], d4 = d * (float)sc[is + 6];
                acc += d1 * (float)q1 * xo[l];
                acc += d2 * (float)q2 * xo[l + 32];
                acc += d3 * (float)q3 * xo[l + 64];
                acc += d4 * (float)q4 * xo[l + 96];
            }
        }
    }
    return acc;
}

/* matVecQ2Kraw (LlamaTransformerHandler.java:1303-1346): per half and l, the
 * eight terms l + 16k (k = 0..7) in that order, each ((d*sc)*q - dmin*m) * x. */
static float row_q2_k(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 256;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 84;
        float d = or_f16_to_f32(le16(bo + 80)), dmin = or_f16_to_f32(le16(bo + 82));
        for (int half = 0; half < 2; half++) {
            const uint8_t *sh = bo + half * 8, *qh = bo + 16 + half * 32;
            const float *xo = x + b * 256 + half * 128;
            for (int l = 0; l < 16; l++) {
                int q0 = qh[l], q1 = qh[l + 16];
                for (int k = 0; k < 8; k++) {
                    int q = ((k & 1) ? q1 : q0) >> (2 * (k / 2)) & 3;
                    acc += (d * (float)(sh[k] & 0x0F) * (float)q - dmin * (float)(sh[k] >> 4)) * xo[l + 16 * k];
                }
            }
        }
    }
    return acc;
}

/* matVecQ3Kraw (LlamaTransformerHandler.java:1358-1425): elements in order,
 * acc += ((d*sc)*q) * x. */
static float row_q3_k(const uint8_t *row, const float *x, int cols) {
    float acc = 0.0f;
    int nb = cols / 256;
    for (int b = 0; b < nb; b++) {
        const uint8_t *bo = row + (size_t)b * 110;
        const uint8_t *hm = bo, *qs = bo + 32;
        float d = or_f16_to_f32(le16(bo + 108));
        int sc[16];
        or_q3k_scales(bo + 96, sc);
        const float *xb = x + b * 256;
        int is = 0, m = 1, xi = 0;
        for (int half = 0; half < 2; half++) {
            const uint8_t *qh = qs + half * 32;
            for (int j = 0, shift = 0; j < 4; j++, shift += 2, m <<= 1)
                for (int r = 0; r < 2; r++) {
                    float dl = d * (float)sc[is++];
                    for (int l = 0; l < 16; l++) {
                        int low2 = (qh[16 * r + l] >> shift) & 3, hi = (hm[16 * r + l] & m) ? 4 : 0;
                        acc += dl * (float)((low2 | hi) - 4) * xb[xi++];
                    }
                }
        }
    }
    return acc;
}

typedef float (*row_fn)(const uint8_t *, const float *, int);

static row_fn row_for(int type) {
    switch (type) {
    case OR_TYPE_F32: return row_f32;
    case OR_TYPE_Q8_0: return row_q8_0;
    case OR_TYPE_Q2_K: return row_q2_k;
    case OR_TYPE_Q3_K: return row_q3_k;
    case OR_TYPE_Q4_K: return row_q4_k;
    case OR_TYPE_Q5_K: return row_q5_k;
    case OR_TYPE_Q6_K: return row_q6_k;
    default: return NULL;
    }
}

typedef struct {
    row_fn fn;
    const uint8_t *raw;
    const float *x;
    float *y;
    size_t pitch;
    int cols, row_start, nrows;
    int next; /* shared work counter (row chunks handed out dynamically) */
    pthread_mutex_t mu;
} mv_job;

enum { MV_CHUNK = 16 };

static void *mv_worker(void *arg) {
    mv_job *j = (mv_job *)arg;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        int r0 = j->next;
        j->next += MV_CHUNK;
        pthread_mutex_unlock(&j->mu);
        if (r0 >= j->nrows) break;
        int r1 = r0 + MV_CHUNK < j->nrows ? r0 + MV_CHUNK : j->nrows;
        for (int r = r0; r < r1; r++)
            j->y[r] = j->fn(j->raw + (size_t)(j->row_start + r) * j->pitch, j->x, j->cols);
    }
    return NULL;
}

/* matVec(QuantizedTensor, x, rowStart, rowEnd, cols) dispatch
 * (LlamaTransformerHandler.java:1200-1254).  Rows are independent and each row
 * is summed sequentially, so the thread split never changes a result; this
 * mirrors IntStream.range(0, rows).parallel() on the common pool. */
int or_matvec(int type, const uint8_t *raw, const float *x, int row_start, int row_end,
              int cols, float *y, int nthreads) {
    int qk, bb;
    row_fn fn = row_for(type);
    if (!fn || block_geometry(type, &qk, &bb) || cols <= 0 || cols % qk || row_start < 0 ||
        row_end < row_start)
        return -1;
    mv_job j;
    j.fn = fn;
    j.raw = raw;
    j.x = x;
    j.y = y;
    j.pitch = (size_t)(cols / qk) * bb;
    j.cols = cols;
    j.row_start = row_start;
    j.nrows = row_end - row_start;
    j.next = 0;
    pthread_mutex_init(&j.mu, NULL);
    if (nthreads <= 0) nthreads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    int started = 0;
    for (int t = 1; t < nthreads; t++)
        if (pthread_create(&th[started], NULL, mv_worker, &j) == 0) started++;
    mv_worker(&j);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&j.mu);
    return 0;
}

/* ---------------------------------------------------------------------------
 * Quantizers (LoraMerge.requantize, LoraMerge.java:226-241).
 * ------------------------------------------------------------------------- */

static inline void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

/* quantizeQ8_0 (LoraMerge.java:265-277). */
static void quant_q8_0(const float *v, uint8_t *o) {
    float absMax = 0.0f;
    for (int i = 0; i < 32; i++) absMax = fmaxf(absMax, fabsf(v[i]));
    float d = absMax / 127.0f;
    float invD = d > 0.0f ? 1.0f / d : 0.0f;
    put16(o, or_f32_to_f16(d));
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)clampi(or_java_round(v[i] * invD), -127, 127);
}

/* Shared by quantizeQ4_K (LoraMerge.java:311-366) and quantizeQ5_K (:376-430):
 * per sub-block min/range, d = maxRange/(63*qmax), dmin = maxAbsMin/63, 6-bit
 * ls/lm, and the 12-byte scale pack. */
static void kquant_scales(const float *v, float qmax_times_63, float *d_out, float *dmin_out,
                          int ls[8], int lm[8], uint8_t sc[12]) {
    float mins[8], ranges[8];
    for (int s = 0; s < 8; s++) {
        float mn = 3.40282347e+38f, mx = -3.40282347e+38f;
        for (int i = 0; i < 32; i++) {
            float e = v[s * 32 + i];
            if (e < mn) mn = e;
            if (e > mx) mx = e;
        }
        if (mn > mx) {
            mn = 0.0f;
            mx = 0.0f;
        }
        mins[s] = mn;
        ranges[s] = mx - mn;
    }
    float maxRange = 0.0f, maxAbsMin = 0.0f;
    for (int s = 0; s < 8; s++) {
        if (ranges[s] > maxRange) maxRange = ranges[s];
        float am = -mins[s];
        if (am > maxAbsMin) maxAbsMin = am;
    }
    float d = maxRange > 0.0f ? maxRange / qmax_times_63 : 0.0f;
    float dmin = maxAbsMin > 0.0f ? maxAbsMin / 63.0f : 0.0f;
    for (int s = 0; s < 8; s++) {
        ls[s] = maxRange > 0.0f ? clampi(or_java_round(ranges[s] * 63.0f / maxRange), 0, 63) : 0;
        lm[s] = maxAbsMin > 0.0f ? clampi(or_java_round(-mins[s] * 63.0f / maxAbsMin), 0, 63) : 0;
    }
    for (int j = 0; j < 4; j++) {
        sc[j] = (uint8_t)((ls[j] & 0x3F) | ((ls[j + 4] & 0x30) << 2));
        sc[j + 4] = (uint8_t)((lm[j] & 0x3F) | ((lm[j + 4] & 0x30) << 2));
        sc[j + 8] = (uint8_t)((ls[j + 4] & 0x0F) | ((lm[j + 4] & 0x0F) << 4));
    }
    *d_out = d;
    *dmin_out = dmin;
}

/* quantizeQ4_K (LoraMerge.java:311-366).  The nibbles are computed with the
 * fp32 d/dmin (not their fp16 roundings), as the reference does. */
static void quant_q4_k(const float *v, uint8_t *o) {
    int ls[8], lm[8];
    float d, dmin;
    kquant_scales(v, 945.0f, &d, &dmin, ls, lm, o + 4);
    put16(o, or_f32_to_f16(d));
    put16(o + 2, or_f32_to_f16(dmin));
    uint8_t *qs = o + 16;
    for (int g = 0; g < 4; g++) {
        int s0 = g * 2, s1 = s0 + 1;
        float sc0 = d * (float)ls[s0], mn0 = dmin * (float)lm[s0];
        float sc1 = d * (float)ls[s1], mn1 = dmin * (float)lm[s1];
        for (int i = 0; i < 32; i++) {
            int q0 = sc0 > 0.0f ? clampi(or_java_round((v[s0 * 32 + i] + mn0) / sc0), 0, 15) : 0;
            int q1 = sc1 > 0.0f ? clampi(or_java_round((v[s1 * 32 + i] + mn1) / sc1), 0, 15) : 0;
            qs[g * 32 + i] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

/* quantizeQ5_K (LoraMerge.java:376-430). */
static void quant_q5_k(const float *v, uint8_t *o) {
    int ls[8], lm[8];
    float d, dmin;
    kquant_scales(v, 1953.0f, &d, &dmin, ls, lm, o + 4);
    put16(o, or_f32_to_f16(d));
    put16(o + 2, or_f32_to_f16(dmin));
    uint8_t *qh = o + 16, *qs = o + 48;
    memset(qh, 0, 32);
    for (int g = 0; g < 4; g++) {
        int s0 = g * 2, s1 = s0 + 1;
        float sc0 = d * (float)ls[s0], mn0 = dmin * (float)lm[s0];
        float sc1 = d * (float)ls[s1], mn1 = dmin * (float)lm[s1];
        for (int l = 0; l < 32; l++) {
            int q0 = sc0 > 0.0f ? clampi(or_java_round((v[s0 * 32 + l] + mn0) / sc0), 0, 31) : 0;
            int q1 = sc1 > 0.0f ? clampi(or_java_round((v[s1 * 32 + l] + mn1) / sc1), 0, 31) : 0;
            qs[g * 32 + l] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
            qh[l] |= (uint8_t)(((q0 >> 4) & 1) << s0);
            qh[l] |= (uint8_t)(((q1 >> 4) & 1) << s1);
        }
    }
}

/* quantizeQ6_K (LoraMerge.java:437-469). */
static void quant_q6_k(const float *v, uint8_t *o) {
    float subMax[16];
    for (int s = 0; s < 16; s++) {
        float m = 0.0f;
        for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[s * 16 + i]));
        subMax[s] = m;
    }
    float globalMax = 0.0f;
    for (int s = 0; s < 16; s++)
        if (subMax[s] > globalMax) globalMax = subMax[s];
    float d = globalMax > 0.0f ? globalMax / 4064.0f : 0.0f;
    float invD = d > 0.0f ? 1.0f / d : 0.0f;
    int8_t sc[16];
    for (int s = 0; s < 16; s++)
        sc[s] = (int8_t)(d > 0.0f ? clampi(or_java_round(subMax[s] * invD / 32.0f), -127, 127) : 0);
    uint8_t ql[128], qh[64];
    memset(ql, 0, sizeof ql);
    memset(qh, 0, sizeof qh);
    for (int p = 0; p < 256; p++) {
        int half = p / 128, lp = p % 128, quad = lp / 32, l = lp % 32;
        int sub = half * 8 + (l / 16) + quad * 2;
        float eff = d * (float)sc[sub];
        int q6 = eff != 0.0f ? clampi(or_java_round(v[p] / eff), -32, 31) : 0;
        int u = q6 + 32;
        int qlIdx = half * 64 + l + ((quad % 2 == 1) ? 32 : 0);
        if (quad < 2) ql[qlIdx] = (uint8_t)((ql[qlIdx] & 0xF0) | (u & 0x0F));
        else ql[qlIdx] = (uint8_t)((ql[qlIdx] & 0x0F) | ((u & 0x0F) << 4));
        int shift = quad * 2;
        int qi = half * 32 + l;
        qh[qi] = (uint8_t)((qh[qi] & ~(0x3 << shift)) | (((u >> 4) & 0x3) << shift));
    }
    memcpy(o, ql, 128);
    memcpy(o + 128, qh, 64);
    memcpy(o + 192, sc, 16);
    put16(o + 208, or_f32_to_f16(d));
}

int or_quantize(int type, const float *data, int64_t n, uint8_t *out) {
    int qk, bb;
    if (block_geometry(type, &qk, &bb) || n < 0 || n % qk) return -1;
    void (*fn)(const float *, uint8_t *) = NULL;
    switch (type) {
    case OR_TYPE_F32: memcpy(out, data, (size_t)n * 4); return 0;
    case OR_TYPE_Q8_0: fn = quant_q8_0; break;
    case OR_TYPE_Q4_K: fn = quant_q4_k; break;
    case OR_TYPE_Q5_K: fn = quant_q5_k; break;
    case OR_TYPE_Q6_K: fn = quant_q6_k; break;
    default: return -1;
    }
    for (int64_t b = 0; b < n / qk; b++) fn(data + b * qk, out + b * bb);
    return 0;
}
