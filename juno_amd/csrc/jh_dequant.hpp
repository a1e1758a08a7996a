// jh_dequant.hpp -- the exact dequantization of one unit of a packed image,
// shared by the dequant kernels (jh_quant.hip) and the staged GEMV's residual
// correction (jh_gemv_staged.hip).
//
// These restate LlamaTransformerHandler.dequantize
// (LlamaTransformerHandler.java:873-1135).  Every product there is exact in
// fp32 (an 11-bit fp16 significand times a 6- or 8-bit scale times a 4-, 6- or
// 8-bit quant), so only the Q4_K "- min" rounds; the explicit _rn intrinsics
// keep each step a separately rounded IEEE operation anyway.
#pragma once

#include "jh_device.hpp"

namespace jh {

// The element loop of a unit: unrolled (the dequant kernels), or kept a loop
// (U = false: register-lean, for code that shares a kernel with a hot path).
template <bool U, typename F>
__device__ __forceinline__ void for_n(int n, F f) {
    if constexpr (U) {
#pragma unroll
        for (int i = 0; i < n; i++) f(i);
    } else {
#pragma nounroll
        for (int i = 0; i < n; i++) f(i);
    }
}

// Each deq_* function expands one unit (a 32- or 16-element sub-block, a Q8_0
// block or one F32 element) t of the packed image W, handing each element to
// put(index, value) with its index in the image's element order.
template <bool U, typename P>
__device__ __forceinline__ void deq_q4k(const uint8_t *__restrict__ W, int64_t t, P put) {
    const int64_t blk = t >> 3;
    const int j = (int)(t & 7), g = j >> 1;
    const uint8_t *bp = W + blk * 144;
    const float d = half_bits_to_float(bp[0] | (bp[1] << 8));
    const float dmin = half_bits_to_float(bp[2] | (bp[3] << 8));
    const uint32_t s0 = bp[4] | (bp[5] << 8) | (bp[6] << 16) | ((uint32_t)bp[7] << 24);
    const uint32_t s1 = bp[8] | (bp[9] << 8) | (bp[10] << 16) | ((uint32_t)bp[11] << 24);
    const uint32_t s2 = bp[12] | (bp[13] << 8) | (bp[14] << 16) | ((uint32_t)bp[15] << 24);
    int ls, lm;
    q4k_scale_min(s0, s1, s2, j, ls, lm);
    const float scale = __fmul_rn(d, (float)ls), mn = __fmul_rn(dmin, (float)lm);
    const uint8_t *qs = bp + 16 + g * 32;
    const int shift = (j & 1) * 4;
    for_n<U>(32, [&](int i) { put(t * 32 + i, __fsub_rn(__fmul_rn(scale, (float)((qs[i] >> shift) & 0x0F)), mn)); });
}

// dequantizeQ5K (LlamaTransformerHandler.java:1052-1093): the Q4_K layout plus a
// 5th bit per element in qh (bit j of qh[l] for sub-block j).
template <bool U, typename P>
__device__ __forceinline__ void deq_q5k(const uint8_t *__restrict__ W, int64_t t, P put) {
    const int64_t blk = t >> 3;
    const int j = (int)(t & 7), g = j >> 1;
    const uint8_t *bp = W + blk * 176;
    const float d = half_bits_to_float(bp[0] | (bp[1] << 8));
    const float dmin = half_bits_to_float(bp[2] | (bp[3] << 8));
    const uint32_t s0 = bp[4] | (bp[5] << 8) | (bp[6] << 16) | ((uint32_t)bp[7] << 24);
    const uint32_t s1 = bp[8] | (bp[9] << 8) | (bp[10] << 16) | ((uint32_t)bp[11] << 24);
    const uint32_t s2 = bp[12] | (bp[13] << 8) | (bp[14] << 16) | ((uint32_t)bp[15] << 24);
    int ls, lm;
    q4k_scale_min(s0, s1, s2, j, ls, lm);
    const float scale = __fmul_rn(d, (float)ls), mn = __fmul_rn(dmin, (float)lm);
    const uint8_t *qh = bp + 16, *qs = bp + 48 + g * 32;
    const int shift = (j & 1) * 4;
    for_n<U>(32, [&](int i) {
        const int q = ((qs[i] >> shift) & 0x0F) | (((qh[i] >> j) & 1) << 4);
        put(t * 32 + i, __fsub_rn(__fmul_rn(scale, (float)q), mn));
    });
}

template <bool U, typename P>
__device__ __forceinline__ void deq_q6k(const uint8_t *__restrict__ W, int64_t t, P put) {
    const int64_t blk = t >> 4;
    const int s = (int)(t & 15), half = s >> 3, k = (s & 7) >> 1, is = s & 1;
    const uint8_t *bp = W + blk * 210;
    const float d = half_bits_to_float(bp[208] | (bp[209] << 8));
    const float dk = __fmul_rn(d, (float)(int8_t)bp[192 + half * 8 + is + 2 * k]);
    const uint8_t *ql = bp + half * 64 + ((k & 1) ? 32 : 0);
    const uint8_t *qh = bp + 128 + half * 32;
    const int nsh = (k >> 1) * 4, hsh = 2 * k;
    const int64_t o = blk * 256 + half * 128 + k * 32 + is * 16;
    for_n<U>(16, [&](int i) {
        const int l = is * 16 + i;
        const int q = (((ql[l] >> nsh) & 0x0F) | (((qh[l] >> hsh) & 3) << 4)) - 32;
        put(o + i, __fmul_rn(dk, (float)q));
    });
}

template <bool U, typename P>
__device__ __forceinline__ void deq_q8_0(const uint8_t *__restrict__ W, int64_t t, P put) {
    const uint8_t *bp = W + t * 34;
    const float d = half_bits_to_float(bp[0] | (bp[1] << 8));
    for_n<U>(32, [&](int i) { put(t * 32 + i, __fmul_rn(d, (float)(int8_t)bp[2 + i])); });
}

// dequantizeQ2K (LlamaTransformerHandler.java:915-952): unit t = 16 elements
// of block t/16, half h = (t/8)&1, group k = t&7: elements h*128 + 16k + l take
// the 2 bits at shift 2(k/2) of qs[32h + 16(k&1) + l] and scale byte sc[8h + k];
// w = (d*(sc&15))*q - dmin*(sc>>4).
template <bool U, typename P>
__device__ __forceinline__ void deq_q2k(const uint8_t *__restrict__ W, int64_t t, P put) {
    const int64_t blk = t >> 4;
    const int h = (int)(t >> 3) & 1, k = (int)t & 7;
    const uint8_t *bp = W + blk * 84;
    const float d = half_bits_to_float(bp[80] | (bp[81] << 8)), dmin = half_bits_to_float(bp[82] | (bp[83] << 8));
    const int sc = bp[8 * h + k];
    const float dl = __fmul_rn(d, (float)(sc & 15)), ml = __fmul_rn(dmin, (float)(sc >> 4));
    const uint8_t *qs = bp + 16 + 32 * h + 16 * (k & 1);
    const int shift = 2 * (k >> 1);
    const int64_t o = blk * 256 + h * 128 + 16 * k;
    for_n<U>(16, [&](int l) { put(o + l, __fsub_rn(__fmul_rn(dl, (float)((qs[l] >> shift) & 3)), ml)); });
}

// dequantizeQ3K (LlamaTransformerHandler.java:954-1015): unit t = 16 elements
// of block t/16, group is = t&15 = 8h + 2j + r: elements h*128 + 32j + 16r + l
// take the 2 bits at shift 2j of qs[32h + 16r + l] and bit 4h + j of
// hmask[16r + l]; w = (d*sc[is]) * ((low2 | hi<<2) - 4), exact.
template <bool U, typename P>
__device__ __forceinline__ void deq_q3k(const uint8_t *__restrict__ W, int64_t t, P put) {
    const int64_t blk = t >> 4;
    const int is = (int)t & 15, h = is >> 3, j = (is >> 1) & 3, r = is & 1;
    const uint8_t *bp = W + blk * 110;
    const float d = half_bits_to_float(bp[108] | (bp[109] << 8));
    // scale is: 4 low bits from byte is&7 (high nibble for is >= 8), 2 high bits
    // from byte 8 + (is&3) at bit 2*(is/4) (the utmp words of :969-985)
    const int lo4 = (bp[96 + (is & 7)] >> (is >= 8 ? 4 : 0)) & 15;
    const int hi2 = (bp[104 + (is & 3)] >> (2 * (is >> 2))) & 3;
    const float dl = __fmul_rn(d, (float)((lo4 | (hi2 << 4)) - 32));
    const uint8_t *qs = bp + 32 + 32 * h + 16 * r, *hm = bp + 16 * r;
    const int m = 1 << (4 * h + j);
    const int64_t o = blk * 256 + h * 128 + 32 * j + 16 * r;
    for_n<U>(16, [&](int l) {
        const int q = (((qs[l] >> (2 * j)) & 3) | ((hm[l] & m) ? 4 : 0)) - 4;
        put(o + l, __fmul_rn(dl, (float)q));
    });
}

template <bool U, typename P>
__device__ __forceinline__ void deq_f32(const uint8_t *__restrict__ W, int64_t t, P put) {
    put(t, reinterpret_cast<const float *>(W)[t]);
}

template <int T, bool U = true, typename P> __device__ __forceinline__ void deq_unit(const uint8_t *W, int64_t t, P put) {
    if constexpr (T == 12) deq_q4k<U>(W, t, put);
    else if constexpr (T == 13) deq_q5k<U>(W, t, put);
    else if constexpr (T == 14) deq_q6k<U>(W, t, put);
    else if constexpr (T == 8) deq_q8_0<U>(W, t, put);
    else if constexpr (T == 10) deq_q2k<U>(W, t, put);
    else if constexpr (T == 11) deq_q3k<U>(W, t, put);
    else deq_f32<U>(W, t, put);
}

}  // namespace jh
