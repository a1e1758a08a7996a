// jh_quant.hip -- dequantization (bit-exact) and quantization kernels.
//
// Dequantization restates LlamaTransformerHandler.dequantize
// (LlamaTransformerHandler.java:873-1135), unit by unit (jh_dequant.hpp).
//
// Quantization restates LoraMerge.requantize (LoraMerge.java:226-469) so that
// benchmark and test inputs are the reference quantizer's bytes, produced on
// the device.  One thread per block: the reference is sequential per block and
// its rounding (Math.round, fp32 divisions) is reproduced exactly.
#include "jh_dequant.hpp"
#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {

// ---------------------------------------------------------------- dequant

template <int T> __device__ __forceinline__ void dequant_unit(const uint8_t *W, int64_t t, float *out) {
    deq_unit<T>(W, t, [out](int64_t i, float v) { out[i] = v; });
}

template <int T> __global__ void dequant_k(const uint8_t *__restrict__ W, int64_t units, float *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < units) dequant_unit<T>(W, t, out);
}

// Embedding lookup (getInitialActivation, LlamaTransformerHandler.java:651-660):
// for output row y = blockIdx.y, row clamp(d_tokens[y], 0, rows - 1) of the
// packed matrix, dequantized into out[y].  Tokens are read on the device so
// that a captured step can be replayed.
template <int T>
__global__ void dequant_row_k(const uint8_t *__restrict__ W, const int *__restrict__ d_tokens, int rows, size_t pitch,
                              int64_t units, int64_t row_elems, float *__restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= units) return;
    const int tok = min(max(d_tokens[blockIdx.y], 0), rows - 1);
    dequant_unit<T>(W + (size_t)tok * pitch, t, out + (int64_t)blockIdx.y * row_elems);
}

int64_t dequant_units(int type, int64_t n) {
    switch (type) {
    case 12:
    case 13:
    case 8: return n / 32;
    case 14:
    case 10:
    case 11: return n / 16;
    case 0: return n;
    default: return -1;
    }
}

hipError_t launch_dequant(int type, const uint8_t *w, int rows, int cols, float *out, hipStream_t s) {
    const int64_t units = dequant_units(type, (int64_t)rows * cols);
    if (units < 0) return hipErrorInvalidValue;
    if (units == 0) return hipSuccess;
    dim3 block(256), grid((unsigned)((units + 255) / 256));
    switch (type) {
    case 12: dequant_k<12><<<grid, block, 0, s>>>(w, units, out); break;
    case 13: dequant_k<13><<<grid, block, 0, s>>>(w, units, out); break;
    case 14: dequant_k<14><<<grid, block, 0, s>>>(w, units, out); break;
    case 8: dequant_k<8><<<grid, block, 0, s>>>(w, units, out); break;
    case 10: dequant_k<10><<<grid, block, 0, s>>>(w, units, out); break;
    case 11: dequant_k<11><<<grid, block, 0, s>>>(w, units, out); break;
    case 0: dequant_k<0><<<grid, block, 0, s>>>(w, units, out); break;
    }
    return hipGetLastError();
}

hipError_t launch_dequant_row(int type, const uint8_t *w, int rows, int cols, size_t pitch, const int *d_tokens,
                              int n_out, float *out, hipStream_t s) {
    const int64_t units = dequant_units(type, cols);
    if (units < 0 || rows <= 0 || n_out < 1 || n_out > 65535) return hipErrorInvalidValue;
    dim3 block(64), grid((unsigned)((units + 63) / 64), (unsigned)n_out);
    switch (type) {
    case 12: dequant_row_k<12><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 13: dequant_row_k<13><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 14: dequant_row_k<14><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 8: dequant_row_k<8><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 10: dequant_row_k<10><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 11: dequant_row_k<11><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    case 0: dequant_row_k<0><<<grid, block, 0, s>>>(w, d_tokens, rows, pitch, units, cols, out); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- quantize

// java.lang.Math.round(float): floor(a + 0.5) exactly (a + 0.5 is exact in
// double), NaN -> 0, saturating.
__device__ __forceinline__ int java_round(float a) {
    if (a != a) return 0;
    const double r = floor(__dadd_rn((double)a, 0.5));
    if (r >= 2147483647.0) return 2147483647;
    if (r <= -2147483648.0) return (int)0x80000000u;
    return (int)r;
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// LoraMerge.f32ToF16 (LoraMerge.java:589-605): round-to-nearest-even on the
// normal range; NaN becomes infinity; the subnormal branch rounds after a
// truncating shift.  Reproduced as-is so the stored d / dmin bytes match.
__device__ uint32_t f32_to_f16_ref(float value) {
    const int32_t bits = __builtin_bit_cast(int32_t, value);
    const int32_t sign = (int32_t)(((uint32_t)bits >> 31) & 1u);
    int32_t exp = (int32_t)(((uint32_t)bits >> 23) & 0xFFu) - 112;
    int32_t mant = bits & 0x7FFFFF;
    if (exp <= 0) {
        if (exp < -10) return (uint32_t)(sign << 15);
        mant = (mant | 0x800000) >> (1 - exp);
        mant = (mant + 0x0FFF + ((mant >> 13) & 1)) >> 13;
        return (uint32_t)((sign << 15) | mant);
    }
    if (exp >= 31) return (uint32_t)((sign << 15) | 0x7C00);
    const int32_t low = mant & 0x1FFF;
    mant >>= 13;
    if (low > 0x1000 || (low == 0x1000 && (mant & 1))) {
        mant++;
        if (mant == 0x400) {
            mant = 0;
            exp++;
        }
    }
    if (exp >= 31) return (uint32_t)((sign << 15) | 0x7C00);
    return (uint32_t)((sign << 15) | (exp << 10) | mant);
}

__device__ __forceinline__ void put16(uint8_t *p, uint32_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

// quantizeQ8_0 (LoraMerge.java:265-277)
__global__ void quant_q8_0(const float *__restrict__ src, int64_t nblk, uint8_t *__restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk) return;
    const float *v = src + t * 32;
    uint8_t *o = dst + t * 34;
    float absMax = 0.f;
    for (int i = 0; i < 32; i++) absMax = fmaxf(absMax, fabsf(v[i]));
    const float d = __fdiv_rn(absMax, 127.f);
    const float invD = d > 0.f ? __fdiv_rn(1.f, d) : 0.f;
    put16(o, f32_to_f16_ref(d));
    for (int i = 0; i < 32; i++) o[2 + i] = (uint8_t)(int8_t)clampi(java_round(__fmul_rn(v[i], invD)), -127, 127);
}

// quantizeQ4_K (LoraMerge.java:311-366) and quantizeQ5_K (:376-430): the same
// scale / min search with q in [0, 15] (d = maxRange / 945) or [0, 31]
// (d = maxRange / 1953, 5th bits in qh); the quants use the fp32 d / dmin.
template <bool Q5>
__global__ void quant_kq(const float *__restrict__ src, int64_t nblk, uint8_t *__restrict__ dst) {
    constexpr int kBytes = Q5 ? 176 : 144, kQs = Q5 ? 48 : 16, kQmax = Q5 ? 31 : 15;
    constexpr float kRange = Q5 ? 1953.f : 945.f;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk) return;
    const float *v = src + t * 256;
    uint8_t *o = dst + t * kBytes;
    float mins[8], ranges[8];
    for (int s = 0; s < 8; s++) {
        float mn = 3.40282347e+38f, mx = -3.40282347e+38f;
        for (int i = 0; i < 32; i++) {
            const float e = v[s * 32 + i];
            if (e < mn) mn = e;
            if (e > mx) mx = e;
        }
        if (mn > mx) {
            mn = 0.f;
            mx = 0.f;
        }
        mins[s] = mn;
        ranges[s] = __fsub_rn(mx, mn);
    }
    float maxRange = 0.f, maxAbsMin = 0.f;
    for (int s = 0; s < 8; s++) {
        if (ranges[s] > maxRange) maxRange = ranges[s];
        const float am = -mins[s];
        if (am > maxAbsMin) maxAbsMin = am;
    }
    const float d = maxRange > 0.f ? __fdiv_rn(maxRange, kRange) : 0.f;
    const float dmin = maxAbsMin > 0.f ? __fdiv_rn(maxAbsMin, 63.f) : 0.f;
    int ls[8], lm[8];
    for (int s = 0; s < 8; s++) {
        ls[s] = maxRange > 0.f ? clampi(java_round(__fdiv_rn(__fmul_rn(ranges[s], 63.f), maxRange)), 0, 63) : 0;
        lm[s] = maxAbsMin > 0.f ? clampi(java_round(__fdiv_rn(__fmul_rn(-mins[s], 63.f), maxAbsMin)), 0, 63) : 0;
    }
    put16(o, f32_to_f16_ref(d));
    put16(o + 2, f32_to_f16_ref(dmin));
    for (int j = 0; j < 4; j++) {
        o[4 + j] = (uint8_t)((ls[j] & 0x3F) | ((ls[j + 4] & 0x30) << 2));
        o[8 + j] = (uint8_t)((lm[j] & 0x3F) | ((lm[j + 4] & 0x30) << 2));
        o[12 + j] = (uint8_t)((ls[j + 4] & 0x0F) | ((lm[j + 4] & 0x0F) << 4));
    }
    uint32_t qh[8] = {};  // 32 bytes of 5th bits, built in registers
    for (int g = 0; g < 4; g++) {
        const int s0 = 2 * g, s1 = s0 + 1;
        const float sc0 = __fmul_rn(d, (float)ls[s0]), mn0 = __fmul_rn(dmin, (float)lm[s0]);
        const float sc1 = __fmul_rn(d, (float)ls[s1]), mn1 = __fmul_rn(dmin, (float)lm[s1]);
        for (int i = 0; i < 32; i++) {
            const int q0 = sc0 > 0.f ? clampi(java_round(__fdiv_rn(__fadd_rn(v[s0 * 32 + i], mn0), sc0)), 0, kQmax) : 0;
            const int q1 = sc1 > 0.f ? clampi(java_round(__fdiv_rn(__fadd_rn(v[s1 * 32 + i], mn1), sc1)), 0, kQmax) : 0;
            o[kQs + g * 32 + i] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
            if (Q5)
                qh[i >> 2] |= (uint32_t)((((q0 >> 4) & 1) << s0) | (((q1 >> 4) & 1) << s1)) << (8 * (i & 3));
        }
    }
    if (Q5)
        for (int i = 0; i < 32; i++) o[16 + i] = (uint8_t)(qh[i >> 2] >> (8 * (i & 3)));
}

// quantizeQ6_K (LoraMerge.java:437-469)
__global__ void quant_q6k(const float *__restrict__ src, int64_t nblk, uint8_t *__restrict__ dst) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nblk) return;
    const float *v = src + t * 256;
    uint8_t *o = dst + t * 210;
    float subMax[16];
    float globalMax = 0.f;
    for (int s = 0; s < 16; s++) {
        float m = 0.f;
        for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[s * 16 + i]));
        subMax[s] = m;
        if (m > globalMax) globalMax = m;
    }
    const float d = globalMax > 0.f ? __fdiv_rn(globalMax, 4064.f) : 0.f;
    const float invD = d > 0.f ? __fdiv_rn(1.f, d) : 0.f;
    int sc[16];
    for (int s = 0; s < 16; s++) {
        sc[s] = d > 0.f ? clampi(java_round(__fdiv_rn(__fmul_rn(subMax[s], invD), 32.f)), -127, 127) : 0;
        o[192 + s] = (uint8_t)(int8_t)sc[s];
    }
    // Each ql / qh byte is assembled from the elements it encodes; the result
    // equals the reference's read-modify-write loop over elements p.
    auto u_of = [&](int p) {
        const int half = p >> 7, lp = p & 127, quad = lp >> 5, l = lp & 31;
        const int sub = half * 8 + (l >> 4) + quad * 2;
        const float eff = __fmul_rn(d, (float)sc[sub]);
        const int q6 = eff != 0.f ? clampi(java_round(__fdiv_rn(v[p], eff)), -32, 31) : 0;
        return q6 + 32;
    };
    for (int idx = 0; idx < 128; idx++) {
        const int half = idx >> 6, odd = (idx >> 5) & 1, l = idx & 31;
        const int lo = u_of(half * 128 + odd * 32 + l), hi = u_of(half * 128 + (odd + 2) * 32 + l);
        o[idx] = (uint8_t)((lo & 0x0F) | ((hi & 0x0F) << 4));
    }
    for (int idx = 0; idx < 64; idx++) {
        const int half = idx >> 5, l = idx & 31;
        uint32_t b = 0;
        for (int quad = 0; quad < 4; quad++) b |= (uint32_t)((u_of(half * 128 + quad * 32 + l) >> 4) & 3) << (2 * quad);
        o[128 + idx] = (uint8_t)b;
    }
    put16(o + 208, f32_to_f16_ref(d));
}

hipError_t launch_quantize(int type, const float *src, int64_t n, uint8_t *dst, hipStream_t s) {
    int64_t nblk;
    switch (type) {
    case 8: nblk = n / 32; break;
    case 12:
    case 13:
    case 14: nblk = n / 256; break;
    case 0: return hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice, s);
    default: return hipErrorInvalidValue;
    }
    if (nblk == 0) return hipSuccess;
    dim3 block(128), grid((unsigned)((nblk + 127) / 128));
    switch (type) {
    case 8: quant_q8_0<<<grid, block, 0, s>>>(src, nblk, dst); break;
    case 12: quant_kq<false><<<grid, block, 0, s>>>(src, nblk, dst); break;
    case 13: quant_kq<true><<<grid, block, 0, s>>>(src, nblk, dst); break;
    case 14: quant_q6k<<<grid, block, 0, s>>>(src, nblk, dst); break;
    }
    return hipGetLastError();
}

}  // namespace jh
