// jh_device.hpp -- device helpers shared by the gfx950 kernels of libjunohip.
//
// Block formats (GGUF, little-endian; the layouts LlamaTransformerHandler.java
// reads at 1017-1050 / 1095-1135 / 895-913):
//   Q4_K  144 B / 256 w : [d f16][dmin f16][scales 12][qs 128]
//   Q6_K  210 B / 256 w : [ql 128][qh 64][scales 16 x int8][d f16]
//   Q8_0   34 B /  32 w : [d f16][q 32 x int8]
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jh {

constexpr int kWave = 64;

typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    // v_cvt_f32_f16 is exact for every half, subnormals included (fp16
    // denormals are on by default on gfx9), like GgufReader.f16ToF32.
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    return (float)v;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xFFu; }

// 16-byte streaming load of weight bytes that are read exactly once.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_stream16(const uint8_t *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float4 load_f4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

// silu(g) * u with silu's exp in double, cast to float (LlamaTransformerHandler.java:1733-1735, 796-797)
__device__ __forceinline__ float silu_times(float g, float u) { return g / (1.f + (float)exp(-(double)g)) * u; }

// Sum over the 64 lanes of a wavefront with DPP row operations, then the four
// 16-lane row totals with readlane.  Every lane returns the full sum.
__device__ __forceinline__ float wave_sum(float v) {
    int x = __builtin_bit_cast(int, v);
    // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror:4, row_ror:8
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true));
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true));
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, true));
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true));
    x = __builtin_bit_cast(int, v);
    float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 0));
    float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 16));
    float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 32));
    float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(x, 48));
    return (r0 + r1) + (r2 + r3);
}

// Q4_K 6-bit scale / min of sub-block j from the 12 scale bytes held in three
// little-endian words (q4kScaleRaw / q4kMinRaw, LlamaTransformerHandler.java:1471-1482).
__device__ __forceinline__ uint32_t sc_byte(uint32_t s0, uint32_t s1, uint32_t s2, int k) {
    uint32_t w = k < 4 ? s0 : (k < 8 ? s1 : s2);
    return byte_of(w, k & 3);
}

__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &ls,
                                              int &lm) {
    if (j < 4) {
        ls = sc_byte(s0, s1, s2, j) & 63;
        lm = sc_byte(s0, s1, s2, j + 4) & 63;
    } else {
        uint32_t hi = sc_byte(s0, s1, s2, j + 4);
        ls = (int)((hi & 0x0F) | ((sc_byte(s0, s1, s2, j - 4) & 0xC0) >> 2));
        lm = (int)((hi >> 4) | ((sc_byte(s0, s1, s2, j) & 0xC0) >> 2));
    }
}

// 8 bytes starting at a 2-byte-aligned address (Q6_K / Q8_0 fields): three
// dword loads from the enclosing aligned window and a byte funnel shift.
__device__ __forceinline__ uint2 load8_a2(const uint8_t *p) {
    uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
    uint32_t sh = (uint32_t)(a & 3u);
    uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

}  // namespace jh
