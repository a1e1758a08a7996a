// jh_gemv_staged.hip -- B = 1 fused dequant-GEMV for Q4_K, Q6_K and Q8_0 on gfx950.
//
// Design (measured on MI355X; each point removed a bottleneck of the simpler
// per-lane-block kernels in jh_gemv.hip):
//
//  * Coalesced weight stream.  A wavefront loads the bytes of its rows as one
//    contiguous span, 16 bytes per lane per instruction (1 KB per wave
//    instruction), and parks them in a wave-private LDS buffer.  Lanes then
//    read the block fields they need from LDS.  Letting each lane fetch its own
//    block fields straight from HBM touches ~4x more cache lines per
//    instruction and costs ~40% of the bandwidth.
//  * Software pipeline.  The next row group's loads are issued into registers
//    before the current group is computed from the wave's LDS buffer, so HBM
//    latency is hidden by the dequant math of the group in hand.
//  * Integer inner product.  x is converted once per workgroup into a 30-bit
//    integer per element (one power-of-two scale per quant sub-block) held as
//    four signed base-256 digits, and the weights' integer quants are
//    multiplied with v_dot4_i32_i8.  This needs ~1.4 VALU instructions per Q4_K weight
//    instead of ~2.8 for an fp32 convert+FMA path, which would otherwise bound
//    the kernel below the HBM roofline.  Block scales (d, dmin, 6-bit / int8
//    sub-scales) are fp32.
//  * Persistent workgroups.  x is converted once per workgroup and kept in
//    registers while the workgroup walks many row groups: with one column
//    tile the waves share one LDS image of all of x; with 2-4 column tiles
//    each lane converts just its own columns straight into registers (no
//    image, no barrier before the walk).
//  * Wide rows (more than 16 super-blocks, or 64 Q8_0 blocks) are split into
//    column tiles over 2 or 4 waves of a workgroup; the partial sums meet in LDS.
//
// Numerics: weights are used exactly; the only approximation beyond fp32
// summation order is rounding x * 2^s to an integer below 2^30 in magnitude,
// with one s per quant sub-block of x: exact for elements within 2^6 of the
// sub-block's maximum |x|, within 2^-18 of themselves down to 2^-12 of it,
// an absolute error of at most 2^-31 of that maximum below.  When that
// rounding is not small against a sub-block's other elements (one outlier
// setting the scale of many small elements), the launch takes an exact fp32
// path instead of the walk (staged_exact below).
#include "jh_dequant.hpp"
#include "jh_device.hpp"
#include "jh_kernels.hpp"

#include <stdlib.h>

namespace jh {
namespace {

// --------------------------------------------------------------------------- helpers

// Sum over the wavefront with DPP only; the total is valid in lane 63.
__device__ __forceinline__ float wave_sum_to63(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true));  // quad_perm 1,0,3,2
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true));  // quad_perm 2,3,0,1
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x124, 0xF, 0xF, true));  // row_ror:4
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true));  // row_ror:8
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false));  // row_bcast:15
    x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));  // row_bcast:31
    return v;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}


__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 4 bytes at a 2-byte-aligned LDS address given as (dword pointer, byte shift).
__device__ __forceinline__ uint32_t lds_word(const uint32_t *w, uint32_t sh, int k) {
    return __builtin_amdgcn_alignbyte(w[k + 1], w[k], sh);
}

// --------------------------------------------------------------------------- x preparation
//
// Every x element a lane needs becomes an integer xi = rint(x * 2^s) with one
// power-of-two scale 2^-s per scale group: the columns of one quant sub-block
// of the weight format (G = 32 for Q4_K / Q5_K sub-blocks and Q8_0 blocks, 16
// for Q6_K sub-blocks).  s puts the group's largest |x| in [2^29, 2^30).
// Scaling by a power of two is exact, and an element within 2^6 of the maximum
// is an integer after it (24 significant bits), so such elements are held
// exactly; an element down to 2^-12 of the maximum is rounded by at most
// 2^-18 of itself.  xi is held as four balanced base-256 digits
//   xi = sum_k d_k 256^(3-k),  d_k in [-128, 127],
// so that sum(q * x) = 2^-s * sum_k 256^(3-k) sum(q * d_k): four signed
// v_dot4_i32_i8 products per 4 quants with exact integer sums.  Every
// format's quants enter as signed bytes, so no bias term has to be removed
// afterwards (a fp32 cancellation when x has an outlier).  Elements below
// 2^-12 of their sub-block's maximum keep an absolute error of at most 2^-31
// of that maximum.
constexpr int kLimbs = 4;

// cols is a multiple of 32: a float4 is either wholly inside or wholly past
// the end.  The load is clamped in range; the caller zeroes the float4s that
// lie past the end (at use, so the load is not waited for here).
__device__ __forceinline__ float4 x_load4(const float *X, int cols, int c) {
    return *reinterpret_cast<const float4 *>(X + min(c, cols - 4));
}
__device__ __forceinline__ float4 x_mask4(float4 v, int cols, int c) {
    return c < cols ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}
__device__ __forceinline__ float amax4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}
// The shift s of a group with maximum |x| = mx (|x * 2^s| < 2^30), and its
// scale 2^-s (0 for an all-zero group, so that it contributes nothing).  s is
// at most 149, so that 2^-s is still an fp32 value (the smallest subnormal):
// an integer times it is then exact below 2^24 and rounded once above, and a
// group whose maximum is below 2^-119 keeps fewer than 30 bits, all of them
// above the fp32 products' own rounding (2^-150) there.
__device__ __forceinline__ int x_shift(float mx) {
    return mx > 0.f ? min(30 - __builtin_amdgcn_frexp_expf(mx), 149) : 0;
}
__device__ __forceinline__ float x_scale(float mx, int s) { return mx > 0.f ? ldexpf(1.f, -s) : 0.f; }

// The residual.  Rounding x * 2^s to an integer xi leaves r = x - 2^-s xi,
// |r| <= 2^-(s+1) <= 2^-30 max|x|, exactly representable (Sterbenz: xi 2^-s
// is within a factor 2 of x whenever xi != 0).  It matters only when one
// large element sets the scale of many much smaller ones: when the mean |x|
// of the group's other elements is below 2^-10 of its maximum (and not 0:
// a lone nonzero element is exact).  Otherwise each element's rounding error
// is at most 2^-19 of that mean.  A normal-range x never meets this (channels
// at 300x do not); x with a 1e4 outlier among 1e-2 elements does.  The test is
// a property of x alone, so every workgroup of a launch reaches the same
// answer.  When any group meets it, the launch computes sum deq(w) * x with
// the fp32 x itself instead (staged_exact): x is then used exactly, as the
// reference uses it.
// mx = max |x|, sa = sum |x| over the group.
template <int G>
__device__ __forceinline__ bool residual_matters(float mx, float sa) {
    const float rest = sa - mx;
    return rest > 0.f && rest * 1024.f < (float)(G - 1) * mx;
}
__device__ __forceinline__ float asum4(float4 v) { return (fabsf(v.x) + fabsf(v.y)) + (fabsf(v.z) + fabsf(v.w)); }

// The digit dwords of 4 consecutive x values: dword k holds digit k of value
// j in byte j (the bytes of xi + 0x80808080, each less 128).
struct Limbs {
    uint32_t b[kLimbs];  // b[0]: the top digit (256^3)
};
// The 4 x 4 byte transpose takes eight byte permutes (v_perm_b32: selector
// bytes 0..3 pick bytes of the second operand, 4..7 of the first).
__device__ __forceinline__ Limbs to_limbs(float4 v, int s) {
    const float e[4] = {v.x, v.y, v.z, v.w};
    uint32_t u[4];
#pragma unroll
    for (int j = 0; j < 4; j++) u[j] = (uint32_t)(int)rintf(ldexpf(e[j], s)) + 0x80808080u;  // |xi| < 2^30
    const uint32_t lo01 = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u);  // u0.b0 u1.b0 u0.b1 u1.b1
    const uint32_t hi01 = __builtin_amdgcn_perm(u[1], u[0], 0x07030602u);  // u0.b2 u1.b2 u0.b3 u1.b3
    const uint32_t lo23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(u[3], u[2], 0x07030602u);
    Limbs r;
    r.b[0] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u) ^ 0x80808080u;  // byte 3 of u0..u3
    r.b[1] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;  // byte 2
    r.b[2] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;  // byte 1
    r.b[3] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;  // byte 0
    return r;
}

// sum of v over the 4 lanes of a quad, in every lane of the quad
__device__ __forceinline__ float quad_sum(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true));  // quad_perm 1,0,3,2
    x = __builtin_bit_cast(int, v);
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true));  // 2,3,0,1
}
// max (MAX) or min of v over the 4 lanes of a quad (G = 16) or the 8 lanes 8k .. 8k+7 (G = 32)
template <int SEL, bool MAX>
__device__ __forceinline__ float dpp_red(float v) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), SEL, 0xF, 0xF, true));
    return MAX ? fmaxf(v, o) : fminf(v, o);
}
template <int G, bool MAX>
__device__ __forceinline__ float group_red(float v) {
    v = dpp_red<0xB1, MAX>(v);                  // quad_perm 1,0,3,2
    v = dpp_red<0x4E, MAX>(v);                  // quad_perm 2,3,0,1
    if (G == 32) v = dpp_red<0x141, MAX>(v);   // row_half_mirror
    return v;
}
// sum of v over the lanes of a group (as group_red)
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    if (G == 32)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    return v;
}

// Rows of one column tile (gw == 1) need all of x in every wave of the
// workgroup: there the waves convert x once, cooperatively, into an LDS image,
// and each lane loads its registers from it.  LDS image (cols_pad = 256 nblk):
//   digit k = 0..3: [cols_pad] bytes each
//   scale [cols_pad / 16] f32: the scale of the group of columns 16i .. 16i+15
//   xs16 [cols_pad / 16] f32: fp32 sums of 16 x (the Q4_K / Q5_K min terms)
// Columns >= cols read as 0.
struct XImage {
    int cols, nblk;
    uint8_t *base;
    __device__ uint32_t *limb(int k) const { return reinterpret_cast<uint32_t *>(base + 256 * k * nblk); }
    __device__ float *scale() const { return reinterpret_cast<float *>(base + 256 * kLimbs * nblk); }
    __device__ float *xs16() const { return scale() + 16 * nblk; }
    static __host__ __device__ size_t bytes(int nblk) { return (size_t)nblk * (256 * kLimbs + 64 + 64); }
};

// LDS of a staged workgroup: [image (shared x)][row-group buffers][ring
// partials][ring arrival / release counters]; then the claim counter and the
// per-wave residual flags.
constexpr int kRing = 4;  // cells per slot of the column-tile ring (a power of two)
// Bounded device-side waits that gave up (the ring's cell waits): counted
// here, read and cleared by sync_faults (jh_sync_faults).
__device__ unsigned int g_sync_faults;

// Timeline builds (-DJH_TIMELINE, juno_amd/timeline.py; never the shipped
// library): per wave of a shared-image walk (DYN, or column tiles), s_memrealtime
// (100 MHz) at entry, after the x prologue's barrier, once the first row group
// has landed, and at the end of the walk; slot = (workgroup * NW + wave) * 4,
// the last launch's values.
#ifdef JH_TIMELINE
constexpr int kTlWaves = 4096;
__device__ unsigned long long g_timeline[kTlWaves * 4];
#define JH_TL(k)                                                                                       \
    do {                                                                                               \
        if (SX && (threadIdx.x & 63) == 0 && (int)blockIdx.x * NW + wave < kTlWaves)                   \
            g_timeline[((int)blockIdx.x * NW + wave) * 4 + (k)] = __builtin_amdgcn_s_memrealtime();    \
    } while (0)
#else
#define JH_TL(k) do {} while (0)
#endif
__host__ __device__ constexpr size_t staged_front(bool sx, int nblk, int nw, int r, int ch) {
    return (sx ? ((XImage::bytes(nblk) + 15) & ~size_t(15)) : 0) + (size_t)nw * r * ch * 16 +
           (size_t)kRing * nw * r * 4 + 2 * kRing * nw * 4;
}

// Block b of 256 columns into the image, one wave: the lane holds columns
// 256 b + 4 lane .. +4.
// Returns whether the lane's group needs the exact path.
template <int G>
__device__ __forceinline__ bool x_quant_block(const XImage &im, int b, float4 v) {
    const int lane = threadIdx.x & 63;
    if (b * 256 + lane * 4 >= im.cols) v = make_float4(0.f, 0.f, 0.f, 0.f);
    const float mx = group_red<G, true>(amax4(v));
    const bool need = residual_matters<G>(mx, group_sum<G>(asum4(v)));
    const int s = x_shift(mx);
    const Limbs l = to_limbs(v, s);
#pragma unroll
    for (int k = 0; k < kLimbs; k++) im.limb(k)[b * 64 + lane] = l.b[k];
    if ((lane & 3) == 0) im.scale()[b * 16 + (lane >> 2)] = x_scale(mx, s);  // per 16 columns (G = 32: twice)
    // sums over 4 lanes (16 columns) with DPP (quad_perm) rather than LDS permutes
    const float xs = quad_sum((v.x + v.y) + (v.z + v.w));
    if ((lane & 3) == 0) im.xs16()[b * 16 + (lane >> 2)] = xs;
    return need;
}

// sum_k 256^(3-k) h_k of the four digit dot products, in fp32: two exact
// int32 partial sums (|h_k| <= 32 * 128 * 128), so only their conversions
// and the add round.
__device__ __forceinline__ float limbs(const int (&h)[kLimbs]) {
    const int top = (h[0] << 8) + h[1], low = (h[2] << 8) + h[3];
    return fmaf((float)top, 65536.f, (float)low);
}

// --------------------------------------------------------------------------- formats

// Per-format constants: block quant count, block bytes, lanes per block, max
// blocks per wave tile, max 16-byte chunks of one row tile in LDS, x scale group.
template <int T> struct Fmt;
template <> struct Fmt<12> { static constexpr int QK = 256, BB = 144, LPB = 4, TBMAX = 16, CH = 145, G = 32; };
template <> struct Fmt<13> { static constexpr int QK = 256, BB = 176, LPB = 4, TBMAX = 16, CH = 177, G = 32; };
template <> struct Fmt<14> { static constexpr int QK = 256, BB = 210, LPB = 4, TBMAX = 16, CH = 212, G = 16; };
template <> struct Fmt<8> { static constexpr int QK = 32, BB = 34, LPB = 1, TBMAX = 64, CH = 138, G = 32; };

// x registers a lane keeps for its block slot: N dwords per digit.
template <int N> struct XLimbs {
    uint32_t b[kLimbs][N];
    __device__ void load_run(const XImage &im, int dw, int at, int n) {  // n dwords from dword index dw
#pragma unroll
        for (int k = 0; k < kLimbs; k++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (r >= n / 4) break;
                const uint4 t = *reinterpret_cast<const uint4 *>(im.limb(k) + dw + 4 * r);
                b[k][at + 4 * r] = t.x; b[k][at + 4 * r + 1] = t.y; b[k][at + 4 * r + 2] = t.z; b[k][at + 4 * r + 3] = t.w;
            }
    }
    __device__ void set(int i, const Limbs &l) {
#pragma unroll
        for (int k = 0; k < kLimbs; k++) b[k][i] = l.b[k];
    }
    // the digit dot products of 4 quants (signed bytes) with x dword i
    __device__ __forceinline__ void dot(uint32_t q, int i, int (&h)[kLimbs]) const {
#pragma unroll
        for (int k = 0; k < kLimbs; k++) h[k] = sdot4(q, b[k][i], h[k]);
    }
    // the same, starting the sums (the three-operand form with a zero addend: the
    // compiler would otherwise zero each sum with a move and then accumulate)
    __device__ __forceinline__ void dot_first(uint32_t q, int i, int (&h)[kLimbs]) const {
#pragma unroll
        for (int k = 0; k < kLimbs; k++) asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(h[k]) : "v"(q), "v"(b[k][i]));
    }
};

// Per-lane conversion (column tiles, no shared image): the group's digit
// dwords for n float4s v[at..at+n), and its scale; need is or-ed with whether
// the group needs the exact path.
template <int N, int M>
__device__ __forceinline__ float convert_group(XLimbs<N> &x, const float4 (&v)[M], int at, int n, bool &need) {
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < M; k++)
        if (k >= at && k < at + n) mx = fmaxf(mx, amax4(v[k]));
    const int s = x_shift(mx);
    float sa = 0.f;
#pragma unroll
    for (int k = 0; k < M; k++)
        if (k >= at && k < at + n) {
            sa += asum4(v[k]);
            x.set(k, to_limbs(v[k], s));
        }
    need |= n == 8 ? residual_matters<32>(mx, sa) : residual_matters<16>(mx, sa);
    return x_scale(mx, s);
}

template <int T> struct XRegs;

// Q4_K: 64 columns b*256 + 64g .. +64, i.e. sub-blocks 2g ([0..7]) and 2g+1 ([8..15])
template <> struct XRegs<12> : XLimbs<16> {
    float a0, a1, xs0, xs1;
    static __device__ __forceinline__ int col(int b, int g, int k) { return b * 256 + 64 * g + 4 * k; }
    __device__ void load(const XImage &im, int b, int g, bool act) {
        load_run(im, (b * 256 + 64 * g) / 4, 0, 16);
        const float4 s = *reinterpret_cast<const float4 *>(im.xs16() + b * 16 + 4 * g);
        a0 = act ? im.scale()[b * 16 + 4 * g] : 0.f;
        a1 = act ? im.scale()[b * 16 + 4 * g + 2] : 0.f;
        xs0 = act ? s.x + s.y : 0.f;
        xs1 = act ? s.z + s.w : 0.f;
    }
    __device__ bool convert(const float4 (&v)[16], bool act) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float s = (v[k].x + v[k].y) + (v[k].z + v[k].w);
            if (k < 8) s0 += s; else s1 += s;
        }
        bool need = false;
        const float c0 = convert_group(*this, v, 0, 8, need), c1 = convert_group(*this, v, 8, 8, need);
        a0 = act ? c0 : 0.f;
        a1 = act ? c1 : 0.f;
        xs0 = act ? s0 : 0.f;
        xs1 = act ? s1 : 0.f;
        return need;
    }
};

// Q5_K: the same columns as Q4_K
template <> struct XRegs<13> : XRegs<12> {};

// Q6_K: runs r = 0..3 of 16 columns b*256 + hh*128 + 32r + l0 (hh = g/2, l0 = 16(g&1)),
// each one Q6_K sub-block with its own x scale
template <> struct XRegs<14> : XLimbs<16> {
    float a[4];
    static __device__ __forceinline__ int col(int b, int g, int k) {
        return b * 256 + (g >> 1) * 128 + 32 * (k >> 2) + 16 * (g & 1) + 4 * (k & 3);
    }
    __device__ void load(const XImage &im, int b, int g, bool act) {
        const int hh = g >> 1, l0 = 16 * (g & 1);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = b * 256 + hh * 128 + 32 * k + l0;
            load_run(im, c / 4, 4 * k, 4);
            a[k] = act ? im.scale()[c / 16] : 0.f;
        }
    }
    __device__ bool convert(const float4 (&v)[16], bool act) {
        bool need = false;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float c = convert_group(*this, v, 4 * r, 4, need);
            a[r] = act ? c : 0.f;
        }
        return need;
    }
};

// Q8_0: the 32 columns of block b
template <> struct XRegs<8> : XLimbs<8> {
    float a;
    static __device__ __forceinline__ int col(int b, int, int k) { return b * 32 + 4 * k; }
    __device__ void load(const XImage &im, int b, int, bool act) {
        load_run(im, b * 8, 0, 8);
        a = act ? im.scale()[b * 2] : 0.f;
    }
    __device__ bool convert(const float4 (&v)[8], bool act) {
        bool need = false;
        const float c = convert_group(*this, v, 0, 8, need);
        a = act ? c : 0.f;
        return need;
    }
};

// Dot product of one block slot of one row (block bytes at LDS byte address p).
// Q4_K (LlamaTransformerHandler.java:1428-1468): sum over sub-blocks 2g, 2g+1 of
//   d*ls*sum(q*x) - dmin*lm*sum(x).
// Q5_K (Q5 = true, :1525-1576): the same with qs at +48 and q's 5th bit from
// qh (+16): bit 2g / 2g+1 of qh[l].
template <bool Q5>
__device__ __forceinline__ void kq_quants(const uint8_t *p, int g, uint32_t (&lo)[8], uint32_t (&hi)[8]) {
    constexpr int kQs = Q5 ? 48 : 16;
    const uint4 qa = *reinterpret_cast<const uint4 *>(p + kQs + 32 * g);
    const uint4 qb = *reinterpret_cast<const uint4 *>(p + kQs + 16 + 32 * g);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    uint32_t q5[8] = {};
    if (Q5) {
        const uint4 ha = *reinterpret_cast<const uint4 *>(p + 16);
        const uint4 hb = *reinterpret_cast<const uint4 *>(p + 32);
        const uint32_t h[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
#pragma unroll
        for (int k = 0; k < 8; k++) q5[k] = h[k] >> (2 * g);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
        lo[k] = q[k] & 0x0F0F0F0Fu;
        hi[k] = (q[k] >> 4) & 0x0F0F0F0Fu;
        if (Q5) {
            lo[k] |= (q5[k] & 0x01010101u) << 4;
            hi[k] |= ((q5[k] >> 1) & 0x01010101u) << 4;
        }
    }
}

template <bool Q5>
__device__ __forceinline__ float kq_block_dot(const XRegs<12> &x, const uint8_t *p, int g) {
    const uint4 hd = *reinterpret_cast<const uint4 *>(p);
    int d0[kLimbs] = {}, d1[kLimbs] = {};
    {
        uint32_t lo[8], hi[8];
        kq_quants<Q5>(p, g, lo, hi);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (k == 0) {
                x.dot_first(lo[k], k, d0);  // quants 0..31: non-negative signed bytes
                x.dot_first(hi[k], 8 + k, d1);
            } else {
                x.dot(lo[k], k, d0);
                x.dot(hi[k], 8 + k, d1);
            }
        }
    }
    const float s0 = x.a0 * limbs(d0), s1 = x.a1 * limbs(d1);
    // 6-bit scale / min of sub-blocks j = 2g, 2g+1 (q4kScaleRaw / q4kMinRaw,
    // LlamaTransformerHandler.java:1471-1482), branch-free: for g >= 2 the low
    // 4 bits come from bytes 8..11 and the top 2 bits from bytes 0..7.
    const bool hiG = g >= 2;
    const int jj = (2 * g) & 3, wl = hiG ? 4 : 6, wh = hiG ? 2 : 0, mo = hiG ? 4 : 0;
    const uint32_t wls = hiG ? hd.w : hd.y, wlm = hiG ? hd.w : hd.z;
    const int ls0 = (int)(__builtin_amdgcn_ubfe(wls, 8 * jj, wl) | (__builtin_amdgcn_ubfe(hd.y, 8 * jj + 6, wh) << 4));
    const int ls1 = (int)(__builtin_amdgcn_ubfe(wls, 8 * jj + 8, wl) | (__builtin_amdgcn_ubfe(hd.y, 8 * jj + 14, wh) << 4));
    const int lm0 = (int)(__builtin_amdgcn_ubfe(wlm, 8 * jj + mo, wl) | (__builtin_amdgcn_ubfe(hd.z, 8 * jj + 6, wh) << 4));
    const int lm1 = (int)(__builtin_amdgcn_ubfe(wlm, 8 * jj + 8 + mo, wl) | (__builtin_amdgcn_ubfe(hd.z, 8 * jj + 14, wh) << 4));
    const float t = fmaf((float)ls1, s1, (float)ls0 * s0);
    const float mn = fmaf((float)lm1, x.xs1, (float)lm0 * x.xs0);
    const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
    return fmaf(d, t, -dmin * mn);
}
__device__ __forceinline__ float block_dot(const XRegs<12> &x, const uint8_t *p, int g) {
    return kq_block_dot<false>(x, p, g);
}
__device__ __forceinline__ float block_dot(const XRegs<13> &x, const uint8_t *p, int g) {
    return kq_block_dot<true>(x, p, g);
}

// Q6_K quants as signed bytes 4 * (u - 32), u = (ql nibble) | (2 qh bits) << 4:
// 4u = (nibble << 2) | (qh bits << 6) fits a byte, and 4u - 128 is 4u with its
// top bit flipped.  The factor 4 leaves the scale once per run (exact).  The
// qh word arrives with bit 1 of every 2-bit field flipped (e ^ 0xAAAAAAAA), so
// each quad is the nibbles (bits 2..5 of each byte) or-ed with the qh bits
// (bits 6..7).
__device__ __forceinline__ uint32_t q6_insert(uint32_t nib, uint32_t hb) {
    return (nib & 0x3C3C3C3Cu) | (hb & 0xC0C0C0C0u);
}
// quads 0..3 of dword k of a lane's Q6_K run (ql words a, b; qh word e)
__device__ __forceinline__ void q6_quads(uint32_t a, uint32_t b, uint32_t e, uint32_t (&q)[4]) {
    const uint32_t f = e ^ 0xAAAAAAAAu;
    q[0] = q6_insert(a << 2, f << 6);
    q[1] = q6_insert(b << 2, f << 4);
    q[2] = q6_insert(a >> 2, f << 2);
    q[3] = q6_insert(b >> 2, f);
}

// Q6_K (LlamaTransformerHandler.java:1587-1638): lane g covers half hh = g/2 and
// l in [l0, l0+16), l0 = 16*(g&1), for the four quads k (elements l + 32k).
// q = u - 32; scale d * sc[hh*8 + (g&1) + 2k].
__device__ __forceinline__ float block_dot(const XRegs<14> &x, const uint8_t *p, int g) {
    const int hh = g >> 1, l0 = 16 * (g & 1);
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p);
    const uint32_t sh = (uint32_t)(pa & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t *wa = w + (hh * 64 + l0) / 4;
    const uint32_t *wb = w + (hh * 64 + 32 + l0) / 4;
    const uint32_t *wq = w + (128 + hh * 32 + l0) / 4;
    const uint32_t *ws = w + (192 + hh * 8) / 4;
    const uint32_t *wd = w + 208 / 4;
    int acc[4][kLimbs] = {};  // [quad j][digit]
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t q[4];
        q6_quads(lds_word(wa, sh, k), lds_word(wb, sh, k), lds_word(wq, sh, k), q);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (k == 0) x.dot_first(q[j], 4 * j + k, acc[j]);
            else x.dot(q[j], 4 * j + k, acc[j]);
        }
    }
    float sj[4];
#pragma unroll
    for (int j = 0; j < 4; j++) sj[j] = x.a[j] * limbs(acc[j]);
    const uint32_t s0 = lds_word(ws, sh, 0), s1 = lds_word(ws, sh, 1);
    const uint32_t dword = lds_word(wd, sh, 0);
    const int is = g & 1;
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int idx = is + 2 * j;  // 0..7 within this half's 8 scale bytes
        const int sc = (int)(int8_t)byte_of(idx < 4 ? s0 : s1, idx & 3);
        r = fmaf((float)sc, sj[j], r);
    }
    return 0.25f * half_bits_to_float(dword) * r;
}

// Q8_0 (LlamaTransformerHandler.java:1486-1508): one lane per 34-byte block.
__device__ __forceinline__ float block_dot(const XRegs<8> &x, const uint8_t *p, int) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p);
    const uint32_t sh = (uint32_t)(pa & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - sh);
    const float d = half_bits_to_float(lds_word(w, sh, 0));
    // quants start 2 bytes into the block
    auto quants = [&](int k) { return __builtin_amdgcn_alignbyte(w[k + 1 + (sh >> 1)], w[k + (sh >> 1)], (sh + 2) & 3); };
    int h[kLimbs] = {};
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if (k == 0) x.dot_first(quants(k), k, h);
        else x.dot(quants(k), k, h);
    }
    const float s = x.a * limbs(h);
    return d * s;
}

// --------------------------------------------------------------------------- kernel

// The kernel walks the concatenation of np matrices of one format and shape
// class (same cols / pitch, same x): virtual row v belongs to problem p with
// cum[p] <= v < cum[p+1] and is row row0[p] + v - cum[p] of w[p].
struct StagedArgs {
    int np;
    const uint8_t *w[kMaxStagedGroup];  // matrix bases, 256-byte aligned (hipMalloc)
    float *y[kMaxStagedGroup];
    int row0[kMaxStagedGroup];
    int cum[kMaxStagedGroup + 1];
    size_t pitch;
    int nb, nrows, cols;  // nrows = cum[np]
    int gw;   // waves per row group (column tiles): 1, 2 or 4
    int tb;   // blocks per tile
    const float *x;
    float *swiglu;  // not null: w = {gate, up} interleaved row by row, out = silu(gate . x) * (up . x)
    // rmsnorm prologue (NORM kernels): the GEMV input is w_n * h * scale with
    // h = x + res and scale = 1 / sqrt(mean(h^2) + eps); workgroup 0 stores h
    // to x_out (not aliasing x or res)
    const float *res, *norm_w;
    float eps;
    float *x_out;
    // attention-combine prologue (COMB kernels): x is the log-sum-exp merge of
    // the chunk partials attn_part ([head][attn_nchmax][m, l, o[head_dim]]) of
    // one request, over the chunks that hold positions 0 .. *attn_pos;
    // workgroup 0 stores that x to x_out when it is not null
    const float *attn_part;
    const int *attn_pos;
    int attn_hd, attn_tc, attn_max_seq, attn_nchmax;
    bool dry;  // host only: the launcher checks that the kernel applies and launches nothing
};

// COMB: the prologue's LDS after the walk's (claim counter, per-wave flags):
// chunk weights [heads][nchmax], normalisers [heads], then the merged x [cols]
__host__ __device__ constexpr size_t staged_comb_offset(int nblk, int nw, int r, int ch) {
    return (staged_front(true, nblk, nw, r, ch) + 4 + 4 * (size_t)nw + 15) & ~size_t(15);
}
__host__ __device__ constexpr size_t staged_comb_x(int heads, int nchmax) {
    return ((size_t)heads * nchmax + heads + 3) & ~size_t(3);  // floats before the merged x
}

// SwiGLU pairing: virtual row v is row v / 2 of gate (v even) or up (v odd),
// so that a row group (R even) holds both halves of its outputs.


__device__ __forceinline__ int staged_problem(const StagedArgs &a, int v) {
    int p = 0;
#pragma unroll
    for (int i = 1; i < kMaxStagedGroup; i++)
        if (i < a.np && v >= a.cum[i]) p = i;
    return p;
}

// The exact path: launches whose x needs it (residual_matters) take it instead of
// the walk, every workgroup alike.  One wave per output (a row, or a gate / up
// pair under the SwiGLU pairing), rows strided over the grid's waves; each lane
// sums deq(w) * x over the quant units lane, lane + 64, .. with the fp32 x
// itself (NORM: formed as the prologue forms it), then the wave adds the lanes'
// sums.  That is the reference's term (LlamaTransformerHandler.java:1457-1460)
// in another summation order, at a fraction of the walk's speed: it is the
// path for x with one outlier among many much smaller elements, which the
// walk's 30-bit fixed point per sub-block does not carry to the GEMV bar.
template <int T, bool NORM, bool COMB = false>
__device__ __forceinline__ void staged_exact(const StagedArgs &args, float nscale, const float *xl = nullptr) {
    constexpr int G = Fmt<T>::G;
    const int lane = threadIdx.x & 63;
    // the wave's index, uniform (readfirstlane): rows and matrices are then chosen
    // with scalar loads of the arguments, as the walk chooses them
    const int waves = (int)(blockDim.x >> 6);
    const int gwave = __builtin_amdgcn_readfirstlane((int)blockIdx.x * waves + (int)(threadIdx.x >> 6));
    const int units = args.cols / G;
    auto xat = [&](int64_t c) {
        if constexpr (COMB) return xl[c];  // the merged x in LDS
        return NORM ? (args.norm_w[c] * (args.x[c] + args.res[c])) * nscale : args.x[c];
    };
    auto row_dot = [&](int vr) {
        const int p = args.swiglu ? (vr & 1) : staged_problem(args, vr);
        const int rr = args.swiglu ? (vr >> 1) : vr - args.cum[p];
        const uint8_t *row = args.w[p] + (size_t)(args.row0[p] + rr) * args.pitch;
        float acc = 0.f;
        for (int u = lane; u < units; u += 64)
            deq_unit<T, false>(row, u, [&](int64_t c, float w) { acc = fmaf(w, xat(c), acc); });
        return wave_sum(acc);
    };
    const int nout = args.swiglu ? args.nrows / 2 : args.nrows;
    for (int o = gwave; o < nout; o += (int)gridDim.x * waves) {
        if (args.swiglu) {
            const float g = row_dot(2 * o), u = row_dot(2 * o + 1);
            if (lane == 0) args.swiglu[o] = silu_times(g, u);
        } else {
            const float v = row_dot(o);
            if (lane == 0) {
                const int p = staged_problem(args, o);
                args.y[p][o - args.cum[p]] = v;
            }
        }
    }
}

// SX: one column tile, x shared through an LDS image; NW: waves per workgroup;
// NORM: x is the residual add and rmsnorm of the arguments (SX only)
// COMB: x is attention's combine of its chunk partials (SX, DYN, every block
// of x converted in the waves' first pass)
// DYN (one column tile only): the workgroup takes a contiguous range of row
// groups and its waves claim them one at a time from an LDS counter.  Waves
// sharing a CU do not progress at one rate (the oldest issue first), so equal
// static shares leave a CU with its last waves running alone; claimed groups
// even that out.
template <int T, int R, bool SX, int NW, bool NORM = false, bool DYN = false, bool COMB = false>
__device__ __forceinline__ void gemv_staged_body(const StagedArgs &args) {
    using F = Fmt<T>;
    constexpr int K = (F::CH + 63) / 64;  // 16-byte loads per lane per row
    extern __shared__ __align__(16) uint8_t lds[];
    // wave-uniform values live in SGPRs: derive them from a readfirstlane'd wave id
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    JH_TL(0);
    const int nb = args.nb, nrows = args.nrows, gw = args.gw, tb = args.tb;
    const size_t pitch = args.pitch;
    constexpr bool shared_x = SX;  // gw == 1: every wave needs all of x
    const int nblk = (args.cols + 255) / 256;
    XImage im{args.cols, nblk, lds};
    uint4 *stage = reinterpret_cast<uint4 *>(lds + (shared_x ? (XImage::bytes(nblk) + 15) & ~size_t(15) : 0));
    uint4 *buf0 = stage + wave * R * F::CH;
    // partial sums of column-tiled rows: [kRing][NW][R] (the shared-x ring below)
    // or [2][NW][R] (per-lane x), then the ring's arrival and release counters
    float *part = reinterpret_cast<float *>(stage + NW * R * F::CH);
    int *ring_arr = reinterpret_cast<int *>(part + kRing * NW * R);  // [slot][cell]: arrivals
    int *ring_done = ring_arr + kRing * NW;                            // [slot][cell]: uses finished
    int *claim = reinterpret_cast<int *>(lds + staged_front(SX, nblk, NW, R, F::CH));  // DYN: next group
    int *xneed = claim + 1;  // [NW]: x needs the exact path

    const int slots = NW / gw;  // row groups processed side by side by one workgroup
    const int tile = wave % gw, slot = wave / gw;
    const int ngroups = (nrows + R - 1) / R;
    const int gstride = gridDim.x * slots;
    int grp = blockIdx.x * slots + slot;
    // DYN: this workgroup's groups [gbeg, gend); wave w starts with gbeg + w, then claims
    const int gper = ngroups / (int)gridDim.x, gext = ngroups - gper * (int)gridDim.x;
    const int gbeg = (int)blockIdx.x * gper + min((int)blockIdx.x, gext);
    const int gend = gbeg + gper + ((int)blockIdx.x < gext ? 1 : 0);
    // the ring's counters start at zero; read only after the barrier of the x prologue
    if (SX && (int)threadIdx.x < 2 * kRing * NW) ring_arr[threadIdx.x] = 0;
    if constexpr (DYN) {
        grp = gbeg + wave;
        if (threadIdx.x == 0) *claim = gbeg + NW;  // read only after the barrier of the x prologue
    }

    const int blk = lane / F::LPB, sub = lane % F::LPB;
    const int b0 = tile * tb;                        // first block of this wave's tile
    const int ntile = min(tb, nb - b0);              // blocks in this tile
    const bool act = blk < ntile;
    const int b = b0 + (act ? blk : 0);
    const size_t tile_off = (size_t)b0 * F::BB;
    const int tile_bytes = ntile * F::BB;
    const int nch = (int)((15 + tile_bytes + 15) >> 4);  // chunks to cover any 2-byte-aligned start
    int ld_off[K];                                        // per-lane chunk offsets (clamped)
#pragma unroll
    for (int k = 0; k < K; k++) ld_off[k] = 16 * min(lane + 64 * k, nch - 1);
    const int lane_blk = (act ? blk : 0) * F::BB;

    // 1. x loads, before any weight load so that waiting for x does not wait
    //    for the weight stream: with a shared image, every block of 256 this
    //    wave converts (up to 16 blocks over 4 waves for one column tile, up to
    //    64 over 8-16 waves for column tiles), all issued here rather than one
    //    round trip per block; otherwise this lane's own columns
    // image blocks each wave converts: one column tile has at most 16 blocks
    constexpr int NXS = (((DYN || NORM || NW < 8) ? 16 : 64) + NW - 1) / NW;
    constexpr int NX = SX ? NXS : (T == 8 ? 8 : 16);
    float4 xv[NX];
    float4 rv[NORM ? NXS : 1], nwv[NORM ? NXS : 1];
    if constexpr (shared_x) {
#pragma unroll
        for (int k = 0; k < NXS; k++) {
            const int c = (wave + NW * k) * 256 + lane * 4;
            if constexpr (!COMB) xv[k] = x_load4(args.x, args.cols, c);
            if constexpr (NORM) {
                rv[k] = x_load4(args.res, args.cols, c);
                nwv[k] = x_load4(args.norm_w, args.cols, c);
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < NX; k++) xv[k] = x_load4(args.x, args.cols, XRegs<T>::col(b, sub, k));
    }
    asm volatile("" ::: "memory");

    // 2. weight loads.  Byte offsets are relative to args.w, which is 256-byte
    //    aligned, so a span's alignment follows from its offset alone.
    uint4 v[R][K];
    int start[R];  // misalignment (byte offset mod 16) of each row tile in flight
    auto issue = [&](int g) {
        const int r0 = min(g, ngroups - 1) * R;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int vr = min(r0 + i, nrows - 1);
            // uniform over the wave: the matrix is chosen with scalar loads
            const int p = __builtin_amdgcn_readfirstlane(args.swiglu ? (vr & 1) : staged_problem(args, vr));
            const int rr = args.swiglu ? (vr >> 1) : vr - args.cum[p];
            const size_t off = (size_t)(args.row0[p] + rr) * pitch + tile_off;
            start[i] = (int)(off & 15);
            const uint8_t *base = args.w[p] + (off & ~size_t(15));
#pragma unroll
            for (int k = 0; k < K; k++) v[i][k] = load_stream16(base + ld_off[k]);
        }
    };
    auto park = [&](uint4 *dst) {
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int k = 0; k < K; k++)
                if (lane + 64 * k < F::CH) dst[i * F::CH + lane + 64 * k] = v[i][k];
    };
    if constexpr (DYN) grp = grp < gend ? grp : ngroups;  // a range shorter than the waves: nothing to do
    // The first weight loads: per-lane x issues them now; a shared image issues
    // them after its barrier.  A CU accepts only so many loads at a time, so the
    // waves' first bursts issue in turns (the last third of a 12-wave workgroup
    // ~1 us after the first); issued before the conversion, they held each
    // wave's share of it, and with it the barrier, until the wave's turn came.
    if constexpr (!shared_x) issue(grp);
    asm volatile("" ::: "memory");

    // 3. x into registers
    XRegs<T> xr;
    float nscale = 1.f;  // NORM: the rmsnorm scale
    if constexpr (NORM) {
        // h = x + res and its sum of squares: per lane, then over the wave (DPP),
        // then over the waves in wave order through LDS (the part area, unused
        // until the walk); rmsNorm, LlamaTransformerHandler.java:818-826
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < NXS; k++) {
            const int c = (wave + NW * k) * 256 + lane * 4;
            const bool in = c < args.cols;
            float4 h = make_float4(xv[k].x + rv[k].x, xv[k].y + rv[k].y, xv[k].z + rv[k].z, xv[k].w + rv[k].w);
            if (!in) h = make_float4(0.f, 0.f, 0.f, 0.f);
            if (blockIdx.x == 0 && in && args.x_out) *reinterpret_cast<float4 *>(args.x_out + c) = h;
            xv[k] = h;
            ss += ((h.x * h.x + h.y * h.y) + (h.z * h.z + h.w * h.w));
        }
        ss = wave_sum(ss);
        if (lane == 0) part[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) tot += part[w];
        const float scale = 1.f / (float)sqrt((double)(tot / (float)args.cols + args.eps));
        nscale = scale;
#pragma unroll
        for (int k = 0; k < NXS; k++)
            xv[k] = make_float4(nwv[k].x * xv[k].x * scale, nwv[k].y * xv[k].y * scale, nwv[k].z * xv[k].z * scale,
                                nwv[k].w * xv[k].w * scale);
    }
    float *cmb_x = nullptr;  // COMB: the merged x in LDS (the exact path reads it)
    if constexpr (COMB) {
        // attn_combine_k's arithmetic in its order (gqa, LlamaTransformerHandler.java:1678-1731):
        // per head, M = the chunks' largest score, weights exp(m_c - M) (double),
        // L = sum_c l_c w_c in chunk order, x[d] = (sum_c o_c[d] w_c in chunk order) / L
        const int hd = args.attn_hd, nh = args.cols / hd, nchmax = args.attn_nchmax, stride = hd + 2;
        float *wcl = reinterpret_cast<float *>(lds + staged_comb_offset(nblk, NW, R, F::CH));
        float *Ll = wcl + nh * nchmax;
        cmb_x = wcl + staged_comb_x(nh, nchmax);
        const int npos = min(*args.attn_pos, args.attn_max_seq - 1) + 1;
        const int nch = min((npos + args.attn_tc - 1) / args.attn_tc, nchmax);
        // a. wave w takes heads w, w + NW, ..: lane c holds chunk c's (m, l)
        constexpr int HW = 4;  // heads per wave (the launcher admits at most 4 NW)
        float mv[HW], lv[HW];
#pragma unroll
        for (int j = 0; j < HW; j++) {
            const int h = min(wave + NW * j, nh - 1), c = min(lane, nch - 1);
            const float *ph = args.attn_part + ((size_t)h * nchmax + c) * stride;
            mv[j] = ph[0];
            lv[j] = ph[1];
        }
#pragma unroll
        for (int j = 0; j < HW; j++) {
            const int h = wave + NW * j;
            if (h >= nh) break;  // uniform over the wave
            const bool in = lane < nch;
            float M = in ? mv[j] : -INFINITY;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
            const float w = in ? (float)exp((double)(mv[j] - M)) : 0.f;
            if (in) wcl[h * nchmax + lane] = w;
            float L = 0.f;
            for (int c = 0; c < nch; c++)
                L = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(lv[j]), c)),
                         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), c)), L);
            if (lane == 0) Ll[h] = L;
        }
        __syncthreads();
        // b. this wave's blocks: lane's 4 columns (one head) merged over the chunks
#pragma unroll
        for (int k = 0; k < NXS; k++) {
            const int c0 = (wave + NW * k) * 256 + lane * 4;
            if (c0 >= args.cols) {
                xv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
                continue;
            }
            const int h = c0 / hd, d = c0 - h * hd;
            const float *op = args.attn_part + (size_t)h * nchmax * stride + 2 + d;
            const float *wh = wcl + h * nchmax;
            float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
            int c = 0;
            for (; c + 8 <= nch; c += 8) {
                float2 a[8], b[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    a[u] = *reinterpret_cast<const float2 *>(op + (size_t)(c + u) * stride);
                    b[u] = *reinterpret_cast<const float2 *>(op + (size_t)(c + u) * stride + 2);
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float wc = wh[c + u];
                    o0 = fmaf(a[u].x, wc, o0);
                    o1 = fmaf(a[u].y, wc, o1);
                    o2 = fmaf(b[u].x, wc, o2);
                    o3 = fmaf(b[u].y, wc, o3);
                }
            }
            for (; c < nch; c++) {
                const float2 a = *reinterpret_cast<const float2 *>(op + (size_t)c * stride);
                const float2 b = *reinterpret_cast<const float2 *>(op + (size_t)c * stride + 2);
                const float wc = wh[c];
                o0 = fmaf(a.x, wc, o0);
                o1 = fmaf(a.y, wc, o1);
                o2 = fmaf(b.x, wc, o2);
                o3 = fmaf(b.y, wc, o3);
            }
            const float L = Ll[h];
            xv[k] = make_float4(o0 / L, o1 / L, o2 / L, o3 / L);
            *reinterpret_cast<float4 *>(cmb_x + c0) = xv[k];
            if (blockIdx.x == 0 && args.x_out) *reinterpret_cast<float4 *>(args.x_out + c0) = xv[k];
        }
    }
    if constexpr (shared_x) {
        // each wave's flag: whether a group it converted needs the exact path
        bool need = false;
#pragma unroll
        for (int k = 0; k < NXS; k++)
            if (wave + NW * k < nblk) need |= x_quant_block<F::G>(im, wave + NW * k, xv[k]);
        for (int bx = wave + NW * NXS; bx < nblk; bx += NW)
            need |= x_quant_block<F::G>(im, bx, x_load4(args.x, args.cols, bx * 256 + lane * 4));
        const bool wneed = __builtin_amdgcn_ballot_w64(need) != 0;  // over all lanes of the wave
        if (lane == 0) xneed[wave] = wneed;
        __syncthreads();
        JH_TL(1);
        int anyneed = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) anyneed |= xneed[w];
        if (__builtin_amdgcn_readfirstlane(anyneed)) {  // uniform over the workgroup; see residual_matters
            staged_exact<T, NORM, COMB>(args, nscale, cmb_x);
            return;
        }
        issue(grp);
        xr.load(im, b, sub, act);
    } else {
#pragma unroll
        for (int k = 0; k < NX; k++) xv[k] = x_mask4(xv[k], args.cols, XRegs<T>::col(b, sub, k));
        if (__syncthreads_or(xr.convert(xv, act))) {  // uniform over the workgroup
            staged_exact<T, NORM>(args, nscale);
            return;
        }
    }

    // 4. pipelined walk over row groups
    if (SX && gw != 1 && grp >= ngroups) return;  // fewer groups than slots: this slot has none
    park(buf0);
    wave_lds_sync();
    JH_TL(2);
    int it = 0;
    while (true) {
        int cstart[R];
#pragma unroll
        for (int i = 0; i < R; i++) cstart[i] = start[i];
        int next = grp + gstride;
        if constexpr (DYN) {
            int c = 0;
            if (lane == 0) c = __hip_atomic_fetch_add(claim, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            next = __builtin_amdgcn_readfirstlane(c);
            next = next < gend ? next : ngroups;  // past the range: the loads below repeat the last group
        }
        issue(next);
        const int r0 = grp * R;
        const uint8_t *cb = reinterpret_cast<const uint8_t *>(buf0);
        float s[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const uint8_t *row = cb + i * F::CH * 16 + cstart[i];
            const float d = block_dot(xr, row + lane_blk, sub);
            s[i] = wave_sum_to63(act ? d : 0.f);
        }
        auto store = [&](int vr, float val) {
            const int p = staged_problem(args, vr);
            args.y[p][vr - args.cum[p]] = val;
        };
        if (gw == 1) {
            if (lane == 63) {
                if (args.swiglu) {
#pragma unroll
                    for (int i = 0; i + 1 < R; i += 2)
                        if (r0 + i < nrows) args.swiglu[(r0 + i) >> 1] = silu_times(s[i], s[i + 1]);
                } else {
#pragma unroll
                    for (int i = 0; i < R; i++)
                        if (r0 + i < nrows) store(r0 + i, s[i]);
                }
            }
            if (next >= ngroups) {
                JH_TL(3);
                break;
            }
        } else if constexpr (SX) {
            // Column tiles meet in a ring of kRing cells per slot instead of at a
            // workgroup barrier, so that a wave's arithmetic overlaps the other
            // waves' loads.  The gw waves of a slot walk the same groups in the same
            // order; the it-th group uses cell it % kRing for the (it / kRing)-th
            // time.  A wave first waits until that cell's previous use is finished
            // (the slowest wave never waits, so the waits end), writes its partial
            // sums, and counts its arrival; the last of the gw waves adds the
            // partials in tile order (as the barrier version did) and stores y.
            const int cell = slot * kRing + (it & (kRing - 1));
            const int use = it / kRing;
            if (use > 0)
                for (int spin = 0;; spin++) {
                    if (__hip_atomic_load(ring_done + cell, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= use) break;
                    if (spin == (1 << 22)) {  // never expected: counted (the sums are then wrong) rather than a hang
                        if (lane == 0) __hip_atomic_fetch_add(&g_sync_faults, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            float *pc = part + cell * gw * R;
            int a = 0;
            if (lane == 63) {
#pragma unroll
                for (int i = 0; i < R; i++) pc[tile * R + i] = s[i];
                a = __hip_atomic_fetch_add(ring_arr + cell, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            a = __builtin_amdgcn_readlane(a, 63);
            if (a == use * gw + gw - 1) {  // the last arrival for this group
                if (lane == 63) {
                    float t[R];
#pragma unroll
                    for (int i = 0; i < R; i++) {
                        t[i] = 0.f;
                        for (int q = 0; q < gw; q++) t[i] += pc[q * R + i];
                    }
                    if (args.swiglu) {
#pragma unroll
                        for (int i = 0; i + 1 < R; i += 2)
                            if (r0 + i < nrows) args.swiglu[(r0 + i) >> 1] = silu_times(t[i], t[i + 1]);
                    } else {
#pragma unroll
                        for (int i = 0; i < R; i++)
                            if (r0 + i < nrows) store(r0 + i, t[i]);
                    }
                    __hip_atomic_store(ring_done + cell, use + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
            if (next >= ngroups) {
                JH_TL(3);
                break;
            }
        } else {
            float *pp = part + (it & 1) * NW * R;
            if (lane == 63)
#pragma unroll
                for (int i = 0; i < R; i++) pp[wave * R + i] = s[i];
            __syncthreads();
            if (tile == 0 && lane == 63 && grp < ngroups) {
                float t[R];
#pragma unroll
                for (int i = 0; i < R; i++) {
                    t[i] = 0.f;
                    for (int q = 0; q < gw; q++) t[i] += pp[(slot * gw + q) * R + i];
                }
                if (args.swiglu) {
#pragma unroll
                    for (int i = 0; i + 1 < R; i += 2)
                        if (r0 + i < nrows) args.swiglu[(r0 + i) >> 1] = silu_times(t[i], t[i + 1]);
                } else {
#pragma unroll
                    for (int i = 0; i < R; i++)
                        if (r0 + i < nrows) store(r0 + i, t[i]);
                }
            }
            // every wave of the workgroup iterates while slot 0 has work
            if (next - slot >= ngroups) break;
        }
        // the group just computed is done with the buffer: park the next one there
        wave_lds_sync();
        park(buf0);
        wave_lds_sync();
        grp = next;
        it++;
    }
}

template <int T, int R, bool SX, int NW, bool NORM, bool DYN, bool COMB = false>
__global__ __launch_bounds__(64 * NW) void gemv_staged(StagedArgs args) {
    gemv_staged_body<T, R, SX, NW, NORM, DYN, COMB>(args);
}

// One-column-tile rows take one workgroup per CU (16 waves of one row, or 12 of
// two for the SwiGLU pairing) whose waves claim row groups (DYN), unless JUNO_STAGED_DYN=0: then 4-wave workgroups, up to 3 per CU,
// with equal static shares (JUNO_STAGED_NW = 8 or 12 widens them), for A/B runs.
// Measured with per-workgroup timestamps on the static layout: on the 8B lm_head
// the first workgroup on each CU ended at ~53 us, the second at ~62, the third at
// ~73 us (the CU issues its oldest waves first).
static bool staged_dyn() {
    static const bool on = [] {
        const char *v = getenv("JUNO_STAGED_DYN");
        return !(v && v[0] == '0');
    }();
    return on;
}

// Waves per workgroup of the static one-column-tile kernels: JUNO_STAGED_NW (4,
// 8 or 12) overrides the default for tuning runs.
static int staged_waves() {
    static const int nw = [] {
        const char *v = getenv("JUNO_STAGED_NW");
        const int x = v ? atoi(v) : 0;
        return (x == 4 || x == 8 || x == 12) ? x : 4;
    }();
    return nw;
}

// Waves per workgroup of the column-tiled kernels (rows of more than 16 blocks):
// 16 (the default), 12 or 8 share one LDS image of x between 4, 3 or 2 row groups
// side by side, so that a CU reads x once instead of once per workgroup (per-lane
// conversion fetched all of x per 4-wave workgroup: 44 MB from L2 for the 8B
// ffn_down, next to its 48 MB of weights); 4 (JUNO_STAGED_WIDE=4) converts x per
// lane into registers.
static int staged_wide_waves() {
    static const int nw = [] {
        const char *v = getenv("JUNO_STAGED_WIDE");
        const int x = v ? atoi(v) : 0;
        return (x == 4 || x == 8 || x == 12 || x == 16) ? x : 16;
    }();
    return nw;
}

// Workgroups of `kern` with `lds` bytes of dynamic LDS that fit on the device
// at once (at most 3 per CU; JUNO_STAGED_PER_CU = 1..8 sets that cap for tuning runs).
static int staged_per_cu_cap() {
    static const int v = [] {
        const char *e = getenv("JUNO_STAGED_PER_CU");
        const int x = e ? atoi(e) : 0;
        return (x >= 1 && x <= 8) ? x : 3;
    }();
    return v;
}
static int cu_count() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
        return n;
    }();
    return cus;
}
static int resident_workgroups(const void *kern, int threads, size_t lds) {
    const int cus = cu_count();
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    const int cap = staged_per_cu_cap();
    return cus * (per_cu > cap ? cap : per_cu);
}

template <int T, int R, bool SX, int NW, bool NORM = false, bool DYN = false, bool COMB = false>
hipError_t launch_staged_nw(const StagedArgs &sa, int nblk, int ngroups, hipStream_t s) {
    using F = Fmt<T>;
    const void *kern = reinterpret_cast<const void *>(&gemv_staged<T, R, SX, NW, NORM, DYN, COMB>);
    // allow more than the default 64 KB of dynamic LDS (160 KB per CU on gfx950).  The
    // call has been refused for some instantiations: its error is cleared here, so
    // that the launch's own status is the one reported, and such a kernel keeps 64 KB.
    static const size_t lds_max = [kern] {
        const bool ok = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        (void)hipGetLastError();
        return ok ? size_t(160) * 1024 : size_t(64) * 1024;
    }();
    // walk, claim counter, per-wave flags
    size_t base = staged_front(SX, nblk, NW, R, F::CH) + 4 + 4 * NW;
    if (COMB) {
        const int nh = sa.cols / sa.attn_hd;
        base = staged_comb_offset(nblk, NW, R, F::CH) + 4 * (staged_comb_x(nh, sa.attn_nchmax) + (size_t)sa.cols);
    }
    if (base > lds_max) return hipErrorNotSupported;
    const int slots = NW / sa.gw;
    const int need = (ngroups + slots - 1) / slots;
    // persistent grid: as many workgroups as fit at once (DYN: one per CU), capped by the work
    int wgs = DYN ? cu_count() : resident_workgroups(kern, 64 * NW, base);
    if (wgs > need) wgs = need;
    if (sa.dry) return hipSuccess;
    gemv_staged<T, R, SX, NW, NORM, DYN, COMB><<<wgs, 64 * NW, base, s>>>(sa);
    return hipGetLastError();
}

template <int T, int R>
hipError_t launch_staged_t(StagedArgs sa, hipStream_t s) {
    using F = Fmt<T>;
    const int nb = sa.nb;
    sa.gw = nb <= F::TBMAX ? 1 : nb <= 2 * F::TBMAX ? 2 : 4;
    sa.tb = (nb + sa.gw - 1) / sa.gw;
    const int nblk = (sa.cols + 255) / 256;
    const int ngroups = (sa.nrows + R - 1) / R;
    if (sa.attn_part) {  // one pass of 16 waves converts every block; one row per group
        if (sa.gw != 1 || nblk > 16 || R != 1 || !staged_dyn()) return hipErrorNotSupported;
        return launch_staged_nw<T, 1, true, 16, false, true, true>(sa, nblk, ngroups, s);
    }
    if (sa.norm_w) {  // the rmsnorm prologue needs the shared image and every block in one pass of the waves
        if (sa.gw != 1 || nblk > 16) return hipErrorNotSupported;
        if (staged_dyn()) {
            if (R == 1) return launch_staged_nw<T, 1, true, 16, true, true>(sa, nblk, ngroups, s);
            return launch_staged_nw<T, R, true, 12, true, true>(sa, nblk, ngroups, s);
        }
        return launch_staged_nw<T, R, true, 4, true>(sa, nblk, ngroups, s);
    }
    if (sa.gw != 1) {
        hipError_t e = hipErrorNotSupported;
        switch (staged_wide_waves()) {  // the shared image needs the LDS for it and the row groups
        case 8: e = launch_staged_nw<T, R, true, 8>(sa, nblk, ngroups, s); break;
        case 12: e = launch_staged_nw<T, R, true, 12>(sa, nblk, ngroups, s); break;
        case 16: e = launch_staged_nw<T, R, true, 16>(sa, nblk, ngroups, s); break;
        default: break;
        }
        if (e != hipErrorNotSupported) return e;
        return launch_staged_nw<T, R, false, 4>(sa, nblk, ngroups, s);
    }
    if (staged_dyn()) {
        // one row per group: 16 waves (what fits 128 VGPRs); two (the SwiGLU pairing): 12
        if (R == 1) return launch_staged_nw<T, 1, true, 16, false, true>(sa, nblk, ngroups, s);
        return launch_staged_nw<T, R, true, 12, false, true>(sa, nblk, ngroups, s);
    }
    switch (staged_waves()) {
    case 8: return launch_staged_nw<T, R, true, 8>(sa, nblk, ngroups, s);
    case 12: return launch_staged_nw<T, R, true, 12>(sa, nblk, ngroups, s);
    default: return launch_staged_nw<T, R, true, 4>(sa, nblk, ngroups, s);
    }
}

}  // namespace

bool staged_supported(int type, int cols) {
    switch (type) {
    case 12: return cols % 256 == 0 && cols / 256 <= 4 * Fmt<12>::TBMAX;
    case 13: return cols % 256 == 0 && cols / 256 <= 4 * Fmt<13>::TBMAX;
    case 14: return cols % 256 == 0 && cols / 256 <= 4 * Fmt<14>::TBMAX;
    case 8: return cols % 32 == 0 && cols / 32 <= 4 * Fmt<8>::TBMAX;
    default: return false;
    }
}

// Rows per group; JUNO_STAGED_R (1, 2 or 4) overrides the default for tuning runs.
static int staged_rows(int def) {
    static const int r = [] {
        const char *v = getenv("JUNO_STAGED_R");
        const int x = v ? atoi(v) : 0;
        return (x == 1 || x == 2 || x == 4) ? x : 0;
    }();
    return r ? r : def;
}

template <int T>
static hipError_t launch_staged_r(const StagedArgs &sa, int R, hipStream_t s) {
    switch (R) {
    case 1: return launch_staged_t<T, 1>(sa, s);
    case 2: return launch_staged_t<T, 2>(sa, s);
    default: return launch_staged_t<T, 4>(sa, s);
    }
}

// Column-tiled rows (more blocks than one wave's tile): one row per group, 16 waves
// sharing the x image (8B ffn_down 20.2 -> 19.3 us, TinyLlama 10.1 -> 7.9 us,
// Phi-3 Q8_0 13.3 -> 10.1 us against two rows and per-lane x).
static bool staged_wide(int type, int nb) {
    switch (type) {
    case 12: return nb > Fmt<12>::TBMAX;
    case 13: return nb > Fmt<13>::TBMAX;
    case 14: return nb > Fmt<14>::TBMAX;
    case 8: return nb > Fmt<8>::TBMAX;
    default: return false;
    }
}
static hipError_t launch_staged_any(const StagedArgs &sa, int type, hipStream_t s) {
    // One row per group unless the SwiGLU pairing needs two.  With one row, 16
    // waves fit a CU (128 VGPRs each) against 12 waves of two rows: the same bytes
    // in flight, but groups half as long, so the claims balance the waves more
    // finely (same box: [gate, up] 17.4 -> 16.3 us, lm_head 75.2 -> 72.2 us, the
    // B = 1 step 1.644 -> 1.617 ms).
    const int R = staged_rows(staged_wide(type, sa.nb) || !sa.swiglu ? 1 : 2);
    switch (type) {
    case 12: return launch_staged_r<12>(sa, R, s);
    case 13: return launch_staged_r<13>(sa, R, s);
    case 14: return launch_staged_r<14>(sa, R, s);
    case 8: return launch_staged_r<8>(sa, R, s);
    default: return hipErrorNotSupported;
    }
}

// The staged kernel pays a fixed prologue (x conversion, one barrier) of a
// few microseconds; below ~28 MB of packed weights per launch the one-shot
// kernels of jh_gemv.hip finish first (measured on MI355X at Llama-3-8B and
// Phi-3 shapes).  JUNO_STAGED_R set forces the staged kernel (tests, tuning).
// Column-tiled rows (16 waves sharing x, no barrier between row groups) win
// from ~16 MB over rotated copies (Phi-3 Q6_K ffn_down 20.6 MB: 16.0 -> 11.3 us,
// Q8_0 26.7 MB: 12.6 -> 9.8 us), but not at the TinyLlama ffn_down (9.5 MB),
// whose input arrives from the previous launch (+0.8 us per layer in the step).
// A launch that also carries the residual add + rmsnorm saves a launch of its
// own, which pays for the prologue from ~8 MB (TinyLlama [gate, up], 13 MB).
constexpr size_t kStagedMinBytes = 28u << 20;
constexpr size_t kStagedMinWideBytes = 16u << 20;
constexpr size_t kStagedMinFusedBytes = 8u << 20;
// With attention's combine in the prologue the launch also saves the combine's
// launch; JUNO_STAGED_MIN_COMB (MB) overrides this for tuning runs.
constexpr size_t kStagedMinCombBytes = 0;

// Thresholds in MB: JUNO_STAGED_MIN (one column tile), JUNO_STAGED_MIN_WIDE
// (column-tiled rows) and JUNO_STAGED_MIN_FUSED (with the rmsnorm prologue)
// override the defaults for tuning runs.
static size_t env_mb(const char *name, size_t def) {
    const char *v = getenv(name);
    return v ? (size_t)atoi(v) << 20 : def;
}
static bool staged_wanted(size_t bytes, int type, int cols, bool fused = false) {
    static const size_t narrow = env_mb("JUNO_STAGED_MIN", kStagedMinBytes);
    static const size_t wideb = env_mb("JUNO_STAGED_MIN_WIDE", kStagedMinWideBytes);
    static const size_t fusedb = env_mb("JUNO_STAGED_MIN_FUSED", kStagedMinFusedBytes);
    const bool wide = staged_wide(type, type == 8 ? cols / 32 : cols / 256);
    size_t min = wide ? wideb : narrow;
    if (fused && fusedb < min) min = fusedb;
    return bytes >= min || getenv("JUNO_STAGED_R") != nullptr;
}

static void set_norm(StagedArgs &sa, const NormSpec *norm) {
    if (!norm) return;
    sa.res = norm->res;
    sa.norm_w = norm->w;
    sa.eps = norm->eps;
    sa.x_out = norm->x_out;
}

hipError_t launch_gemv_staged(const GemvArgs &a, hipStream_t s, const NormSpec *norm) {
    if (a.batch != 1 || !staged_supported(a.type, a.cols)) return hipErrorNotSupported;
    const int nrows = a.row_end - a.row_start;
    if (!staged_wanted((size_t)nrows * a.pitch, a.type, a.cols, norm != nullptr)) return hipErrorNotSupported;
    StagedArgs sa = {};
    sa.np = 1;
    sa.w[0] = a.w;
    sa.y[0] = a.y;
    sa.row0[0] = a.row_start;
    sa.cum[0] = 0;
    sa.cum[1] = nrows;
    sa.pitch = a.pitch;
    sa.nb = a.type == 8 ? a.cols / 32 : a.cols / 256;
    sa.nrows = nrows;
    sa.cols = a.cols;
    sa.x = a.x;
    set_norm(sa, norm);
    return launch_staged_any(sa, a.type, s);
}

hipError_t launch_gemv_staged_combine(const GemvArgs &a, const CombineSpec &c, hipStream_t s, bool check_only) {
    if (a.batch != 1 || !staged_supported(a.type, a.cols) || a.cols % 256 || c.head_dim < 4 || c.head_dim % 4 ||
        a.cols % c.head_dim || a.cols / c.head_dim > 4 * 16 || c.nchmax < 1 || c.nchmax > 64 || c.tc < 1)
        return hipErrorNotSupported;
    const int nrows = a.row_end - a.row_start;
    static const size_t comb_min = env_mb("JUNO_STAGED_MIN_COMB", kStagedMinCombBytes);
    if ((size_t)nrows * a.pitch < comb_min && !getenv("JUNO_STAGED_R")) return hipErrorNotSupported;
    StagedArgs sa = {};
    sa.np = 1;
    sa.w[0] = a.w;
    sa.y[0] = a.y;
    sa.row0[0] = a.row_start;
    sa.cum[0] = 0;
    sa.cum[1] = nrows;
    sa.pitch = a.pitch;
    sa.nb = a.type == 8 ? a.cols / 32 : a.cols / 256;
    sa.nrows = nrows;
    sa.cols = a.cols;
    sa.x = nullptr;
    sa.x_out = c.x_out;
    sa.attn_part = c.part;
    sa.attn_pos = c.pos;
    sa.attn_hd = c.head_dim;
    sa.attn_tc = c.tc;
    sa.attn_max_seq = c.max_seq;
    sa.attn_nchmax = c.nchmax;
    sa.dry = check_only;
    return launch_staged_any(sa, a.type, s);
}

hipError_t launch_gemv_swiglu(const GroupProblem &gate, const GroupProblem &up, float *out, hipStream_t s,
                              const NormSpec *norm) {
    const int R = staged_rows(2);
    if (R % 2 || gate.type != up.type || gate.cols != up.cols || gate.pitch != up.pitch || gate.x != up.x ||
        gate.nrows != up.nrows || gate.nrows < 1 || !staged_supported(gate.type, gate.cols))
        return hipErrorNotSupported;
    if (!staged_wanted(2 * (size_t)gate.nrows * gate.pitch, gate.type, gate.cols, norm != nullptr)) return hipErrorNotSupported;
    // Column-tiled rows take one row per group in the grouped launch, so that pairing
    // cannot reproduce their sums bit for bit: the caller's grouped launch + product does.
    if (staged_wide(gate.type, gate.type == 8 ? gate.cols / 32 : gate.cols / 256)) return hipErrorNotSupported;
    StagedArgs sa = {};
    sa.np = 2;
    sa.w[0] = gate.w;
    sa.w[1] = up.w;
    sa.cum[1] = gate.nrows;
    sa.cum[2] = 2 * gate.nrows;
    sa.pitch = gate.pitch;
    sa.nb = gate.type == 8 ? gate.cols / 32 : gate.cols / 256;
    sa.nrows = 2 * gate.nrows;
    sa.cols = gate.cols;
    sa.x = gate.x;
    sa.swiglu = out;
    set_norm(sa, norm);
    return launch_staged_any(sa, gate.type, s);
}

hipError_t launch_gemv_staged_group(int n, const GroupProblem *p, hipStream_t s) {
    if (n < 1 || n > kMaxStagedGroup) return hipErrorNotSupported;
    size_t bytes = 0;
    for (int i = 0; i < n; i++) {
        if (p[i].type != p[0].type || p[i].cols != p[0].cols || p[i].pitch != p[0].pitch || p[i].x != p[0].x ||
            !staged_supported(p[i].type, p[i].cols))
            return hipErrorNotSupported;
        bytes += (size_t)p[i].nrows * p[i].pitch;
    }
    if (!staged_wanted(bytes, p[0].type, p[0].cols)) return hipErrorNotSupported;
    StagedArgs sa = {};
    sa.np = n;
    int total = 0;
    for (int i = 0; i < n; i++) {
        sa.w[i] = p[i].w;
        sa.y[i] = p[i].y;
        sa.row0[i] = 0;
        sa.cum[i] = total;
        total += p[i].nrows;
    }
    sa.cum[n] = total;
    sa.pitch = p[0].pitch;
    sa.nb = p[0].type == 8 ? p[0].cols / 32 : p[0].cols / 256;
    sa.nrows = total;
    sa.cols = p[0].cols;
    sa.x = p[0].x;
    if (total == 0) return hipSuccess;
    return launch_staged_any(sa, p[0].type, s);
}

hipError_t sync_faults(unsigned *count) {
    unsigned v = 0;
    hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_sync_faults), sizeof(v));
    if (e != hipSuccess) return e;
    const unsigned zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_sync_faults), &zero, sizeof(zero));
    *count = v;
    return e;
}

hipError_t timeline_read(unsigned long long *out, size_t n) {
#ifdef JH_TIMELINE
    if (n > (size_t)kTlWaves * 4) n = (size_t)kTlWaves * 4;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_timeline), n * sizeof(unsigned long long));
#else
    (void)out;
    (void)n;
    return hipErrorNotSupported;
#endif
}

}  // namespace jh
