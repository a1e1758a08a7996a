// jh_mfma.hip -- batched decode (3 <= B <= 64) on Q4_K / Q5_K / Q6_K / Q8_0 through
// LDS + fp16 MFMA.
//
// Y[b][r] = sum_c deq(W[r][c]) * X[b][c] is a dense contraction once B >= 16:
// per HBM byte it needs 2B/0.5625 flops (Q4_K), more than the VALU can issue
// without packed fp32, but below the MFMA ridge (~312 flop/B).  The kernels
// keep every weight integer exact and move the arithmetic to
// v_mfma_f32_32x32x16_f16 with x as the A operand and weights as B, so the
// accumulator of a lane holds one weight row (its own) for 16 batch columns:
//
//  * Weights: each format turns its packed integers into exact fp16 integers
//    (Q4_K: ls*q <= 945 from 1024 + ls*q by one 24-bit multiply-add and one
//    fp16 subtraction per pair; Q6_K:
//    u - 32; Q8_0: q) and applies its fp32 scales per row in registers -- Q4_K
//    once per 256 columns with d and dmin (the min term is one extra MFMA
//    against per-sub-block sums of x), Q6_K per 16-column sub-block with the
//    reference's d*sc, Q8_0 per 32-column block with d.
//  * Activations: x is split into fp16 hi + lo limbs (x = hi + lo to ~2^-22,
//    so only the order of summation differs from fp32) after a power-of-two
//    scale per (column, 256-column super-block) that keeps fp16 in range.
//    Each workgroup converts the fp32 x slice of a super-block straight into
//    its LDS image while it stages the weights (no separate prep launch).
//  * Work split: a workgroup is kWaves waves x 32 rows, all B columns, and a
//    range of super-blocks.  Per super-block it stages the x slice in LDS
//    (shared by all its rows) and each wave stages its rows' packed blocks in
//    a wave-private LDS window with aligned, coalesced 16-byte loads; the
//    next super-block's loads are in flight during the current one's math.
//    When the row tiles are too few to fill the GPU the K range is split
//    across workgroups; each split writes its partial tile to the workspace
//    and bumps the tile's arrival counter, and the split that arrives last
//    adds all partials in split order into y in the same launch
//    (deterministic; no float atomics; see store_tile).
#include "jh_device.hpp"
#include "jh_kernels.hpp"

#include <mutex>
#include <stdlib.h>

namespace jh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// 2-byte-aligned views for Q6_K / Q8_0 fields (gfx950 global loads take any
// byte address; the compiler still emits single dwordx2 / dwordx4 loads)
typedef uint32_t u32x2a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef uint32_t u32x4a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32a2 __attribute__((aligned(2)));
constexpr int kPrefetch = 1;  // super-blocks of weight chunks in flight per wave (B <= 32)
constexpr int kMinWorkgroups = 256;  // split K until the grid has this many

// Timeline builds (-DJH_TIMELINE, juno_amd/timeline.py; never the shipped
// library): per wave of the B <= 32 double-buffered walk, s_memrealtime at entry
// and, per super-block step, after the step's barrier, once its weight chunks
// are parked, once the next x is staged, and after its MFMAs and fold; then in
// the epilogue (store_tile) once its partials are acknowledged, once the
// arrival is counted, and at its end.
#ifdef JH_TIMELINE
constexpr int kMtWg = 512, kMtSteps = 16, kMtEpi = 1 + 4 * kMtSteps, kMtPer = kMtEpi + 3;
__device__ unsigned long long g_mtimeline[kMtWg * 8 * kMtPer];
#define JH_MT(slot)                                                                                         \
    do {                                                                                                    \
        if ((threadIdx.x & 63) == 0 && blockIdx.x < kMtWg && (slot) < kMtPer)                               \
            g_mtimeline[((size_t)blockIdx.x * 8 + (threadIdx.x >> 6)) * kMtPer + (slot)] =                 \
                __builtin_amdgcn_s_memrealtime();                                                           \
    } while (0)
#else
#define JH_MT(slot) do {} while (0)
#endif

constexpr int kRowsPerWave = 32;
constexpr int kWaves = 8;  // waves per workgroup: 256 rows share each staged x slice
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWG = kWaves * kRowsPerWave;
constexpr int kXPad = 8;  // halves of padding per LDS column (spreads banks)

// Reductions over the 16 lanes of one DPP row (lanes 16 r .. 16 r + 15): xor-1
// and xor-2 butterflies, then the half-row and row mirrors.  Each step adds two
// values that are equal across the lanes being paired, so every lane ends with
// the bit-identical result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_f<0x4E>(v);   // quad_perm 2,3,0,1
    v += dpp_f<0x141>(v);  // row_half_mirror
    return v + dpp_f<0x140>(v);  // row_mirror
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}

// x into the LDS image of one column and super-block, inside the GEMM: 16
// consecutive lanes hold its 256 values, 16 each (xv).  A power-of-two scale
// puts max |x s| in [2^12, 2^13) (exact, undone on the partial sums), then x s
// is split into fp16 hi + lo limbs, and the 32-column sub-block sums (as hi and
// lo halves) and the super-block sum S are formed over 4-value groups with
// fixed butterflies (deterministic).
__device__ __forceinline__ void stage_x_column(const float (&xv)[16], int q, _Float16 *sh_hi, _Float16 *sh_lo,
                                               _Float16 *sh_xs, _Float16 *sh_x16, float2 *sh_S, int col, int colh) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) m = fmaxf(m, fabsf(xv[j]));
    m = row16_max(m);  // the 16 lanes of the column
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);
    const float s = m > 0.f ? ldexpf(1.f, 13 - e) : 1.f;
    float g[4];  // sums of the 4-value groups
#pragma unroll
    for (int k = 0; k < 4; k++) {
        _Float16 h4[4], l4[4];
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = xv[4 * k + j] * s;
            const _Float16 h = (_Float16)v;
            const _Float16 l = (_Float16)(v - (float)h);
            h4[j] = h;
            l4[j] = l;
            sum += (float)h + (float)l;
        }
        _Float16 *ph = sh_hi + col * colh + 16 * q + 4 * k, *pl = sh_lo + col * colh + 16 * q + 4 * k;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ph[j] = h4[j];
            pl[j] = l4[j];
        }
        g[k] = sum;
    }
    // 16-value group q (this lane's values): hi + lo in sh_x16 (the Q2_K min term)
    float sub = (g[0] + g[1]) + (g[2] + g[3]);
    {
        const _Float16 h = (_Float16)sub;
        sh_x16[col * 32 + q] = h;
        sh_x16[col * 32 + 16 + q] = (_Float16)(sub - (float)h);
    }
    // sub-block (32 values = groups 8i .. 8i+7 = this lane and its neighbour)
    sub += dpp_f<0xB1>(sub);
    if ((q & 1) == 0) {
        const _Float16 h = (_Float16)sub;
        sh_xs[col * 16 + (q >> 1)] = h;
        sh_xs[col * 16 + 8 + (q >> 1)] = (_Float16)(sub - (float)h);
    }
    // super-block total: the lane's 4 groups, then across the column's 16 lanes
    const float tot = row16_sum((g[0] + g[2]) + (g[1] + g[3]));
    if (q == 0) sh_S[col] = make_float2(tot, 1.f / s);
}

// ------------------------------------------------------------------ format policies
// Each format supplies, for one 256-column stretch ("super-block") of a row:
//   Regs              the lane's weight bytes (row lr, K half kh), in VGPRs
//   load(r, p, kh)    p = first byte of the row's stretch
//   Smem / publish    per-row fp32 scales, shared through LDS
//   compute<NT>(...)  the MFMAs and the fold into the fp32 totals
// K-step t covers 16 columns; lane half kh supplies 8 of them.  Every weight
// enters the MFMA as an exact fp16 integer; scales are applied in fp32.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int COLH = 256 + kXPad;  // halves per LDS column of the staged x slice

// x fragments of the padded image the fused kernel converts into LDS: column
// col at col * COLH halves (hi and lo), its sub-block sums at col * 16.
struct Ctx {
    int wave, lr, kh;
    const _Float16 *sh_hi, *sh_lo, *sh_xs, *sh_x16;
    const float2 *sh_S;
    // 16-column group sums of x, K-half kh: hi limbs, then lo limbs
    __device__ __forceinline__ half8 x16h(int col) const { return *reinterpret_cast<const half8 *>(sh_x16 + col * 32 + 8 * kh); }
    __device__ __forceinline__ half8 x16l(int col) const {
        return *reinterpret_cast<const half8 *>(sh_x16 + col * 32 + 16 + 8 * kh);
    }
    __device__ __forceinline__ half8 xh(int col, int xoff) const {
        return *reinterpret_cast<const half8 *>(sh_hi + col * COLH + xoff);
    }
    __device__ __forceinline__ half8 xl(int col, int xoff) const {
        return *reinterpret_cast<const half8 *>(sh_lo + col * COLH + xoff);
    }
    __device__ __forceinline__ half8 xm(int col) const { return *reinterpret_cast<const half8 *>(sh_xs + col * 16 + 8 * kh); }
    __device__ __forceinline__ const float2 *S() const { return sh_S; }
};

// ------------------------------------------------------------------ prepared x (B <= 32)
// One super-block of x for 32 batch columns, laid out exactly as the GEMM's
// LDS image so that it moves in as a contiguous DMA copy:
//   [hi: 32 columns x 32 units][lo: the same][sub-block sums: 32 x 16 halves]
//   [(S, 1 / scale): 32 x float2][pad to 34 x 1 KB]
// A unit is 16 bytes (8 consecutive values of one column).  Unit u of column
// col sits at slot col * 32 + (u ^ (col & 31)): the XOR swizzle lets the 32
// lanes that read unit u of 32 columns hit distinct LDS banks without padding.
constexpr int kSlabHi = 0, kSlabLo = 16384, kSlabXs = 32768, kSlabS = 33792;
constexpr int kSlabRows = 34;  // 1 KB DMA rows
constexpr int kSlabBytes = kSlabRows * 1024;

struct CtxP {
    int lr, kh;
    const uint8_t *x;  // the slab in LDS
    __device__ __forceinline__ static int slot(int col, int xoff) { return (col << 5) | ((xoff >> 3) ^ (col & 31)); }
    __device__ __forceinline__ half8 xh(int col, int xoff) const {
        return *reinterpret_cast<const half8 *>(x + kSlabHi + 16 * slot(col, xoff));
    }
    __device__ __forceinline__ half8 xl(int col, int xoff) const {
        return *reinterpret_cast<const half8 *>(x + kSlabLo + 16 * slot(col, xoff));
    }
    __device__ __forceinline__ half8 xm(int col) const {
        return *reinterpret_cast<const half8 *>(x + kSlabXs + 32 * col + 16 * kh);
    }
    __device__ __forceinline__ const float2 *S() const { return reinterpret_cast<const float2 *>(x + kSlabS); }
};

// Operand roles: x is the A operand (its 32 rows are batch columns) and the
// weights are B, so D[b][r] = sum_k x[b][k] w[r][k].  In the 32x32x16 layout
// lane (lr, kh) supplies weight row lr (K elements 8kh .. 8kh+7) and holds
// D for row lr and batch columns 8(i/4) + 4kh + (i%4), i < 16: every per-row
// scale (d, dmin, d*sc) lives in the lane's own registers, and consecutive
// lanes store consecutive rows.
__device__ __forceinline__ int batch_of(int n, int i, int kh) { return n * 32 + 8 * (i >> 2) + 4 * kh + (i & 3); }

// four byte pairs of two words -> fp16 1024 + u in 16-bit lanes: one byte
// permute per pair takes u from the word and the exponent byte 0x64 from a
// constant second source
__device__ __forceinline__ half8 bytes_to_h8(uint32_t w0, uint32_t w1, half2v off) {
    const uint32_t e = 0x64646464u;
    const uint32_t p[4] = {__builtin_amdgcn_perm(e, w0, 0x04010400u), __builtin_amdgcn_perm(e, w0, 0x04030402u),
                           __builtin_amdgcn_perm(e, w1, 0x04010400u), __builtin_amdgcn_perm(e, w1, 0x04030402u)};
    half8 a;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const half2v h = __builtin_bit_cast(half2v, p[j]) - off;  // exact: small integers
        a[2 * j] = h[0];
        a[2 * j + 1] = h[1];
    }
    return a;
}

// acc[n] += x_hi . w + x_lo . w over one K-step (x columns at xoff)
template <int NT, class C>
__device__ __forceinline__ void mfma_xw(const C &c, const half8 &w, int xoff, f32x16 *acc) {
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int col = n * 32 + c.lr;
        const half8 xh = c.xh(col, xoff);
        const half8 xl = c.xl(col, xoff);
        acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, w, acc[n], 0, 0, 0);
        acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, w, acc[n], 0, 0, 0);
    }
}

// (S, 1/scale) of the 16 batch columns a lane holds for tile n
template <int NT, class C>
__device__ __forceinline__ void col_terms(const C &c, int n, float (&S)[16], float (&cs)[16]) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 v = *reinterpret_cast<const float4 *>(c.S() + n * 32 + 8 * q + 4 * c.kh + 2 * h);
            S[4 * q + 2 * h] = v.x;
            cs[4 * q + 2 * h] = v.y;
            S[4 * q + 2 * h + 1] = v.z;
            cs[4 * q + 2 * h + 1] = v.w;
        }
}

// N dwords at a 2-byte-aligned LDS address, read as aligned dwords and
// realigned in registers with v_alignbyte.  Unaligned 8- and 16-byte LDS reads
// stall the LDS pipeline (and the x-fragment reads queued behind them).  One
// dword past the field is read and ignored when p is dword-aligned, so the
// weight windows end with kWinPad bytes of padding.
constexpr int kWinPad = 16;
template <int N>
__device__ __forceinline__ void lds_read_u(const uint8_t *p, uint32_t (&out)[N]) {
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);
    const uint32_t *b = reinterpret_cast<const uint32_t *>(p - sh);
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i <= N; i++) w[i] = b[i];
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}
__device__ __forceinline__ u32x2 lds_u32x2(const uint8_t *p) {
    uint32_t v[2];
    lds_read_u<2>(p, v);
    return u32x2{v[0], v[1]};
}
__device__ __forceinline__ u32x4 lds_u32x4(const uint8_t *p) {
    uint32_t v[4];
    lds_read_u<4>(p, v);
    return u32x4{v[0], v[1], v[2], v[3]};
}

// Window position (in chunks) of chunk j of a wave's 32 x CH chunk grid when
// rows are RC >= CH chunks apart.
template <int CH, int RC>
__device__ __forceinline__ int win_chunk(int j) { return RC == CH ? j : j + (RC - CH) * (j / CH); }

// Q4_K (matVecQ4Kraw, LlamaTransformerHandler.java:1428-1468): w = d*ls*q - dmin*lm.
// B = ls*q (<= 945, exact), built as fp16 1024 + ls*q by one 24-bit multiply-
// add per pair into the exponent byte and one packed fp16 subtraction of 1024
// (exact); the min term (one more MFMA: A = [sub-block sums hi | lo], B =
// [lm | lm]) is removed per super-block with d and dmin.  Keeping the 1024 in
// B and subtracting 1024 * sum(x) afterwards would cost fp32 cancellation
// wherever |x| is large and the row's weights there are small.
// Q5_K (Q5 = true, matVecQ5Kraw :1525-1576): q has a 5th bit from qh, so
// ls*q reaches 1953 and 1024 + ls*q would pass fp16's exact integers; B =
// ls*q is converted instead (v_cvt_f16_u16, exact below 2048).
template <bool Q5>
struct FmtKQ {
    static constexpr int kBytes = Q5 ? 176 : 144;
    static constexpr int kChunks = kBytes / 16;  // rows are 16-byte aligned (pitch kBytes * n, aligned base)
    static constexpr int kRowChunks = kChunks;   // LDS window row stride (16-byte chunks)
    static constexpr int kQs = Q5 ? 48 : 16;
    static constexpr bool kSums = true;
    struct Regs {
        u32x4 hd;
        u32x2 qp[4][2];
        u32x2 qh[2];  // Q5_K: qh bytes 16 j + 8 kh .. +8 (bit s for sub-block s)
    };
    template <bool RA>  // rows are 16-byte aligned: the reads are aligned either way
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
        r.hd = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            r.qp[g][0] = *reinterpret_cast<const u32x2 *>(p + kQs + 32 * g + 8 * kh);
            r.qp[g][1] = *reinterpret_cast<const u32x2 *>(p + kQs + 32 * g + 16 + 8 * kh);
        }
        if (Q5) {
            r.qh[0] = *reinterpret_cast<const u32x2 *>(p + 16 + 8 * kh);
            r.qh[1] = *reinterpret_cast<const u32x2 *>(p + 32 + 8 * kh);
        }
    }
    template <int NT, class C>
    static __device__ __forceinline__ void compute(const Regs &r, const C &c, f32x16 *tot) {
        // 6-bit scales and mins of the 8 sub-blocks (q4kScaleRaw / q4kMinRaw, :1471-1482)
        int ls[8], lm[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ls[j] = (int)byte_of(r.hd.y, j) & 63;
            lm[j] = (int)byte_of(r.hd.z, j) & 63;
            ls[j + 4] = (int)((byte_of(r.hd.w, j) & 0x0F) | ((byte_of(r.hd.y, j) & 0xC0) >> 2));
            lm[j + 4] = (int)((byte_of(r.hd.w, j) >> 4) | ((byte_of(r.hd.z, j) & 0xC0) >> 2));
        }
        const half2v k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        f32x16 acc[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) acc[n] = (f32x16){};
#pragma unroll
        for (int t = 0; t < 16; t++) {
            // sub-block s = t/2: low nibbles of qs group s/2 for even s, high for odd
            const int s = t >> 1, g = s >> 1, hiN = s & 1;
            const u32x2 q = r.qp[g][t & 1];
            uint32_t nib0 = hiN ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
            uint32_t nib1 = hiN ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
            if (Q5) {
                const u32x2 h = r.qh[t & 1];
                nib0 |= ((h.x >> s) & 0x01010101u) << 4;
                nib1 |= ((h.y >> s) & 0x01010101u) << 4;
            }
            const uint32_t pr[4] = {__builtin_amdgcn_perm(0u, nib0, 0x0C010C00u),
                                    __builtin_amdgcn_perm(0u, nib0, 0x0C030C02u),
                                    __builtin_amdgcn_perm(0u, nib1, 0x0C010C00u),
                                    __builtin_amdgcn_perm(0u, nib1, 0x0C030C02u)};
            half8 w;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (Q5) {
                    const uint32_t v = __umul24(pr[j], (uint32_t)ls[s]);  // two 16-bit products <= 1953
                    w[2 * j] = (_Float16)(uint16_t)(v & 0xFFFF);
                    w[2 * j + 1] = (_Float16)(uint16_t)(v >> 16);
                } else {
                    // 1024 + ls*q by the exponent byte, then 1024 off in fp16: exact, and
                    // the MFMA sums stay the size of the weights' own products
                    const uint32_t v = __umul24(pr[j], (uint32_t)ls[s]) + 0x64006400u;
                    const half2v h = __builtin_bit_cast(half2v, v) - k1024;
                    w[2 * j] = h[0];
                    w[2 * j + 1] = h[1];
                }
            }
            mfma_xw<NT>(c, w, 16 * t + 8 * c.kh, acc);
        }
        half8 wm;
#pragma unroll
        for (int j = 0; j < 8; j++) wm[j] = (_Float16)lm[j];
        const float d = half_bits_to_float(r.hd.x), dmin = half_bits_to_float(r.hd.x >> 16);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int col = n * 32 + c.lr;
            const half8 xm = c.xm(col);
            const f32x16 mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(xm, wm, (f32x16){}, 0, 0, 0);
            float S[16], cs[16];
            col_terms<NT>(c, n, S, cs);
#pragma unroll
            for (int i = 0; i < 16; i++) tot[n][i] = fmaf(cs[i], fmaf(d, acc[n][i], -dmin * mn[i]), tot[n][i]);
        }
    }
};

using FmtQ4K = FmtKQ<false>;
using FmtQ5K = FmtKQ<true>;

// Q6_K (matVecQ6Kraw, LlamaTransformerHandler.java:1587-1638): w = (d*sc_j)*(u - 32)
// with u = 4 bits of ql | 2 bits of qh.  A 16-column sub-block is exactly one
// K-step, so B = u - 32 (exact) and each K-step is folded with the fp32
// d*sc_j of the lane's row (the reference's dN).  Step t = 8n + 2qd + j
// covers columns 128n + 32qd + 16j .. +16 and uses scale t.
struct FmtQ6K {
    static constexpr int kBytes = 210;
    static constexpr int kChunks = (kBytes + 14 + 15) / 16;  // a 2-byte-aligned block spans <= 14 chunks
    // window rows 15 chunks (60 dwords) apart: the dword reads of 32 rows hit 16
    // banks (2-way) instead of the 8 of a 56-dword stride
    static constexpr int kRowChunks = kChunks + 1;
    static constexpr bool kSums = false;
    struct Regs {
        u32x2 ql[2][2][2];  // [half n][ql +32 p][j]: bytes 64n + 32p + 16j + 8kh
        u32x2 qh[2][2];     // [n][j]: bytes 128 + 32n + 16j + 8kh
        u32x4 sc;           // bytes 192..207
        uint32_t dw;        // bytes 206..209: d in the high half
    };
    template <bool RA>  // realign in registers (aligned LDS reads) or read the 2-byte-aligned fields directly
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint8_t *a = p + 64 * n + 16 * j + 8 * kh, *h = p + 128 + 32 * n + 16 * j + 8 * kh;
                r.ql[n][0][j] = RA ? lds_u32x2(a) : *reinterpret_cast<const u32x2a2 *>(a);
                r.ql[n][1][j] = RA ? lds_u32x2(a + 32) : *reinterpret_cast<const u32x2a2 *>(a + 32);
                r.qh[n][j] = RA ? lds_u32x2(h) : *reinterpret_cast<const u32x2a2 *>(h);
            }
        if (RA) {
            r.sc = lds_u32x4(p + 192);
            uint32_t dw[1];
            lds_read_u<1>(p + 206, dw);
            r.dw = dw[0];
        } else {
            r.sc = *reinterpret_cast<const u32x4a2 *>(p + 192);
            r.dw = *reinterpret_cast<const u32a2 *>(p + 206);
        }
    }
    template <int NT, class C>
    static __device__ __forceinline__ void compute(const Regs &r, const C &c, f32x16 *tot) {
        const half2v off = {(_Float16)1056.f, (_Float16)1056.f};  // 1024 + 32
        const float d = half_bits_to_float(r.dw >> 16);
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int n = t >> 3, qd = (t >> 1) & 3, j = t & 1;
            const u32x2 l = r.ql[n][qd & 1][j], h = r.qh[n][j];
            const uint32_t u0 = ((qd >= 2 ? l.x >> 4 : l.x) & 0x0F0F0F0Fu) | (((h.x >> (2 * qd)) & 0x03030303u) << 4);
            const uint32_t u1 = ((qd >= 2 ? l.y >> 4 : l.y) & 0x0F0F0F0Fu) | (((h.y >> (2 * qd)) & 0x03030303u) << 4);
            f32x16 acc[NT];
#pragma unroll
            for (int m = 0; m < NT; m++) acc[m] = (f32x16){};
            mfma_xw<NT>(c, bytes_to_h8(u0, u1, off), 16 * t + 8 * c.kh, acc);
            const float ds = d * (float)(int8_t)byte_of(t < 4 ? r.sc.x : t < 8 ? r.sc.y : t < 12 ? r.sc.z : r.sc.w, t & 3);
#pragma unroll
            for (int m = 0; m < NT; m++)
#pragma unroll
                for (int i = 0; i < 16; i++) tot[m][i] = fmaf(ds, acc[m][i], tot[m][i]);
        }
    }
};

// Q8_0 (matVecQ8_0raw, LlamaTransformerHandler.java:1486-1508): w = d_b * q, 8 blocks
// of 34 B per 256 columns.  Lane half kh holds columns 16kh .. 16kh+15 of
// block b (one 16-byte load), split over the block's two K-steps; B = q exact.
struct FmtQ8_0 {
    static constexpr int kBytes = 8 * 34;
    static constexpr int kChunks = (kBytes + 14 + 15) / 16;
    static constexpr int kRowChunks = kChunks + 1;  // 76-dword window rows (see FmtQ6K)
    static constexpr bool kSums = false;
    struct Regs {
        u32x4 q[8];     // block b: bytes 34b + 2 + 16kh .. +16
        uint32_t d[8];  // d of block b (low half)
    };
    template <bool RA>
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const uint8_t *a = p + 34 * b + 2 + 16 * kh;
            r.q[b] = RA ? lds_u32x4(a) : *reinterpret_cast<const u32x4a2 *>(a);
            r.d[b] = *reinterpret_cast<const uint16_t *>(p + 34 * b);
        }
    }
    template <int NT, class C>
    static __device__ __forceinline__ void compute(const Regs &r, const C &c, f32x16 *tot) {
        const half2v off = {(_Float16)1152.f, (_Float16)1152.f};  // 1024 + 128
#pragma unroll
        for (int b = 0; b < 8; b++) {
            f32x16 acc[NT];
#pragma unroll
            for (int m = 0; m < NT; m++) acc[m] = (f32x16){};
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t w0 = (j ? r.q[b].z : r.q[b].x) ^ 0x80808080u;  // q + 128
                const uint32_t w1 = (j ? r.q[b].w : r.q[b].y) ^ 0x80808080u;
                mfma_xw<NT>(c, bytes_to_h8(w0, w1, off), 32 * b + 16 * c.kh + 8 * j, acc);
            }
            const float d = half_bits_to_float(r.d[b]);
#pragma unroll
            for (int m = 0; m < NT; m++)
#pragma unroll
                for (int i = 0; i < 16; i++) tot[m][i] = fmaf(d, acc[m][i], tot[m][i]);
        }
    }
};

// Q2_K (matVecQ2Kraw, LlamaTransformerHandler.java): 84-byte blocks [scales 16]
// [qs 64][d][dmin]; element 128h + 16k + l takes 2 bits at shift 2(k/2) of
// qs[32h + 16(k&1) + l] and sub-block scale byte sc[8h + k] (low nibble scale,
// high nibble min): w = d*(sc&15)*q - dmin*(sc>>4).  A 16-column sub-block is one
// K-step t = 8h + k: B = q (exact), folded per K-step with d*(sc&15); the min
// term is one MFMA pair per super-block against the 16-column sums of x.
// Blocks are 4-byte aligned (84 = 4 * 21).
struct FmtQ2K {
    static constexpr int kBytes = 84;
    static constexpr int kChunks = (kBytes + 12 + 15) / 16;  // a 4-byte-aligned block spans <= 6 chunks
    static constexpr int kRowChunks = kChunks + 1;           // 28-dword window rows (2-way bank conflicts)
    static constexpr bool kSums = false;
    struct Regs {
        u32x2 q[2][2];  // [h][k&1]: qs bytes 32h + 16(k&1) + 8kh .. +8
        u32x4 sc;       // the 16 scale bytes
        uint32_t dm;    // d (low half), dmin (high half)
    };
    template <bool RA>
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int o = 0; o < 2; o++) r.q[h][o] = lds_u32x2(p + 16 + 32 * h + 16 * o + 8 * kh);
        r.sc = lds_u32x4(p);
        uint32_t dm[1];
        lds_read_u<1>(p + 80, dm);
        r.dm = dm[0];
    }
    template <int NT, class C>
    static __device__ __forceinline__ void compute(const Regs &r, const C &c, f32x16 *tot) {
        const half2v off = {(_Float16)1024.f, (_Float16)1024.f};
        const float d = half_bits_to_float(r.dm), dmin = half_bits_to_float(r.dm >> 16);
        auto scb = [&](int t) { return byte_of(t < 4 ? r.sc.x : t < 8 ? r.sc.y : t < 12 ? r.sc.z : r.sc.w, t & 3); };
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int h = t >> 3, k = t & 7;
            const u32x2 q = r.q[h][k & 1];
            const uint32_t u0 = (q.x >> (2 * (k >> 1))) & 0x03030303u, u1 = (q.y >> (2 * (k >> 1))) & 0x03030303u;
            f32x16 acc[NT];
#pragma unroll
            for (int m = 0; m < NT; m++) acc[m] = (f32x16){};
            mfma_xw<NT>(c, bytes_to_h8(u0, u1, off), 16 * t + 8 * c.kh, acc);
            const float ds = d * (float)(scb(t) & 15u);
#pragma unroll
            for (int m = 0; m < NT; m++)
#pragma unroll
                for (int i = 0; i < 16; i++) tot[m][i] = fmaf(ds, acc[m][i], tot[m][i]);
        }
        // min term: sum_t (sc_t >> 4) * X16_t, K-half kh holding t = 8kh .. 8kh+7
        half8 wm;
#pragma unroll
        for (int j = 0; j < 8; j++) wm[j] = (_Float16)(float)(scb(8 * c.kh + j) >> 4);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int col = n * 32 + c.lr;
            f32x16 mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(c.x16h(col), wm, (f32x16){}, 0, 0, 0);
            mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(c.x16l(col), wm, mn, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) tot[n][i] = fmaf(-dmin, mn[i], tot[n][i]);
        }
    }
};

// Q3_K (matVecQ3Kraw, LlamaTransformerHandler.java): 110-byte blocks [hmask 32]
// [qs 64][scales 12][d]; sub-block t = 8h + 2j + r covers columns 128h + 32j +
// 16r + l, whose 3-bit quant is 2 bits at shift 2j of qs[32h + 16r + l] and bit
// 4h + j of hmask[16r + l], minus 4, with the 6-bit scale of t minus 32:
// w = d*(sc - 32)*(q - 4).  B = q - 4 (exact), folded per K-step.  Blocks are
// 2-byte aligned: fields are read as aligned dwords and realigned.
struct FmtQ3K {
    static constexpr int kBytes = 110;
    static constexpr int kChunks = (kBytes + 14 + 15) / 16;  // a 2-byte-aligned block spans <= 8 chunks
    static constexpr int kRowChunks = kChunks + 1;           // 36-dword window rows (2-way bank conflicts)
    static constexpr bool kSums = false;
    struct Regs {
        u32x2 q[2][2];  // [h][r]: qs bytes 32 + 32h + 16r + 8kh .. +8
        u32x2 hm[2];    // [r]: hmask bytes 16r + 8kh .. +8
        u32x4 sd;       // scale bytes 96..107 (aux0, aux1, aux2), then d in the low half of .w
    };
    template <bool RA>
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int o = 0; o < 2; o++) r.q[h][o] = lds_u32x2(p + 32 + 32 * h + 16 * o + 8 * kh);
#pragma unroll
        for (int o = 0; o < 2; o++) r.hm[o] = lds_u32x2(p + 16 * o + 8 * kh);
        r.sd = lds_u32x4(p + 96);
    }
    template <int NT, class C>
    static __device__ __forceinline__ void compute(const Regs &r, const C &c, f32x16 *tot) {
        const half2v off = {(_Float16)1028.f, (_Float16)1028.f};  // 1024 + 4
        const float d = half_bits_to_float(r.sd.w);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            // the scale words of this half (utmp[2h], utmp[2h+1] of dequantizeQ3K)
            const uint32_t aux2 = r.sd.z;
            const uint32_t ua = ((r.sd.x >> (4 * h)) & 0x0f0f0f0fu) | (((aux2 >> (4 * h)) & 0x03030303u) << 4);
            const uint32_t ub = ((r.sd.y >> (4 * h)) & 0x0f0f0f0fu) | (((aux2 >> (4 * h + 2)) & 0x03030303u) << 4);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int rr = 0; rr < 2; rr++) {
                    const int t = 8 * h + 2 * j + rr;
                    const u32x2 q = r.q[h][rr], hm = r.hm[rr];
                    const int hb = 4 * h + j;
                    const uint32_t u0 = ((q.x >> (2 * j)) & 0x03030303u) | (((hm.x >> hb) & 0x01010101u) << 2);
                    const uint32_t u1 = ((q.y >> (2 * j)) & 0x03030303u) | (((hm.y >> hb) & 0x01010101u) << 2);
                    f32x16 acc[NT];
#pragma unroll
                    for (int m = 0; m < NT; m++) acc[m] = (f32x16){};
                    mfma_xw<NT>(c, bytes_to_h8(u0, u1, off), 16 * t + 8 * c.kh, acc);
                    const int s6 = (int)byte_of(j < 2 ? ua : ub, 2 * (j & 1) + rr) - 32;
                    const float ds = d * (float)s6;
#pragma unroll
                    for (int m = 0; m < NT; m++)
#pragma unroll
                        for (int i = 0; i < 16; i++) tot[m][i] = fmaf(ds, acc[m][i], tot[m][i]);
                }
        }
    }
};

// ------------------------------------------------------------------ tile output
// A workgroup's tile goes straight into y when K is not split.  Otherwise
// each split stores its partial tile with coherent (L2-bypassing) stores and
// bumps the tile's counter; the split that arrives last adds all partials in
// split order into y -- a fixed order, whatever the arrival order, so the
// result is deterministic -- and re-arms the counter for the next launch.
// Coherent stores plus a wait for their completion before the counter
// increment avoid a device-scope release, which on a multi-XCD part writes
// back the whole L2 (~100 us per workgroup measured); a separate reduction
// launch costs ~5 us.
constexpr int kMaxTileCounters = kCounterSlots;

template <int NT>
__device__ __forceinline__ void store_tile(const f32x16 (&tot)[NT], int r, int nrows, int kh, int B, float *__restrict__ Y,
                                           float *part, int *counters, int tile, int split, int ksplit) {
    const bool live = r < nrows;
    if (ksplit == 1) {
        if (!live) return;
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int b = batch_of(n, i, kh);
                if (b < B) Y[(size_t)b * nrows + r] = tot[n][i];
            }
        return;
    }
    const size_t plane = (size_t)B * nrows;
    if (live) {
        float *mine = part + split * plane;
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int b = batch_of(n, i, kh);
                if (b < B) __hip_atomic_store(mine + (size_t)b * nrows + r, tot[n][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    // Ordering of the hand-off.  The partials are agent-scope atomic stores, which
    // gfx950 performs at the memory-side coherence point (past the per-XCD L2s);
    // s_waitcnt(0) returns only once each of this wave's stores is acknowledged
    // there, and the barrier makes every wave's acknowledgement precede the
    // counter's fetch_add, itself performed at that point.  The last arriver then
    // reads the partials with agent-scope atomic loads, which are served from the
    // same point.  A release / acquire pair on the counter would order them
    // formally, but an agent-scope release writes back the whole L2 of the XCD
    // (buffer_wbl2), which measured ~100 us per GEMV; there are no non-atomic
    // stores for it to publish.
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partials have reached the coherence point
    JH_MT(kMtEpi);
    __shared__ int s_last;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counters + tile * kCounterStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == ksplit - 1;
        if (last) __hip_atomic_store(counters + tile * kCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    JH_MT(kMtEpi + 1);
    if (!s_last || !live) return;
    // KB splits' partials in flight at a time, added in split order
    constexpr int KB = 4 / NT;
    const int ks = ksplit;
    float acc[NT][16];
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[n][i] = 0.f;
    for (int k0 = 0; k0 < ks; k0 += KB) {
        float v[KB][NT][16];
#pragma unroll
        for (int kk = 0; kk < KB; kk++) {
            const int k = k0 + kk;
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    // unconditional (clamped) loads, so that they issue back to back;
                    // this split's own partial comes back from memory unchanged
                    const int b = min(batch_of(n, i, kh), B - 1);
                    v[kk][n][i] = __hip_atomic_load(part + min(k, ks - 1) * plane + (size_t)b * nrows + r,
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
        }
#pragma unroll
        for (int kk = 0; kk < KB; kk++)
            if (k0 + kk < ks)
#pragma unroll
                for (int n = 0; n < NT; n++)
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[n][i] += v[kk][n][i];
    }
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int b = batch_of(n, i, kh);
            if (b < B) Y[(size_t)b * nrows + r] = acc[n][i];
        }
    JH_MT(kMtEpi + 2);
}

// ------------------------------------------------------------------ batched kernel
// One matrix of a grouped launch: the workgroups [wg0, wg0 + tiles * ksplit)
// are its row tiles x K splits (split fastest); its partial planes start at
// part0 floats into the group's partial buffer and its tile counters at cnt0.
struct MfmaProblem {
    const uint8_t *w;
    const float *x;
    float *y;
    size_t pitch, part0;
    int type, row0, rows, tiles, wg0, cnt0;
};
struct MfmaGroup {
    MfmaProblem p[kMaxMfmaGroup];
    float *part;
    int *counters;
    int n, nsb, ksb, ksplit, B;
    // SwiGLU pairs (mfma_group<.., true>): p[0] is gate, w2 the up matrix of the
    // same shape; a workgroup's waves 0-3 take 128 gate rows and waves 4-7 the
    // same up rows, and swiglu[b][r] = silu(gate) * up replaces both outputs
    const uint8_t *w2;
    float *swiglu;
};

// format mask bits: Q4_K, Q5_K, Q6_K, Q8_0, Q2_K, Q3_K
template <int MASK>
__host__ __device__ constexpr int max_chunks() {
    int c = 0;
    if (MASK & 1) c = c > FmtQ4K::kRowChunks ? c : FmtQ4K::kRowChunks;
    if (MASK & 2) c = c > FmtQ5K::kRowChunks ? c : FmtQ5K::kRowChunks;
    if (MASK & 4) c = c > FmtQ6K::kRowChunks ? c : FmtQ6K::kRowChunks;
    if (MASK & 8) c = c > FmtQ8_0::kRowChunks ? c : FmtQ8_0::kRowChunks;
    if (MASK & 16) c = c > FmtQ2K::kRowChunks ? c : FmtQ2K::kRowChunks;
    if (MASK & 32) c = c > FmtQ3K::kRowChunks ? c : FmtQ3K::kRowChunks;
    return c;
}
// LDS image: [x hi: BP x COLH][x lo: BP x COLH][32-column sums: BP x 16 halves][16-column sums: BP x 32 halves]
// [(S, 1/s): BP][weight windows]
template <int NT>
__host__ __device__ constexpr int lds_w_offset() { return (2 * 32 * NT * COLH + 32 * NT * 16 + 32 * NT * 32) * 2 + 32 * NT * 8; }
template <int NT, int MASK>
__host__ __device__ constexpr int lds_bytes() {
    return (NT == 1 ? 2 : 1) * lds_w_offset<NT>() + kWaves * kRowsPerWave * max_chunks<MASK>() * 16 + kWinPad;
}

// store_tile for a SwiGLU pair workgroup (B <= 32): split partials over virtual
// rows (gate r, up rows + r) in planes of B x 2 rows, the usual hand-off, then
// the up waves pass their totals to the gate waves through LDS and those store
// silu(gate) * up.  r is the lane's row within its matrix, lw its row within
// the workgroup's 128.
__device__ __forceinline__ void store_pair(const f32x16 (&tot)[1], int r, int lw, bool up, int nrows, int kh, int B,
                                           float *__restrict__ out, float *part, int *counters, int tile, int split,
                                           int ksplit, uint8_t *lds) {
    const bool live = r < nrows;
    const int vr = r + (up ? nrows : 0);
    float fin[16];
#pragma unroll
    for (int i = 0; i < 16; i++) fin[i] = tot[0][i];
    if (ksplit > 1) {
        const size_t plane = (size_t)B * 2 * nrows;
        if (live) {
            float *mine = part + split * plane;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int b = batch_of(0, i, kh);
                if (b < B) __hip_atomic_store(mine + (size_t)b * 2 * nrows + vr, tot[0][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the same hand-off ordering as store_tile
        __shared__ int s_last;
        __syncthreads();
        if (threadIdx.x == 0) {
            const int old = __hip_atomic_fetch_add(counters + tile * kCounterStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = old == ksplit - 1;
            if (last) __hip_atomic_store(counters + tile * kCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;  // uniform across the workgroup
        constexpr int KB = 4;
        float acc[16];
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = 0.f;
        const int rr = min(vr, 2 * nrows - 1);
        for (int k0 = 0; k0 < ksplit; k0 += KB) {
            float v[KB][16];
#pragma unroll
            for (int kk = 0; kk < KB; kk++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int b = min(batch_of(0, i, kh), B - 1);
                    v[kk][i] = __hip_atomic_load(part + min(k0 + kk, ksplit - 1) * plane + (size_t)b * 2 * nrows + rr,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
            for (int kk = 0; kk < KB; kk++)
                if (k0 + kk < ksplit)
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[i] += v[kk][i];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) fin[i] = acc[i];
    }
    float *xl = reinterpret_cast<float *>(lds);  // [128 rows][33]: the up totals
    __syncthreads();  // every wave is done with the x buffers
    if (up)
#pragma unroll
        for (int i = 0; i < 16; i++) xl[lw * 33 + batch_of(0, i, kh)] = fin[i];
    __syncthreads();
    if (!up && live)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int b = batch_of(0, i, kh);
            if (b < B) out[(size_t)b * nrows + r] = silu_times(fin[i], xl[lw * 33 + b]);
        }
}

// One workgroup's tile (32 rows per wave x all batch columns) over the K
// range of its split, x converted into LDS super-block by super-block.
template <class F, int NT, int PD, bool PAIR>  // NT = padded batch / 32, PD = weight prefetch depth (super-blocks)
__device__ __forceinline__ void gemm_body(const MfmaProblem &P, int tile, int split, const MfmaGroup &g, uint8_t *lds) {
    constexpr int BP = 32 * NT;
    constexpr int CPT = BP / 32;  // x columns converted per thread (16 lanes per column and super-block)
    constexpr int CH = F::kChunks;          // 16-byte chunks staged per row and super-block
    constexpr int CL = (kRowsPerWave * CH + 63) / 64;  // chunks per lane
    _Float16 *sh_hi = reinterpret_cast<_Float16 *>(lds);
    _Float16 *sh_lo = sh_hi + BP * COLH;
    _Float16 *sh_xs = sh_lo + BP * COLH;
    _Float16 *sh_x16 = sh_xs + BP * 16;
    float2 *sh_S = reinterpret_cast<float2 *>(sh_x16 + BP * 32);  // (sum of x, 1 / column scale) per column
    const bool up_half = PAIR && (threadIdx.x >> 6) >= kWaves / 2;  // SwiGLU pairs: waves 4-7 take the up rows
    const uint8_t *__restrict__ W = up_half ? g.w2 : P.w;
    const float *__restrict__ X = P.x;
    const size_t pitch = P.pitch;
    const int nrows = P.rows, row0 = P.row0, B = g.B, cols = 256 * g.nsb;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const Ctx c{wave, lane & 31, lane >> 5, sh_hi, sh_lo, sh_xs, sh_x16, sh_S};
    const int rbase = PAIR ? tile * (kRowsPerWG / 2) + (wave & (kWaves / 2 - 1)) * kRowsPerWave
                           : tile * kRowsPerWG + wave * kRowsPerWave;
    const int sb0 = split * g.ksb, sb1 = min(g.nsb, sb0 + g.ksb);
    auto row_off = [&](int rho) { return (size_t)(row0 + min(rbase + rho, nrows - 1)) * pitch; };
    // Weight staging: chunk j = lane + 64 k of the wave's 32 x CH chunk grid is
    // row j / CH, 16-byte piece j % CH of that row's aligned window.  Whole
    // aligned 16-byte lanes, consecutive within a row: few cache accesses per
    // load, instead of 8-byte gathers from 32 rows at 2-byte alignment.
    size_t coff[CL];
#pragma unroll
    for (int k = 0; k < CL; k++) {
        const int j = min(lane + 64 * k, kRowsPerWave * CH - 1);
        coff[k] = row_off(j / CH) + 16 * (j % CH);
    }
    const size_t myoff = row_off(c.lr);
    constexpr int RC = NT == 1 ? F::kRowChunks : CH;  // window row stride (chunks): padded for the realigned reads
    uint8_t *wslot = lds + lds_w_offset<NT>() + wave * (kRowsPerWave * RC * 16);

    u32x4 ch_n[PD][CL];
    float xv_n[CPT][16];  // the next super-block's raw x: column (threadIdx.x >> 4) + 32 i, values 16 q .. +16
    const int xq = threadIdx.x & 15, xcol = threadIdx.x >> 4;
    // (a macro rather than a lambda: the register arrays must stay in VGPRs)
#define JH_LOAD_W(ST, SB)                                                                                  \
    do {                                                                                                   \
        const size_t sbo = (size_t)(SB) * F::kBytes;                                                       \
        _Pragma("unroll") for (int k = 0; k < CL; k++)                                                     \
            ch_n[ST][k] = *reinterpret_cast<const u32x4 *>(W + ((coff[k] + sbo) & ~size_t(15)));           \
    } while (0)
#define JH_LOAD_X(SB)                                                                                      \
    do {                                                                                                   \
        _Pragma("unroll") for (int i = 0; i < CPT; i++) {                                                  \
            const int b = xcol + 32 * i;                                                                   \
            const float4 *xp = reinterpret_cast<const float4 *>(X + (size_t)min(b, B - 1) * cols +        \
                                                                (SB) * 256 + 16 * xq);                     \
            _Pragma("unroll") for (int k = 0; k < 4; k++) {                                                \
                const float4 v = b < B ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);                         \
                xv_n[i][4 * k] = v.x; xv_n[i][4 * k + 1] = v.y; xv_n[i][4 * k + 2] = v.z; xv_n[i][4 * k + 3] = v.w; \
            }                                                                                              \
        }                                                                                                  \
    } while (0)

    f32x16 tot[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) tot[n] = (f32x16){};

    auto fold = [&](const typename F::Regs &w, const Ctx &cx) {
        if constexpr (F::kSums) {
            F::template compute<NT>(w, cx, tot);
        } else {
            f32x16 part[NT];
#pragma unroll
            for (int n = 0; n < NT; n++) part[n] = (f32x16){};
            F::template compute<NT>(w, cx, part);
#pragma unroll
            for (int n = 0; n < NT; n++) {
                float S[16], cs[16];
                col_terms<NT>(cx, n, S, cs);
#pragma unroll
                for (int i = 0; i < 16; i++) tot[n][i] = fmaf(cs[i], part[n][i], tot[n][i]);
            }
        }
    };

    if constexpr (NT == 1 && PD == 1) {
        // Two x buffers: super-block sb + 1's x is converted into the free
        // buffer while sb's MFMAs run, with one barrier per super-block.  The
        // buffer a step writes was last read by the previous step's MFMAs,
        // which every wave finished before this step's barrier.
        constexpr int XS = lds_w_offset<1>();  // bytes of one x buffer
        auto ctx_at = [&](int buf) {
            _Float16 *hi = reinterpret_cast<_Float16 *>(lds + buf * XS);
            _Float16 *lo = hi + BP * COLH, *xs = lo + BP * COLH, *x16 = xs + BP * 16;
            return Ctx{wave, lane & 31, lane >> 5, hi, lo, xs, x16, reinterpret_cast<float2 *>(x16 + BP * 32)};
        };
        auto stage_into = [&](int buf) {
            const Ctx cx = ctx_at(buf);
            stage_x_column(xv_n[0], xq, const_cast<_Float16 *>(cx.sh_hi), const_cast<_Float16 *>(cx.sh_lo),
                           const_cast<_Float16 *>(cx.sh_xs), const_cast<_Float16 *>(cx.sh_x16),
                           const_cast<float2 *>(cx.sh_S), xcol, COLH);
        };
        uint8_t *wslot2 = lds + 2 * XS + wave * (kRowsPerWave * RC * 16);
        JH_MT(0);
        if (sb0 < sb1) {
            JH_LOAD_X(sb0);
            JH_LOAD_W(0, sb0);
            stage_into(0);
            if (sb0 + 1 < sb1) JH_LOAD_X(sb0 + 1);
        }
        for (int sb = sb0; sb < sb1; sb++) {
            const int buf = (sb - sb0) & 1;
            __syncthreads();  // x of sb is staged; the other buffer is free
            JH_MT(1 + 4 * (sb - sb0));
#pragma unroll
            for (int k = 0; k < CL; k++)
                if (lane + 64 * k < kRowsPerWave * CH) *reinterpret_cast<u32x4 *>(wslot2 + 16 * win_chunk<CH, RC>(lane + 64 * k)) = ch_n[0][k];
            JH_MT(2 + 4 * (sb - sb0));
            typename F::Regs w;
            F::template load<true>(w, wslot2 + c.lr * RC * 16 + ((myoff + (size_t)sb * F::kBytes) & 15), c.kh);
            if (sb + 1 < sb1) {
                stage_into(buf ^ 1);
                if (sb + 2 < sb1) JH_LOAD_X(sb + 2);
                JH_LOAD_W(0, sb + 1);
            }
            JH_MT(3 + 4 * (sb - sb0));
            fold(w, ctx_at(buf));
            JH_MT(4 + 4 * (sb - sb0));
        }
    } else {
    if (sb0 < sb1) JH_LOAD_X(sb0);
#pragma unroll
    for (int st = 0; st < PD; st++)
        if (sb0 + st < sb1) JH_LOAD_W(st, sb0 + st);
    for (int sb = sb0; sb < sb1; sb++) {
        __syncthreads();  // the previous super-block's LDS contents are consumed
#pragma unroll
        for (int i = 0; i < CPT; i++)
            stage_x_column(xv_n[i], xq, sh_hi, sh_lo, sh_xs, sh_x16, sh_S, xcol + 32 * i, COLH);
#pragma unroll
        for (int k = 0; k < CL; k++)
            if (lane + 64 * k < kRowsPerWave * CH) *reinterpret_cast<u32x4 *>(wslot + 16 * win_chunk<CH, RC>(lane + 64 * k)) = ch_n[0][k];
        // this lane's row block inside its staged window (same wave: no barrier)
        typename F::Regs w;
        F::template load<NT == 1>(w, wslot + c.lr * RC * 16 + ((myoff + (size_t)sb * F::kBytes) & 15), c.kh);
        // the loads below overlap this super-block's math
        if (sb + 1 < sb1) JH_LOAD_X(sb + 1);
#pragma unroll
        for (int st = 0; st + 1 < PD; st++)
#pragma unroll
            for (int k = 0; k < CL; k++) ch_n[st][k] = ch_n[st + 1][k];
        if (sb + PD < sb1) JH_LOAD_W(PD - 1, sb + PD);
        __syncthreads();
        fold(w, c);
    }
    }
#undef JH_LOAD_X
#undef JH_LOAD_W

    if constexpr (PAIR) {
        store_pair(tot, rbase + c.lr, (wave & (kWaves / 2 - 1)) * kRowsPerWave + c.lr, up_half, nrows, c.kh, B,
                   g.swiglu, g.part, g.counters, tile, split, g.ksplit, lds);
        return;
    }
    store_tile<NT>(tot, rbase + c.lr, nrows, c.kh, B, P.y, g.part + P.part0, g.counters + (size_t)P.cnt0 * kCounterStride, tile, split,
                   g.ksplit);
}

// A group of matrices with the same K in one launch (1-D grid): each
// workgroup finds its matrix and runs that matrix's format.
template <int NT, int MASK, bool PAIR = false>
__global__ __launch_bounds__(kThreads) void mfma_group(MfmaGroup g) {
    __shared__ __align__(16) uint8_t lds[lds_bytes<NT, MASK>()];
    const int id = blockIdx.x;
    int m = 0;
    for (int i = 1; i < g.n; i++)
        if (id >= g.p[i].wg0) m = i;
    const MfmaProblem &P = g.p[m];
    const int local = id - P.wg0, tile = local / g.ksplit, split = local - tile * g.ksplit;
    constexpr int PD = NT == 1 ? kPrefetch : 1;
    switch (P.type) {
        case 12: if constexpr ((MASK & 1) != 0) gemm_body<FmtQ4K, NT, PD, PAIR>(P, tile, split, g, lds); break;
        case 13: if constexpr ((MASK & 2) != 0) gemm_body<FmtQ5K, NT, PD, PAIR>(P, tile, split, g, lds); break;
        case 14: if constexpr ((MASK & 4) != 0) gemm_body<FmtQ6K, NT, PD, PAIR>(P, tile, split, g, lds); break;
        case 10: if constexpr ((MASK & 16) != 0) gemm_body<FmtQ2K, NT, PD, PAIR>(P, tile, split, g, lds); break;
        case 11: if constexpr ((MASK & 32) != 0) gemm_body<FmtQ3K, NT, PD, PAIR>(P, tile, split, g, lds); break;
        default: if constexpr ((MASK & 8) != 0) gemm_body<FmtQ8_0, NT, PD, PAIR>(P, tile, split, g, lds); break;
    }
}

// x of one column and super-block into its prepared slab: 16 consecutive
// lanes hold the column's 256 values, 16 each (xv).  The same arithmetic as
// stage_x_column (scale, limbs, sums, butterflies), so both layouts carry
// identical values.
__device__ __forceinline__ void prep_x_column(const float (&xv)[16], int q, uint8_t *slab, int col) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) m = fmaxf(m, fabsf(xv[j]));
    m = row16_max(m);
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);
    const float s = m > 0.f ? ldexpf(1.f, 13 - e) : 1.f;
    half8 h[2], l[2];
    float g[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = xv[4 * k + j] * s;
            const _Float16 hh = (_Float16)v;
            const _Float16 ll = (_Float16)(v - (float)hh);
            h[k >> 1][4 * (k & 1) + j] = hh;
            l[k >> 1][4 * (k & 1) + j] = ll;
            sum += (float)hh + (float)ll;
        }
        g[k] = sum;
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int slot = CtxP::slot(col, 8 * (2 * q + i));
        *reinterpret_cast<half8 *>(slab + kSlabHi + 16 * slot) = h[i];
        *reinterpret_cast<half8 *>(slab + kSlabLo + 16 * slot) = l[i];
    }
    float sub = (g[0] + g[1]) + (g[2] + g[3]);
    sub += dpp_f<0xB1>(sub);
    if ((q & 1) == 0) {
        _Float16 *xs = reinterpret_cast<_Float16 *>(slab + kSlabXs) + col * 16;
        const _Float16 hs = (_Float16)sub;
        xs[q >> 1] = hs;
        xs[8 + (q >> 1)] = (_Float16)(sub - (float)hs);
    }
    const float tot = row16_sum((g[0] + g[2]) + (g[1] + g[3]));
    if (q == 0) reinterpret_cast<float2 *>(slab + kSlabS)[col] = make_float2(tot, 1.f / s);
}

// one workgroup per super-block: 32 columns x 16 lanes (columns >= B are zero)
__global__ __launch_bounds__(512) void x_prep(const float *__restrict__ X, int B, int cols, uint8_t *__restrict__ slabs) {
    const int sb = blockIdx.x, q = threadIdx.x & 15, col = threadIdx.x >> 4;
    float xv[16];
    const float4 *xp = reinterpret_cast<const float4 *>(X + (size_t)min(col, B - 1) * cols + sb * 256 + 16 * q);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 v = col < B ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);
        xv[4 * k] = v.x;
        xv[4 * k + 1] = v.y;
        xv[4 * k + 2] = v.z;
        xv[4 * k + 3] = v.w;
    }
    prep_x_column(xv, q, slabs + (size_t)sb * kSlabBytes, col);
}

// The B <= 32 kernel on prepared x, for matrices with enough row tiles to
// fill the GPU without splitting K (the output projection).  It reads x once
// per super-block from a slab that x_prep wrote, instead of converting it in
// every workgroup.  Per super-block each wave:
//  1. waits until its share of this super-block's x slab (DMA) and its
//     weight chunks have landed, and meets the others at the one barrier;
//  2. starts the DMA of the next slab into the other LDS buffer (everyone has
//     finished the super-block that used it);
//  3. moves its weight chunks through its LDS window into the format's
//     registers and starts the loads of the super-block after next into the
//     freed register set (two sets alternate: weights stay two super-blocks
//     ahead with no register copies);
//  4. runs the MFMAs.
// Loads are issued unconditionally (addresses clamped to the last super-block
// of the range) so that every wave's count of memory operations in flight is
// the same static number at each wait.
template <class F>
__global__ __launch_bounds__(kThreads) void mfma_px(const uint8_t *__restrict__ W, size_t pitch, int row0, int nrows,
                                                    int nsb, const uint8_t *__restrict__ slabs,
                                                    float *__restrict__ Y, int B) {
    constexpr int CH = F::kChunks;
    constexpr int CL = (kRowsPerWave * CH + 63) / 64;
    constexpr int XI = (kSlabRows + kWaves - 1) / kWaves;  // slab rows per wave
    __shared__ __align__(16) uint8_t sh_x[2][kSlabBytes];
    constexpr int RC = F::kRowChunks;  // window row stride (chunks)
    __shared__ __align__(16) uint8_t sh_w[kWaves * kRowsPerWave * RC * 16 + kWinPad];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, lr = lane & 31, kh = lane >> 5;
    const int rbase = blockIdx.x * kRowsPerWG + wave * kRowsPerWave;
    const int sb0 = 0, last = nsb - 1;
    auto row_off = [&](int rho) { return (size_t)(row0 + min(rbase + rho, nrows - 1)) * pitch; };
    size_t coff[CL];
#pragma unroll
    for (int k = 0; k < CL; k++) {
        const int j = min(lane + 64 * k, kRowsPerWave * CH - 1);
        coff[k] = row_off(j / CH) + 16 * (j % CH);
    }
    const size_t myoff = row_off(lr);
    uint8_t *wslot = sh_w + wave * (kRowsPerWave * RC * 16);

    // The slab DMA is issued from inline asm, outside the compiler's
    // bookkeeping: its own waits would otherwise drain every load in flight
    // before the first LDS read after a DMA.  Unknown memory operations can
    // only make the compiler's remaining waits stricter, and the order below
    // keeps them exact (each step's weight chunks are waited for before the
    // step issues its DMA).
    auto dma_x = [&](int sb, int buf) {
        const uint8_t *src = slabs + (size_t)min(sb, last) * kSlabBytes + 16 * lane;
        const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)sh_x[buf];
#pragma unroll
        for (int k = 0; k < XI; k++) {
            const int r = min(wave + kWaves * k, kSlabRows - 1);  // surplus waves repeat the last row (same bytes)
            asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src + 1024 * r),
                         "s"(dst + 1024 * r)
                         : "memory", "m0");
        }
    };
    u32x4 wa[CL], wb[CL];
#define JH_LOAD_W(SET, SB)                                                                                 \
    do {                                                                                                   \
        const size_t sbo = (size_t)min((SB), last) * F::kBytes;                                            \
        _Pragma("unroll") for (int k = 0; k < CL; k++)                                                     \
            SET[k] = *reinterpret_cast<const u32x4 *>(W + ((coff[k] + sbo) & ~size_t(15)));                \
    } while (0)

    f32x16 tot[1] = {(f32x16){}};
#define JH_STEP(SET, SB, BUF)                                                                              \
    do {                                                                                                   \
        /* this wave's part of slab SB and its chunks of SB have landed (only SB + 1's are in flight) */   \
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CL) : "memory");                                        \
        _Pragma("unroll") for (int k = 0; k < CL; k++)                                                     \
            if (lane + 64 * k < kRowsPerWave * CH) *reinterpret_cast<u32x4 *>(wslot + 16 * win_chunk<CH, RC>(lane + 64 * k)) = SET[k]; \
        /* every wave's part of slab SB is in, and every wave is done with slab SB - 1 */                \
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");                                   \
        dma_x((SB) + 1, (BUF) ^ 1);                                                                        \
        typename F::Regs w;                                                                                \
        F::template load<true>(w, wslot + lr * RC * 16 + ((myoff + (size_t)(SB) * F::kBytes) & 15), kh);  \
        JH_LOAD_W(SET, (SB) + 2);                                                                          \
        const CtxP c{lr, kh, sh_x[BUF]};                                                                   \
        if constexpr (F::kSums) {                                                                          \
            F::template compute<1>(w, c, tot);                                                             \
        } else {                                                                                           \
            f32x16 pt[1] = {(f32x16){}};                                                                   \
            F::template compute<1>(w, c, pt);                                                              \
            float S[16], cs[16];                                                                           \
            col_terms<1>(c, 0, S, cs);                                                                     \
            _Pragma("unroll") for (int i = 0; i < 16; i++) tot[0][i] = fmaf(cs[i], pt[0][i], tot[0][i]);   \
        }                                                                                                  \
    } while (0)

    dma_x(sb0, 0);
    JH_LOAD_W(wa, sb0);
    JH_LOAD_W(wb, sb0 + 1);
    int sb = sb0;
    for (; sb < last; sb += 2) {  // pairs of steps: the register sets alternate by name
        JH_STEP(wa, sb, 0);
        JH_STEP(wb, sb + 1, 1);
    }
    if (sb == last) JH_STEP(wa, sb, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA into LDS outlives the workgroup
#undef JH_STEP
#undef JH_LOAD_W

    store_tile<1>(tot, rbase + lr, nrows, kh, B, Y, nullptr, nullptr, blockIdx.x, 0, 1);
}

}  // namespace

// ------------------------------------------------------------------ host side
static bool mfma_applies(const MfmaDesc &d, int B) {
    if ((d.type != 12 && d.type != 13 && d.type != 14 && d.type != 8 && d.type != 10 && d.type != 11) ||
        B < kMfmaMinBatch || B > 64 || d.cols % 256 ||
        d.cols <= 0 || d.row_end <= d.row_start)
        return false;
    if ((d.type == 12 || d.type == 13) && ((reinterpret_cast<uintptr_t>(d.w) | d.pitch) & 15))
        return false;  // K-quant rows are staged as whole aligned 16-byte chunks
    return (reinterpret_cast<uintptr_t>(d.x) & 15) == 0;  // x is read as float4
}

namespace {
struct Plan {
    int nsb, ksb, ksplit, grid;
    bool prepared;  // one unsplit matrix, B <= 32: x_prep + mfma_px
    size_t slab_bytes, part_floats;
};
}  // namespace

// Row tiles of 256 rows; K split the same way for every matrix of the group.
static bool plan_group(int n, const MfmaDesc *d, int B, Plan &p) {
    if (n < 1 || n > kMaxMfmaGroup) return false;
    int tiles = 0;
    size_t rows = 0;
    for (int i = 0; i < n; i++) {
        if (!mfma_applies(d[i], B) || d[i].cols != d[0].cols) return false;
        tiles += (d[i].row_end - d[i].row_start + kRowsPerWG - 1) / kRowsPerWG;
        rows += d[i].row_end - d[i].row_start;
    }
    p.nsb = d[0].cols / 256;
    // One workgroup fits per CU (LDS, VGPRs), so the grid runs in rounds of
    // kMinWorkgroups.  Cost of a split, in super-block steps: rounds x (super-
    // blocks per workgroup + a workgroup's fixed prologue and epilogue, ~5
    // steps), plus one for the hand-off when K is split and a quarter step per
    // split (the partials the last workgroup sums); the smallest split wins
    // ties.  Fitted to the 8B B = 32 shapes ([gate, up]: 2 splits 44 us,
    // 3 splits 57 us, 16 splits 96 us; [o]: 8 splits ahead of 16).
    int best = 1 << 30;
    p.ksb = p.nsb;
    p.ksplit = 1;
    for (int ks = 1; ks <= p.nsb; ks++) {
        const int ksb = (p.nsb + ks - 1) / ks, kse = (p.nsb + ksb - 1) / ksb;
        if (kse > 1 && tiles > kMaxTileCounters) break;  // a split needs a counter per tile
        const int rounds = (tiles * kse + kMinWorkgroups - 1) / kMinWorkgroups;
        const int cost = 4 * (rounds * (ksb + 5) + (kse > 1 ? 1 : 0)) + (kse > 1 ? kse : 0);  // quarter steps
        if (cost < best) {
            best = cost;
            p.ksb = ksb;
            p.ksplit = kse;
        }
    }
    if (const char *f = getenv("JUNO_MFMA_KSPLIT")) {  // tuning runs: a forced split
        const int want = atoi(f);
        if (want >= 1 && want <= p.nsb && (want == 1 || tiles <= kMaxTileCounters)) {
            p.ksb = (p.nsb + want - 1) / want;
            p.ksplit = (p.nsb + p.ksb - 1) / p.ksb;
        }
    }
    p.grid = tiles * p.ksplit;
    p.prepared = n == 1 && p.ksplit == 1 && B <= 32 && d[0].type != 10 && d[0].type != 11;  // slabs carry no 16-column sums
    p.slab_bytes = p.prepared ? (size_t)p.nsb * kSlabBytes : 0;
    p.part_floats = p.ksplit > 1 ? (size_t)p.ksplit * B * rows : 0;
    return true;
}

size_t mfma_group_workspace_bytes(int n, const MfmaDesc *d, int B) {
    Plan p;
    if (!plan_group(n, d, B, p)) return 0;
    const size_t bytes = p.slab_bytes + p.part_floats * sizeof(float);
    return bytes > 256 ? bytes : 256;  // nonzero: the MFMA path applies
}

int mfma_group_plan(int n, const MfmaDesc *d, int B, int *ksplit) {
    Plan p;
    if (!plan_group(n, d, B, p)) return 0;
    *ksplit = p.ksplit;
    return p.prepared ? 2 : 1;
}

template <int NT>
static void launch_group_nt(const MfmaGroup &g, int mask, int grid, hipStream_t s) {
    switch (mask) {
        case 1: mfma_group<NT, 1><<<grid, kThreads, 0, s>>>(g); break;
        case 2: mfma_group<NT, 2><<<grid, kThreads, 0, s>>>(g); break;
        case 4: mfma_group<NT, 4><<<grid, kThreads, 0, s>>>(g); break;
        case 8: mfma_group<NT, 8><<<grid, kThreads, 0, s>>>(g); break;
        case 16: mfma_group<NT, 16><<<grid, kThreads, 0, s>>>(g); break;
        case 32: mfma_group<NT, 32><<<grid, kThreads, 0, s>>>(g); break;
        default: mfma_group<NT, 63><<<grid, kThreads, 0, s>>>(g); break;
    }
}

// JUNO_MFMA_PAIR=0: the batched SwiGLU takes the grouped launch and silu_mul (A/B runs)
static bool mfma_pair_wanted() {
    static const bool on = [] {
        const char *v = getenv("JUNO_MFMA_PAIR");
        return !(v && v[0] == '0');
    }();
    return on;
}

bool mfma_swiglu_applies(const MfmaDesc &gate, const MfmaDesc &up, int B) {
    if (!mfma_pair_wanted()) return false;
    if (B < kMfmaMinBatch || B > 32 || gate.type != up.type || gate.cols != up.cols || gate.pitch != up.pitch ||
        gate.x != up.x || gate.row_start != 0 || up.row_start != 0 || gate.row_end != up.row_end)
        return false;
    if (gate.type != 12 && gate.type != 13 && gate.type != 14 && gate.type != 8) return false;
    if (((reinterpret_cast<uintptr_t>(up.w) | up.pitch) & 15) && (up.type == 12 || up.type == 13)) return false;
    MfmaDesc v = gate;
    v.row_end = 2 * gate.row_end;  // the pair's virtual rows: same tiles and K split as one matrix of 2 x rows
    Plan p;
    return plan_group(1, &v, B, p) && (p.ksplit == 1 || (gate.row_end + kRowsPerWG / 2 - 1) / (kRowsPerWG / 2) <= kMaxTileCounters);
}

size_t mfma_swiglu_workspace_bytes(const MfmaDesc &gate, int B) {
    MfmaDesc v = gate;
    v.row_end = 2 * gate.row_end;
    Plan p;
    if (!plan_group(1, &v, B, p)) return 0;
    return p.ksplit > 1 ? sizeof(float) * (size_t)p.ksplit * B * v.row_end : 16;
}

hipError_t launch_mfma_swiglu(const MfmaDesc &gate, const MfmaDesc &up, int B, float *out, void *workspace,
                              int *counters, hipStream_t s) {
    if (!mfma_swiglu_applies(gate, up, B)) return hipErrorNotSupported;
    MfmaDesc v = gate;
    v.row_end = 2 * gate.row_end;
    Plan p;
    plan_group(1, &v, B, p);
    if (p.ksplit > 1 && !counters) return hipErrorNotSupported;
    MfmaGroup g = {};
    g.part = reinterpret_cast<float *>(workspace);
    g.counters = counters;
    g.n = 1;
    g.nsb = p.nsb;
    g.ksb = p.ksb;
    g.ksplit = p.ksplit;
    g.B = B;
    g.w2 = up.w;
    g.swiglu = out;
    MfmaProblem &q = g.p[0];
    q.w = gate.w;
    q.x = gate.x;
    q.y = nullptr;
    q.pitch = gate.pitch;
    q.type = gate.type;
    q.row0 = 0;
    q.rows = gate.row_end;
    q.tiles = (q.rows + kRowsPerWG / 2 - 1) / (kRowsPerWG / 2);
    q.wg0 = q.cnt0 = 0;
    q.part0 = 0;
    const int grid = q.tiles * p.ksplit;
    switch (gate.type) {
        case 12: mfma_group<1, 1, true><<<grid, kThreads, 0, s>>>(g); break;
        case 13: mfma_group<1, 2, true><<<grid, kThreads, 0, s>>>(g); break;
        case 14: mfma_group<1, 4, true><<<grid, kThreads, 0, s>>>(g); break;
        default: mfma_group<1, 8, true><<<grid, kThreads, 0, s>>>(g); break;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ static scratch
// Split-K counters (kCounterSlots lines of kCounterStride ints), then
// kStaticScratchBytes of workspace.  In host code `scratch` names a host-side
// stand-in, not device memory: kernels get the per-device address that
// hipGetSymbolAddress returns.  Every call on a device shares that device's
// copy, so calls that overlap on one device race.
constexpr size_t kStaticCounterBytes = sizeof(int) * (size_t)kCounterSlots * kCounterStride;
static __device__ __align__(256) uint8_t scratch[kStaticCounterBytes + kStaticScratchBytes];

namespace {
__global__ void zero_words(uint32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}
}  // namespace

hipError_t static_scratch(int device, hipStream_t s, void **workspace, int **counters) {
    static std::mutex mu;
    static uint8_t *ptr[64];
    static bool zeroed[64];
    if (device < 0 || device >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(mu);
    if (!ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // the current device's copy
        if (e != hipSuccess) return e;
        ptr[device] = static_cast<uint8_t *>(p);
    }
    if (!zeroed[device]) {
        // a kernel, not a memset: the first call may be under graph capture
        const int n = (int)(kStaticCounterBytes / 4);
        zero_words<<<(n + 255) / 256, 256, 0, s>>>(reinterpret_cast<uint32_t *>(ptr[device]), n);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        zeroed[device] = true;
    }
    *counters = reinterpret_cast<int *>(ptr[device]);
    *workspace = ptr[device] + kStaticCounterBytes;
    return hipSuccess;
}

hipError_t launch_mfma_group(int n, const MfmaDesc *d, int B, void *workspace, int *counters, hipStream_t s) {
    Plan p;
    if (!plan_group(n, d, B, p)) return hipErrorNotSupported;
    if (p.ksplit > 1 && !counters) return hipErrorNotSupported;
    uint8_t *ws = reinterpret_cast<uint8_t *>(workspace);
    if (p.prepared) {
        const MfmaDesc &m = d[0];
        const int nrows = m.row_end - m.row_start;
        x_prep<<<p.nsb, 512, 0, s>>>(m.x, B, m.cols, ws);
#define JH_PX(F) mfma_px<F><<<p.grid, kThreads, 0, s>>>(m.w, m.pitch, m.row_start, nrows, p.nsb, ws, m.y, B)
        if (m.type == 12) JH_PX(FmtQ4K);
        else if (m.type == 13) JH_PX(FmtQ5K);
        else if (m.type == 14) JH_PX(FmtQ6K);
        else JH_PX(FmtQ8_0);
#undef JH_PX
        return hipGetLastError();
    }
    MfmaGroup g = {};
    g.part = reinterpret_cast<float *>(ws);
    g.counters = counters;
    g.n = n;
    g.nsb = p.nsb;
    g.ksb = p.ksb;
    g.ksplit = p.ksplit;
    g.B = B;
    int mask = 0, wg = 0, cnt = 0;
    size_t part = 0;
    for (int i = 0; i < n; i++) {
        MfmaProblem &q = g.p[i];
        q.w = d[i].w;
        q.x = d[i].x;
        q.y = d[i].y;
        q.pitch = d[i].pitch;
        q.type = d[i].type;
        q.row0 = d[i].row_start;
        q.rows = d[i].row_end - d[i].row_start;
        q.tiles = (q.rows + kRowsPerWG - 1) / kRowsPerWG;
        q.wg0 = wg;
        q.cnt0 = cnt;
        q.part0 = part;
        wg += q.tiles * p.ksplit;
        cnt += q.tiles;
        part += p.ksplit > 1 ? (size_t)p.ksplit * B * q.rows : 0;
        mask |= q.type == 12 ? 1 : q.type == 13 ? 2 : q.type == 14 ? 4 : q.type == 10 ? 16 : q.type == 11 ? 32 : 8;
    }
    if (B <= 32) launch_group_nt<1>(g, mask, p.grid, s);
    else launch_group_nt<2>(g, mask, p.grid, s);
    return hipGetLastError();
}

hipError_t mfma_timeline_read(unsigned long long *out, size_t n) {
#ifdef JH_TIMELINE
    if (n > (size_t)kMtWg * 8 * kMtPer) n = (size_t)kMtWg * 8 * kMtPer;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_mtimeline), n * sizeof(unsigned long long));
#else
    (void)out;
    (void)n;
    return hipErrorNotSupported;
#endif
}

}  // namespace jh
