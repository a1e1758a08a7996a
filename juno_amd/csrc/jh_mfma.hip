// jh_mfma.hip -- batched decode (16 <= B <= 64) on Q4_K / Q5_K / Q6_K / Q8_0 through
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
//    (Q4_K: 1024 + ls*q <= 1969 by one 24-bit multiply-add per pair; Q6_K:
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
//    and a small kernel adds the partials in split order (deterministic; no
//    float atomics).
#include "jh_device.hpp"
#include "jh_kernels.hpp"

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

constexpr int kRowsPerWave = 32;
constexpr int kWaves = 8;  // waves per workgroup: 256 rows share each staged x slice
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWG = kWaves * kRowsPerWave;
constexpr int kXPad = 8;  // halves of padding per LDS column (spreads banks)

// ------------------------------------------------------------------ workspace layout
// Split-K partials [ksplit][B][rows] f32 (only when the K range is split).
struct XWork {
    int Bp, cols, nsb;  // padded batch, columns, super-blocks (cols / 256)
    int rows, ksplit;
    uint8_t *base;
    __host__ __device__ size_t bytes() const { return ksplit > 1 ? (size_t)ksplit * Bp * rows * 4 : 0; }
    __device__ float *part() const { return reinterpret_cast<float *>(base); }
};

// x into the LDS image of one column and super-block, inside the GEMM: 16
// consecutive lanes hold its 256 values, 16 each (xv).  A power-of-two scale
// puts max |x s| in [2^12, 2^13) (exact, undone on the partial sums), then x s
// is split into fp16 hi + lo limbs, and the 32-column sub-block sums (as hi and
// lo halves) and the super-block sum S are formed over 4-value groups with
// fixed butterflies (deterministic).
__device__ __forceinline__ void stage_x_column(const float (&xv)[16], int q, _Float16 *sh_hi, _Float16 *sh_lo,
                                               _Float16 *sh_xs, float2 *sh_S, int col, int colh) {
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) m = fmaxf(m, fabsf(xv[j]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));  // the 16 lanes of the column
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
    // sub-block (32 values = groups 8i .. 8i+7 = this lane and its neighbour)
    float sub = (g[0] + g[1]) + (g[2] + g[3]);
    sub += __shfl_xor(sub, 1);
    if ((q & 1) == 0) {
        const _Float16 h = (_Float16)sub;
        sh_xs[col * 16 + (q >> 1)] = h;
        sh_xs[col * 16 + 8 + (q >> 1)] = (_Float16)(sub - (float)h);
    }
    // super-block total: a butterfly over the column's 64 groups (across the
    // 16 lanes, then within the lane)
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) g[k] += __shfl_xor(g[k], o);
    const float tot = (g[0] + g[2]) + (g[1] + g[3]);
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

struct Ctx {
    int wave, lr, kh;
    const _Float16 *sh_hi, *sh_lo, *sh_xs;
    const float2 *sh_S;
};
constexpr int COLH = 256 + kXPad;  // halves per LDS column of the staged x slice

// Operand roles: x is the A operand (its 32 rows are batch columns) and the
// weights are B, so D[b][r] = sum_k x[b][k] w[r][k].  In the 32x32x16 layout
// lane (lr, kh) supplies weight row lr (K elements 8kh .. 8kh+7) and holds
// D for row lr and batch columns 8(i/4) + 4kh + (i%4), i < 16: every per-row
// scale (d, dmin, d*sc) lives in the lane's own registers, and consecutive
// lanes store consecutive rows.
__device__ __forceinline__ int batch_of(int n, int i, int kh) { return n * 32 + 8 * (i >> 2) + 4 * kh + (i & 3); }

// four byte pairs of two words -> 16-bit lanes, OR'ed into fp16 1024 + u
__device__ __forceinline__ half8 bytes_to_h8(uint32_t w0, uint32_t w1, half2v off) {
    const uint32_t p[4] = {__builtin_amdgcn_perm(0u, w0, 0x0C010C00u), __builtin_amdgcn_perm(0u, w0, 0x0C030C02u),
                           __builtin_amdgcn_perm(0u, w1, 0x0C010C00u), __builtin_amdgcn_perm(0u, w1, 0x0C030C02u)};
    half8 a;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const half2v h = __builtin_bit_cast(half2v, p[j] | 0x64006400u) - off;  // exact: small integers
        a[2 * j] = h[0];
        a[2 * j + 1] = h[1];
    }
    return a;
}

// acc[n] += x_hi . w + x_lo . w over one K-step (x columns at xoff)
template <int NT>
__device__ __forceinline__ void mfma_xw(const Ctx &c, const half8 &w, int xoff, f32x16 *acc) {
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int col = n * 32 + c.lr;
        const half8 xh = *reinterpret_cast<const half8 *>(c.sh_hi + col * COLH + xoff);
        const half8 xl = *reinterpret_cast<const half8 *>(c.sh_lo + col * COLH + xoff);
        acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, w, acc[n], 0, 0, 0);
        acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, w, acc[n], 0, 0, 0);
    }
}

// (S, 1/scale) of the 16 batch columns a lane holds for tile n
template <int NT>
__device__ __forceinline__ void col_terms(const Ctx &c, int n, float (&S)[16], float (&cs)[16]) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float4 v = *reinterpret_cast<const float4 *>(c.sh_S + n * 32 + 8 * q + 4 * c.kh + 2 * h);
            S[4 * q + 2 * h] = v.x;
            cs[4 * q + 2 * h] = v.y;
            S[4 * q + 2 * h + 1] = v.z;
            cs[4 * q + 2 * h + 1] = v.w;
        }
}

// Q4_K (matVecQ4Kraw, LlamaTransformerHandler.java:1428-1468): w = d*ls*q - dmin*lm.
// B = 1024 + ls*q (<= 1969, exact), built with one 24-bit multiply-add per
// pair; 1024 * sum(x) and the min term (one more MFMA: A = [sub-block sums
// hi | lo], B = [lm | lm]) are removed per super-block with d and dmin.
// Q5_K (Q5 = true, matVecQ5Kraw :1525-1576): q has a 5th bit from qh, so
// ls*q reaches 1953 and 1024 + ls*q would pass fp16's exact integers; B =
// ls*q is converted instead (v_cvt_f16_u16, exact below 2048).
template <bool Q5>
struct FmtKQ {
    static constexpr int kBytes = Q5 ? 176 : 144;
    static constexpr int kChunks = kBytes / 16;  // rows are 16-byte aligned (pitch kBytes * n, aligned base)
    static constexpr int kQs = Q5 ? 48 : 16;
    static constexpr bool kSums = true;
    struct Regs {
        u32x4 hd;
        u32x2 qp[4][2];
        u32x2 qh[2];  // Q5_K: qh bytes 16 j + 8 kh .. +8 (bit s for sub-block s)
    };
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
    template <int NT>
    static __device__ __forceinline__ void compute(const Regs &r, const Ctx &c, f32x16 *tot) {
        // 6-bit scales and mins of the 8 sub-blocks (q4kScaleRaw / q4kMinRaw, :1471-1482)
        int ls[8], lm[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ls[j] = (int)byte_of(r.hd.y, j) & 63;
            lm[j] = (int)byte_of(r.hd.z, j) & 63;
            ls[j + 4] = (int)((byte_of(r.hd.w, j) & 0x0F) | ((byte_of(r.hd.y, j) & 0xC0) >> 2));
            lm[j + 4] = (int)((byte_of(r.hd.w, j) >> 4) | ((byte_of(r.hd.z, j) & 0xC0) >> 2));
        }
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
                    const uint32_t v = __umul24(pr[j], (uint32_t)ls[s]) + 0x64006400u;
                    w[2 * j] = __builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFF));
                    w[2 * j + 1] = __builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
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
            const half8 xm = *reinterpret_cast<const half8 *>(c.sh_xs + col * 16 + 8 * c.kh);
            const f32x16 mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(xm, wm, (f32x16){}, 0, 0, 0);
            float S[16], cs[16];
            col_terms<NT>(c, n, S, cs);
#pragma unroll
            for (int i = 0; i < 16; i++)
                tot[n][i] = fmaf(cs[i], fmaf(d, fmaf(Q5 ? 0.f : -1024.f, S[i], acc[n][i]), -dmin * mn[i]), tot[n][i]);
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
    static constexpr bool kSums = false;
    struct Regs {
        u32x2 ql[2][2][2];  // [half n][ql +32 p][j]: bytes 64n + 32p + 16j + 8kh
        u32x2 qh[2][2];     // [n][j]: bytes 128 + 32n + 16j + 8kh
        u32x4 sc;           // bytes 192..207
        uint32_t dw;        // bytes 206..209: d in the high half
    };
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                r.ql[n][0][j] = *reinterpret_cast<const u32x2a2 *>(p + 64 * n + 16 * j + 8 * kh);
                r.ql[n][1][j] = *reinterpret_cast<const u32x2a2 *>(p + 64 * n + 32 + 16 * j + 8 * kh);
                r.qh[n][j] = *reinterpret_cast<const u32x2a2 *>(p + 128 + 32 * n + 16 * j + 8 * kh);
            }
        r.sc = *reinterpret_cast<const u32x4a2 *>(p + 192);
        r.dw = *reinterpret_cast<const u32a2 *>(p + 206);
    }
    template <int NT>
    static __device__ __forceinline__ void compute(const Regs &r, const Ctx &c, f32x16 *tot) {
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
    static constexpr bool kSums = false;
    struct Regs {
        u32x4 q[8];     // block b: bytes 34b + 2 + 16kh .. +16
        uint32_t d[8];  // d of block b (low half)
    };
    static __device__ __forceinline__ void load(Regs &r, const uint8_t *p, int kh) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            r.q[b] = *reinterpret_cast<const u32x4a2 *>(p + 34 * b + 2 + 16 * kh);
            r.d[b] = *reinterpret_cast<const uint16_t *>(p + 34 * b);
        }
    }
    template <int NT>
    static __device__ __forceinline__ void compute(const Regs &r, const Ctx &c, f32x16 *tot) {
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

// ------------------------------------------------------------------ batched kernel
template <class F, int NT, int PD>  // NT = padded batch / 32, PD = weight prefetch depth (super-blocks)
__global__ __launch_bounds__(kThreads) void mfma_gemm(const uint8_t *__restrict__ W, size_t pitch, int row0, int nrows,
                                                      int nsb, int ksb, XWork xw, const float *__restrict__ X,
                                                      float *__restrict__ Y, int B) {
    constexpr int BP = 32 * NT;
    constexpr int CPT = BP / 32;  // x columns converted per thread (16 lanes per column and super-block)
    constexpr int CH = F::kChunks;          // 16-byte chunks staged per row and super-block
    constexpr int CL = (kRowsPerWave * CH + 63) / 64;  // chunks per lane
    __shared__ __align__(16) _Float16 sh_hi[BP * COLH];
    __shared__ __align__(16) _Float16 sh_lo[BP * COLH];
    __shared__ __align__(16) _Float16 sh_xs[BP * 16];
    __shared__ __align__(16) float2 sh_S[BP];  // (sum of x, 1 / column scale) per column
    __shared__ __align__(16) uint8_t sh_w[kWaves][kRowsPerWave * CH * 16];  // wave-private row blocks

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const Ctx c{wave, lane & 31, lane >> 5, sh_hi, sh_lo, sh_xs, sh_S};
    const int rbase = blockIdx.x * kRowsPerWG + wave * kRowsPerWave;
    const int sb0 = blockIdx.y * ksb, sb1 = min(nsb, sb0 + ksb);
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
    uint8_t *wslot = sh_w[wave];

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
            const float4 *xp = reinterpret_cast<const float4 *>(X + (size_t)min(b, B - 1) * xw.cols +     \
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

    if (sb0 < sb1) JH_LOAD_X(sb0);
#pragma unroll
    for (int st = 0; st < PD; st++)
        if (sb0 + st < sb1) JH_LOAD_W(st, sb0 + st);
    for (int sb = sb0; sb < sb1; sb++) {
        __syncthreads();  // the previous super-block's LDS contents are consumed
#pragma unroll
        for (int i = 0; i < CPT; i++)
            stage_x_column(xv_n[i], xq, sh_hi, sh_lo, sh_xs, sh_S, xcol + 32 * i, COLH);
#pragma unroll
        for (int k = 0; k < CL; k++)
            if (lane + 64 * k < kRowsPerWave * CH) *reinterpret_cast<u32x4 *>(wslot + 16 * (lane + 64 * k)) = ch_n[0][k];
        // this lane's row block inside its staged window (same wave: no barrier)
        typename F::Regs w;
        F::load(w, wslot + c.lr * CH * 16 + ((myoff + (size_t)sb * F::kBytes) & 15), c.kh);
        // the loads below overlap this super-block's math
        if (sb + 1 < sb1) JH_LOAD_X(sb + 1);
#pragma unroll
        for (int st = 0; st + 1 < PD; st++)
#pragma unroll
            for (int k = 0; k < CL; k++) ch_n[st][k] = ch_n[st + 1][k];
        if (sb + PD < sb1) JH_LOAD_W(PD - 1, sb + PD);
        __syncthreads();
        if constexpr (F::kSums) {
            F::template compute<NT>(w, c, tot);
        } else {
            f32x16 part[NT];
#pragma unroll
            for (int n = 0; n < NT; n++) part[n] = (f32x16){};
            F::template compute<NT>(w, c, part);
#pragma unroll
            for (int n = 0; n < NT; n++) {
                float S[16], cs[16];
                col_terms<NT>(c, n, S, cs);
#pragma unroll
                for (int i = 0; i < 16; i++) tot[n][i] = fmaf(cs[i], part[n][i], tot[n][i]);
            }
        }
    }
#undef JH_LOAD_X
#undef JH_LOAD_W

    // a single split writes y; otherwise each split writes its partial tile
    // and reduce_splits adds them in split order (deterministic).  A hand-off
    // between workgroups inside this kernel would need a device-scope release
    // per workgroup, which on a multi-XCD part writes back the whole L2 each
    // time (~100 us measured).
    const int r = rbase + c.lr;
    if (r >= nrows) return;
    float *out = gridDim.y == 1 ? Y : xw.part() + (size_t)blockIdx.y * B * nrows;
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int b = batch_of(n, i, c.kh);
            if (b < B) out[(size_t)b * nrows + r] = tot[n][i];
        }
}

// y[i] = sum over splits k (in order) of part[k][i]; V outputs per thread
template <typename T>
__device__ __forceinline__ void add_to(T &a, const T &b) { a += b; }
template <>
__device__ __forceinline__ void add_to<float4>(float4 &a, const float4 &b) {
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
}
template <typename T>
__global__ __launch_bounds__(256) void reduce_splits(XWork xw, int n, int ksplit, float *__restrict__ Y) {
    const T *p = reinterpret_cast<const T *>(xw.part());
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        T v[16];
        T acc{};
        for (int k0 = 0; k0 < ksplit; k0 += 16) {
            const int nk = min(16, ksplit - k0);
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (k < nk) v[k] = p[(size_t)(k0 + k) * n + i];
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (k < nk) add_to(acc, v[k]);
        }
        reinterpret_cast<T *>(Y)[i] = acc;
    }
}

}  // namespace

static void mfma_split(int nrows, int nsb, int &tiles, int &ksplit, int &ksb) {
    tiles = (nrows + kRowsPerWG - 1) / kRowsPerWG;
    ksplit = (kMinWorkgroups + tiles - 1) / tiles;
    if (ksplit > nsb) ksplit = nsb;
    if (ksplit < 1) ksplit = 1;
    ksb = (nsb + ksplit - 1) / ksplit;
    ksplit = (nsb + ksb - 1) / ksb;
}

size_t mfma_workspace_bytes(int type, int B, int cols, int rows) {
    if ((type != 12 && type != 13 && type != 14 && type != 8) || B < 16 || B > 64 || cols % 256 || rows < 1) return 0;
    int tiles, ksplit, ksb;
    mfma_split(rows, cols / 256, tiles, ksplit, ksb);
    XWork w{(B + 31) / 32 * 32, cols, cols / 256, rows, ksplit, nullptr};
    return w.bytes() > 256 ? w.bytes() : 256;  // nonzero: the MFMA path applies
}

hipError_t launch_gemm_mfma_ws(const GemvArgs &a, void *workspace, hipStream_t s) {
    if ((a.type != 12 && a.type != 13 && a.type != 14 && a.type != 8) || a.batch < 16 || a.batch > 64 || a.cols % 256)
        return hipErrorNotSupported;
    if ((a.type == 12 || a.type == 13) && ((reinterpret_cast<uintptr_t>(a.w) | a.pitch) & 15))
        return hipErrorNotSupported;  // K-quant rows are staged as whole aligned 16-byte chunks
    const int B = a.batch, Bp = (B + 31) / 32 * 32;
    const int nrows = a.row_end - a.row_start;
    const int nsb = a.cols / 256;
    int tiles, ksplit, ksb;
    mfma_split(nrows, nsb, tiles, ksplit, ksb);
    XWork w{Bp, a.cols, nsb, nrows, ksplit, reinterpret_cast<uint8_t *>(workspace)};
    dim3 grid(tiles, ksplit);
#define JH_GEMM(F, NT) mfma_gemm<F, NT, NT == 1 ? kPrefetch : 1><<<grid, kThreads, 0, s>>>(a.w, a.pitch, a.row_start, nrows, nsb, ksb, w, a.x, a.y, B)
    if (a.type == 12) {
        if (Bp == 32) JH_GEMM(FmtQ4K, 1); else JH_GEMM(FmtQ4K, 2);
    } else if (a.type == 13) {
        if (Bp == 32) JH_GEMM(FmtQ5K, 1); else JH_GEMM(FmtQ5K, 2);
    } else if (a.type == 14) {
        if (Bp == 32) JH_GEMM(FmtQ6K, 1); else JH_GEMM(FmtQ6K, 2);
    } else {
        if (Bp == 32) JH_GEMM(FmtQ8_0, 1); else JH_GEMM(FmtQ8_0, 2);
    }
#undef JH_GEMM
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || ksplit == 1) return e;
    const int n = B * nrows;
    if (n % 4 == 0 && reinterpret_cast<uintptr_t>(a.y) % 16 == 0)
        reduce_splits<float4><<<(unsigned)std::min((n / 4 + 255) / 256, 2048), 256, 0, s>>>(w, n / 4, ksplit, a.y);
    else
        reduce_splits<float><<<(unsigned)std::min((n + 255) / 256, 2048), 256, 0, s>>>(w, n, ksplit, a.y);
    return hipGetLastError();
}

}  // namespace jh
