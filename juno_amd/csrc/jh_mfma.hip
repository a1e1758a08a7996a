// jh_mfma.hip -- batched decode (16 <= B <= 64) on Q4_K through LDS + fp16 MFMA.
//
// Y[b][r] = sum_c deq(W[r][c]) * X[b][c] is a dense contraction once B >= 16:
// per HBM byte it needs 2B/0.5625 flops, more than the VALU can issue without
// packed fp32, but far below the MFMA ridge (~312 flop/B).  The kernel keeps
// the weights exact and moves the arithmetic to v_mfma_f32_32x32x16_f16:
//
//  * A (weights): for Q4_K, w = d*ls*q - dmin*lm with 6-bit ls and 4-bit q, so
//    ls*q <= 945 is an exact fp16 integer.  Each lane builds its A fragment as
//    the fp16 bit pattern 0x6400 | ls*q, i.e. 1024 + ls*q, with one integer
//    multiply-add per pair; the 1024 offset is removed after the super-block
//    as 1024 * sum(x).  The per-row d and dmin are applied in fp32 once per
//    256-column super-block (fresh accumulators per super-block).
//  * The min term dmin * sum_s lm_s * sum(x over sub-block s) is one more
//    MFMA per super-block: A = [lm_0..7 | lm_0..7], B = [xsum_hi | xsum_lo].
//  * B (activations): x is split into fp16 hi + lo limbs (x = hi + lo to
//    ~2^-22; one fp16 rounding of x alone would exceed the 1e-3 bar), after a
//    per-column power-of-two scaling that keeps fp16 in range.  A small prep
//    kernel writes hi, lo, sub-block sums and super-block sums once per call
//    into a workspace; workgroups stage each super-block's slice in LDS.
//  * Work split: a workgroup is 4 waves x 32 rows = 128 rows, all B columns,
//    and a range of super-blocks.  Every x fragment staged in LDS feeds 128
//    rows (operand traffic ~3.5x the weight bytes at B = 32, within LDS
//    bandwidth).  The next super-block's weights and x slice are loaded while
//    the current one is multiplied.  When the row tiles are too few to fill
//    256 CUs the K range is split across workgroups; each split writes its
//    partial tile to the workspace and a small kernel adds the partials in
//    split order (deterministic; no float atomics).
#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kMinWorkgroups = 512;  // split K until the grid has this many

constexpr int kRowsPerWave = 32;
constexpr int kRowsPerWG = 4 * kRowsPerWave;
constexpr int kXPad = 8;  // halves of padding per LDS column (spreads banks)

// ------------------------------------------------------------------ workspace layout
struct XWork {
    int Bp, cols, nsb;  // padded batch, columns, super-blocks (cols / 256)
    int rows, ksplit;  // split-K partials: [ksplit][B][rows] f32
    uint8_t *base;
    // The prepared x is super-block major: one contiguous slab per super-block,
    //   [hi: Bp x 256 halves][lo: Bp x 256 halves][xs: Bp x 16 halves][S: Bp f32]
    // so the slice every workgroup stages for a super-block is one linear
    // stretch of memory (a column-major image would put the 32 column segments
    // of a slice a power-of-two stride apart, on the same memory channels).
    __host__ __device__ size_t slab() const { return ((size_t)Bp * 1060 + 255) & ~size_t(255); }
    __host__ __device__ size_t x_off() const { return 0; }
    __host__ __device__ size_t sc_off() const { return x_off() + slab() * nsb; }  // [Bp] f32
    __host__ __device__ size_t part_off() const { return (sc_off() + (size_t)Bp * 4 + 255) & ~size_t(255); }
    __host__ __device__ size_t bytes() const { return part_off() + (ksplit > 1 ? (size_t)ksplit * Bp * rows * 4 : 0); }  // [ksplit][B][rows]
    __device__ float *part() const { return reinterpret_cast<float *>(base + part_off()); }
    __device__ uint8_t *sbx(int sb) const { return base + x_off() + slab() * sb; }
    __device__ _Float16 *hi(int sb) const { return reinterpret_cast<_Float16 *>(sbx(sb)); }
    __device__ _Float16 *lo(int sb) const { return reinterpret_cast<_Float16 *>(sbx(sb) + (size_t)Bp * 512); }
    __device__ _Float16 *xs(int sb) const { return reinterpret_cast<_Float16 *>(sbx(sb) + (size_t)Bp * 1024); }
    __device__ float *S(int sb) const { return reinterpret_cast<float *>(sbx(sb) + (size_t)Bp * 1056); }
    __device__ float *scale() const { return reinterpret_cast<float *>(base + sc_off()); }
};

__device__ __forceinline__ float wave_reduce_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_reduce_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// One workgroup per (padded) batch column.
__global__ __launch_bounds__(256) void x_prep_mfma(const float *__restrict__ X, int B, XWork w) {
    __shared__ float red[4];
    const int b = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cols = w.cols;
    const float *xb = X + (size_t)b * cols;
    const bool real = b < B;
    float m = 0.f;
    if (real)
        for (int c = threadIdx.x * 4; c < cols; c += 1024) {
            const float4 v = *reinterpret_cast<const float4 *>(xb + c);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    m = wave_reduce_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // power-of-two scale: max |x * s| in [2^12, 2^13); exact, and undone on y
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);
    const float s = m > 0.f ? ldexpf(1.f, 13 - e) : 1.f;
    if (threadIdx.x == 0) w.scale()[b] = 1.f / s;
    for (int sb = wave; sb < w.nsb; sb += 4) {
        const int c = sb * 256 + lane * 4;
        _Float16 *hi = w.hi(sb) + (size_t)b * 256 + lane * 4, *lo = w.lo(sb) + (size_t)b * 256 + lane * 4;
        float4 v = real ? *reinterpret_cast<const float4 *>(xb + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float e4[4] = {v.x * s, v.y * s, v.z * s, v.w * s};
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const _Float16 h = (_Float16)e4[j];
            const _Float16 l = (_Float16)(e4[j] - (float)h);
            hi[j] = h;
            lo[j] = l;
            sum += (float)h + (float)l;
        }
        // sub-block (32 columns = 8 lanes) sums, and the super-block sum
        float sub = sum;
        sub += __shfl_xor(sub, 1);
        sub += __shfl_xor(sub, 2);
        sub += __shfl_xor(sub, 4);
        const float tot = wave_reduce_sum(sum);
        _Float16 *xs = w.xs(sb) + (size_t)b * 16;
        if ((lane & 7) == 0) {
            const _Float16 h = (_Float16)sub;
            xs[lane >> 3] = h;
            xs[8 + (lane >> 3)] = (_Float16)(sub - (float)h);
        }
        if (lane == 0) w.S(sb)[b] = tot;
    }
}

// ------------------------------------------------------------------ Q4_K batched kernel
template <int NT>  // NT = padded batch / 32
__global__ __launch_bounds__(256) void mfma_q4k(const uint8_t *__restrict__ W, size_t pitch, int row0, int nrows,
                                                int nsb, int ksb, XWork xw, float *__restrict__ Y, int B) {
    constexpr int BP = 32 * NT;
    constexpr int COLH = 256 + kXPad;   // halves per LDS column
    constexpr int XU = BP * 32 / 256;   // 16-byte x units per thread per limb
    __shared__ __align__(16) _Float16 sh_hi[BP * COLH];
    __shared__ __align__(16) _Float16 sh_lo[BP * COLH];
    __shared__ __align__(16) _Float16 sh_xs[BP * 16];
    __shared__ float sh_S[BP];
    __shared__ __align__(16) float sh_d[4][kRowsPerWave], sh_dm[4][kRowsPerWave];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int kh = lane >> 5, lr = lane & 31;
    const int rbase = blockIdx.x * kRowsPerWG + wave * kRowsPerWave;
    const int myrow = min(rbase + lr, nrows - 1);
    const uint8_t *rowp = W + (size_t)(row0 + myrow) * pitch;
    const int sb0 = blockIdx.y * ksb, sb1 = min(nsb, sb0 + ksb);

    // register sets for the next super-block: x slice units and weight bytes
    u32x4 xh_n[XU], xl_n[XU], xs_n;
    float S_n = 0.f;
    u32x4 hd_n;
    u32x2 qp_n[4][2];
    // (macros rather than lambdas: the register arrays must stay in VGPRs)
#define JH_LOAD_X(SB)                                                                                     \
    do {                                                                                                  \
        const u32x4 *hp = reinterpret_cast<const u32x4 *>(xw.hi(SB));                                    \
        const u32x4 *lp = reinterpret_cast<const u32x4 *>(xw.lo(SB));                                    \
        _Pragma("unroll") for (int k = 0; k < XU; k++) {                                                  \
            xh_n[k] = hp[threadIdx.x + 256 * k];                                                          \
            xl_n[k] = lp[threadIdx.x + 256 * k];                                                          \
        }                                                                                                 \
        xs_n = reinterpret_cast<const u32x4 *>(xw.xs(SB))[min((int)threadIdx.x, BP * 2 - 1)];            \
        S_n = xw.S(SB)[min((int)threadIdx.x, BP - 1)];                                                    \
    } while (0)
#define JH_LOAD_W(SB)                                                                                     \
    do {                                                                                                  \
        const uint8_t *bp = rowp + (size_t)(SB) * 144;                                                    \
        hd_n = *reinterpret_cast<const u32x4 *>(bp);                                                      \
        _Pragma("unroll") for (int g = 0; g < 4; g++) {                                                   \
            qp_n[g][0] = *reinterpret_cast<const u32x2 *>(bp + 16 + 32 * g + 8 * kh);                     \
            qp_n[g][1] = *reinterpret_cast<const u32x2 *>(bp + 16 + 32 * g + 16 + 8 * kh);                \
        }                                                                                                 \
    } while (0)

    f32x16 tot[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) tot[n] = (f32x16){};

    if (sb0 < sb1) {
        JH_LOAD_X(sb0);  // x first: waiting for it must not wait for the weight stream
        JH_LOAD_W(sb0);
    }
    for (int sb = sb0; sb < sb1; sb++) {
        __syncthreads();  // the previous super-block's LDS slice is consumed
#pragma unroll
        for (int k = 0; k < XU; k++) {
            const int i = threadIdx.x + 256 * k, col = i >> 5, u = i & 31;
            *reinterpret_cast<u32x4 *>(sh_hi + col * COLH + 8 * u) = xh_n[k];
            *reinterpret_cast<u32x4 *>(sh_lo + col * COLH + 8 * u) = xl_n[k];
        }
        if (threadIdx.x < BP * 2) *reinterpret_cast<u32x4 *>(sh_xs + (threadIdx.x >> 1) * 16 + 8 * (threadIdx.x & 1)) = xs_n;
        if (threadIdx.x < BP) sh_S[threadIdx.x] = S_n;
        const u32x4 hd = hd_n;
        u32x2 qp[4][2];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            qp[g][0] = qp_n[g][0];
            qp[g][1] = qp_n[g][1];
        }
        const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
        if (kh == 0) {
            sh_d[wave][lr] = d;
            sh_dm[wave][lr] = dmin;
        }
        if (sb + 1 < sb1) {  // prefetch the next super-block during this one's math
            JH_LOAD_X(sb + 1);
            JH_LOAD_W(sb + 1);
        }
        __syncthreads();

        // 6-bit scales and mins of the 8 sub-blocks (q4kScaleRaw / q4kMinRaw)
        int ls[8], lm[8];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ls[j] = (int)byte_of(hd.y, j) & 63;
            lm[j] = (int)byte_of(hd.z, j) & 63;
            ls[j + 4] = (int)((byte_of(hd.w, j) & 0x0F) | ((byte_of(hd.y, j) & 0xC0) >> 2));
            lm[j + 4] = (int)((byte_of(hd.w, j) >> 4) | ((byte_of(hd.z, j) & 0xC0) >> 2));
        }

        f32x16 acc[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) acc[n] = (f32x16){};
#pragma unroll
        for (int t = 0; t < 16; t++) {
            // K-step t covers sub-block s = t/2, elements 16*(t&1) + 8*kh .. +8
            const int s = t >> 1, g = s >> 1, hiN = s & 1;
            const u32x2 q = qp[g][t & 1];
            const uint32_t nib0 = hiN ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
            const uint32_t nib1 = hiN ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
            // pairs (e0,e1),(e2,e3),... as 16-bit lanes; then 0x6400 + ls*q per lane
            uint32_t pr[4];
            pr[0] = __builtin_amdgcn_perm(0u, nib0, 0x0C010C00u);  // e0 | e1 << 16
            pr[1] = __builtin_amdgcn_perm(0u, nib0, 0x0C030C02u);
            pr[2] = __builtin_amdgcn_perm(0u, nib1, 0x0C010C00u);
            pr[3] = __builtin_amdgcn_perm(0u, nib1, 0x0C030C02u);
            half8 a;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t v = __umul24(pr[j], (uint32_t)ls[s]) + 0x64006400u;
                a[2 * j] = __builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFF));
                a[2 * j + 1] = __builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
            }
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int col = n * 32 + lr;
                const half8 bh = *reinterpret_cast<const half8 *>(sh_hi + col * COLH + 16 * t + 8 * kh);
                const half8 bl = *reinterpret_cast<const half8 *>(sh_lo + col * COLH + 16 * t + 8 * kh);
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, acc[n], 0, 0, 0);
                acc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, acc[n], 0, 0, 0);
            }
        }
        // min term: sum_s lm_s * xsum_s, with [lm | lm] x [xsum_hi ; xsum_lo]
        half8 am;
#pragma unroll
        for (int j = 0; j < 8; j++) am[j] = (_Float16)lm[j];
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int col = n * 32 + lr;
            const half8 bm = *reinterpret_cast<const half8 *>(sh_xs + col * 16 + 8 * kh);
            const f32x16 mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, (f32x16){}, 0, 0, 0);
            const float S1024 = 1024.f * sh_S[col];
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const float4 dd = *reinterpret_cast<const float4 *>(&sh_d[wave][q4 * 8 + 4 * kh]);
                const float4 dm = *reinterpret_cast<const float4 *>(&sh_dm[wave][q4 * 8 + 4 * kh]);
                const float dv[4] = {dd.x, dd.y, dd.z, dd.w}, mv[4] = {dm.x, dm.y, dm.z, dm.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int i = q4 * 4 + k;
                    tot[n][i] = fmaf(dv[k], acc[n][i] - S1024, fmaf(-mv[k], mn[i], tot[n][i]));
                }
            }
        }
    }

#undef JH_LOAD_X
#undef JH_LOAD_W

    // results, scaled back by the column's power of two
    const int ksplit = gridDim.y;
    if (ksplit == 1) {
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int col = n * 32 + lr;
            if (col >= B) continue;
            const float cs = xw.scale()[col];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int r = rbase + (i >> 2) * 8 + 4 * kh + (i & 3);
                if (r < nrows) Y[(size_t)col * nrows + r] = tot[n][i] * cs;
            }
        }
        return;
    }
    // split K: each split writes its partial tile; reduce_splits adds them in
    // split order (deterministic).  A cross-workgroup hand-off inside this
    // kernel would need a device-scope release per workgroup, which on a
    // multi-XCD part writes back the whole L2 each time (~100 us measured).
    float *part = xw.part() + (size_t)blockIdx.y * B * nrows;
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int col = n * 32 + lr;
        if (col >= B) continue;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = rbase + (i >> 2) * 8 + 4 * kh + (i & 3);
            if (r < nrows) part[(size_t)col * nrows + r] = tot[n][i];
        }
    }
}

// y[c][r] = scale[c] * sum over splits k (in order) of part[k][c][r]
__global__ __launch_bounds__(256) void reduce_splits(XWork xw, int B, int nrows, int ksplit, float *__restrict__ Y) {
    const size_t n = (size_t)B * nrows;
    const float *p = xw.part();
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float v = 0.f;
        for (int k = 0; k < ksplit; k++) v += p[(size_t)k * n + i];
        Y[i] = v * xw.scale()[i / nrows];
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
    if (type != 12 || B < 16 || B > 64 || cols % 256 || rows < 1) return 0;
    int tiles, ksplit, ksb;
    mfma_split(rows, cols / 256, tiles, ksplit, ksb);
    XWork w{(B + 31) / 32 * 32, cols, cols / 256, rows, ksplit, nullptr};
    return w.bytes();
}

hipError_t launch_gemm_mfma_ws(const GemvArgs &a, void *workspace, hipStream_t s) {
    if (a.type != 12 || a.batch < 16 || a.batch > 64 || a.cols % 256) return hipErrorNotSupported;
    const int B = a.batch, Bp = (B + 31) / 32 * 32;
    const int nrows = a.row_end - a.row_start;
    const int nsb = a.cols / 256;
    int tiles, ksplit, ksb;
    mfma_split(nrows, nsb, tiles, ksplit, ksb);
    XWork w{Bp, a.cols, nsb, nrows, ksplit, reinterpret_cast<uint8_t *>(workspace)};
    x_prep_mfma<<<Bp, 256, 0, s>>>(a.x, B, w);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    dim3 grid(tiles, ksplit);
    if (Bp == 32)
        mfma_q4k<1><<<grid, 256, 0, s>>>(a.w, a.pitch, a.row_start, nrows, nsb, ksb, w, a.y, B);
    else
        mfma_q4k<2><<<grid, 256, 0, s>>>(a.w, a.pitch, a.row_start, nrows, nsb, ksb, w, a.y, B);
    e = hipGetLastError();
    if (e != hipSuccess || ksplit == 1) return e;
    const size_t n = (size_t)B * nrows;
    reduce_splits<<<(unsigned)std::min<size_t>((n + 255) / 256, 2048), 256, 0, s>>>(w, B, nrows, ksplit, a.y);
    return hipGetLastError();
}

}  // namespace jh
