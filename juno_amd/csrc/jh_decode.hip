// jh_decode.hip -- the rest of a Llama decode step on the device, around the
// quantized GEMVs: RMS normalisation (fused with the residual add), rotary
// embeddings with the KV-cache append (alone, or fused into attention),
// grouped-query attention over the cache, and the SwiGLU product.  Each kernel restates one method of
// LlamaTransformerHandler (citations per kernel) with the reference's
// precision choices: fp32 data, double where the reference computes in double
// (the rsqrt argument, rope's frequency / angle / cos / sin, softmax's and
// silu's exp, each cast to float as the reference casts it).  Parallel sums
// change only the order of fp32 summation.
//
// The decode position is read from device memory (const int *d_pos), so a
// captured HIP graph of a whole step can be replayed step after step with the
// position advanced on the device (pos_increment).
#include <math.h>
#include <stdlib.h>

#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {
namespace {

// ------------------------------------------------------------------ rmsNorm (+ residual)
// rmsNorm, LlamaTransformerHandler.java:818-826; the residual add of
// transformerLayer (:778, :783) is fused in front: v = x + res, x_out = v.
constexpr int kNormThreads = 1024;

// x_out may alias x (in-place residual); out must not alias x or x_out.  One
// workgroup per row of [rows][n] (a batch of requests).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_k(const float *x, const float *__restrict__ res,
                                                         const float *__restrict__ w, int n, float eps, float *x_out,
                                                         float *__restrict__ out) {
    __shared__ float part[kNormThreads / 64];
    const size_t row = (size_t)blockIdx.x * n;
    x += row;
    if (res) res += row;
    if (x_out) x_out += row;
    out += row;
    // up to kKeep values per thread stay in registers across the reduction (rows
    // up to 8192); wider rows re-read them
    constexpr int kKeep = 8;
    float keep[kKeep];
    float ss = 0.f;
    // every load of the thread's values first (addresses clamped in range), so
    // that they are in flight together rather than one per branch
    float xr[kKeep], rr[kKeep];
#pragma unroll
    for (int k = 0; k < kKeep; k++) {
        const int i = min(threadIdx.x + k * kNormThreads, n - 1);
        xr[k] = x[i];
        rr[k] = res ? res[i] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kKeep; k++) {
        const int i = threadIdx.x + k * kNormThreads;
        float v = 0.f;
        if (i < n) {
            v = res ? xr[k] + rr[k] : xr[k];
            if (x_out) x_out[i] = v;
        }
        keep[k] = v;
        ss += v * v;
    }
    for (int i = threadIdx.x + kKeep * kNormThreads; i < n; i += kNormThreads) {
        const float v = res ? x[i] + res[i] : x[i];
        if (x_out) x_out[i] = v;
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < kNormThreads / 64; k++) tot += part[k];
    const float scale = 1.f / (float)sqrt((double)(tot / (float)n + eps));
#pragma unroll
    for (int k = 0; k < kKeep; k++) {
        const int i = threadIdx.x + k * kNormThreads;
        if (i < n) out[i] = w[i] * keep[k] * scale;
    }
    for (int i = threadIdx.x + kKeep * kNormThreads; i < n; i += kNormThreads) {  // x_out[i] is this thread's
        const float v = x_out ? x_out[i] : (res ? x[i] + res[i] : x[i]);
        out[i] = w[i] * v * scale;
    }
}

// ------------------------------------------------------------------ rope + KV append
// rope, LlamaTransformerHandler.java:1657-1671 (adjacent pairs), applied to q
// in place and to k, and the cache stores of transformerLayer :769-770.
__global__ __launch_bounds__(256) void rope_kv_k(float *__restrict__ q, const float *__restrict__ k,
                                                 const float *__restrict__ v, int n_heads, int n_kv_heads,
                                                 int head_dim, const int *__restrict__ d_pos, int max_seq, float theta,
                                                 float *__restrict__ k_cache, float *__restrict__ v_cache) {
    const int pos = min(*d_pos, max_seq - 1);
    const int half = head_dim / 2, kv_dim = n_kv_heads * head_dim;
    const int nq = n_heads * half, nk = n_kv_heads * half;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < nq + nk) {
        const bool isq = i < nq;
        const int pi = isq ? i : i - nq;     // pair index within q or k
        const int h = pi / half, p = pi % half;
        const double freq = 1.0 / pow((double)theta, (2.0 * p) / head_dim);
        const double angle = pos * freq;
        const float c = (float)cos(angle), s = (float)sin(angle);
        const int o = h * head_dim + 2 * p;
        const float x0 = isq ? q[o] : k[o], x1 = isq ? q[o + 1] : k[o + 1];
        const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        if (isq) {
            q[o] = y0;
            q[o + 1] = y1;
        } else {
            k_cache[(size_t)pos * kv_dim + o] = y0;
            k_cache[(size_t)pos * kv_dim + o + 1] = y1;
        }
    } else if (i < nq + nk + kv_dim) {
        const int j = i - nq - nk;
        v_cache[(size_t)pos * kv_dim + j] = v[j];
    }
}

// ------------------------------------------------------------------ gqa
// gqa, LlamaTransformerHandler.java:1678-1715, with softmax :1718-1731.
// Split over the sequence: one wavefront per (query head h, chunk c of 64
// positions; 32 for head_dim > 128).  The chunk's K and V rows are staged in
// LDS with coalesced 16-byte loads; then one position per lane for the
// scores and one output dimension per lane (per 64) for the weighted V sum.
// It writes the chunk's max score m, sum of exp(s - m) l and sum of
// exp(s - m) v; attn_combine_k rescales the chunks to the global max and
// normalises.  Each dot product q . k runs over d in order, as the reference's.
//
// FUSED: q, k, v are the raw projections of this position; the kernel applies
// rope (:765-766) to q (per wavefront) and k, and the wavefronts whose chunk
// holds the position append rotated k and v to the cache (:769-770; the R
// wavefronts of a KV head write identical values) and use them from LDS.
__device__ __forceinline__ void rope_pair(float &x0, float &x1, int p, int head_dim, int pos, float theta) {
    const double freq = 1.0 / pow((double)theta, (2.0 * p) / head_dim);
    const double angle = pos * freq;
    const float c = (float)cos(angle), s = (float)sin(angle);
    const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
    x0 = y0;
    x1 = y1;
}

// rope_pair's rotation with its (cos, sin) already formed
__device__ __forceinline__ void rope_rot(float &x0, float &x1, float c, float s) {
    const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
    x0 = y0;
    x1 = y1;
}

// chunk length: one position per lane, fewer for wide heads (LDS holds the
// chunk's K and V)
__host__ __device__ constexpr int attn_tc(int head_dim) { return head_dim <= 128 ? 64 : 32; }
constexpr int kAttnSmallTc = 32;  // chunk of the one-round kernel when the grid is small

constexpr int kAttnWaves = 4;  // most waves per workgroup; they share the chunk's K and V

// Split-sequence attention (gqa, LlamaTransformerHandler.java:1678-1731): one
// workgroup per (KV head g, chunk c of tc positions, request z) stages the
// chunk's K and V rows of head g in LDS once; its waves then take the query
// heads h = g*R .. g*R+R-1 that share them (GQA), each writing the chunk's
// (max score, sum of exp, sum of exp * v) for the combine kernel.  With FUSED,
// rope (:1657-1671) is applied to q and to the new k, and the new k and v row
// is appended to the cache at pos (transformerLayer :765-770) by the chunk that
// holds pos, once per KV head.
template <bool FUSED>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_chunk_k(
    const float *__restrict__ q, const float *__restrict__ k_new, const float *__restrict__ v_new,
    float *__restrict__ k_cache, float *__restrict__ v_cache, int n_heads, int n_kv_heads, int head_dim,
    const int *__restrict__ d_pos, int max_seq, float theta, float scale, float *__restrict__ part,
    const int *__restrict__ d_slot, int n_slots) {
    extern __shared__ float lds[];
    const int tc = attn_tc(head_dim), kst = head_dim + 1;  // padded K rows: lane t in its own bank
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    float *sk = lds;                          // [tc][head_dim + 1]
    float *sv = sk + tc * kst;                // [tc][head_dim]
    float *sq = sv + tc * head_dim + wave * (head_dim + tc);  // this wave's [head_dim] q, then [tc] weights
    float *sp = sq + head_dim;
    // request z of a batch: its q / k / v rows, position, cache slot and partials
    const int z = blockIdx.z, kv_dim = n_kv_heads * head_dim;
    q += (size_t)z * n_heads * head_dim;
    if (FUSED) {
        k_new += (size_t)z * kv_dim;
        v_new += (size_t)z * kv_dim;
    }
    {
        const size_t cb = d_slot ? (size_t)min(max(d_slot[z], 0), n_slots - 1) * max_seq * kv_dim : 0;
        k_cache += cb;
        v_cache += cb;
    }
    part += (size_t)z * n_heads * gridDim.y * (head_dim + 2);
    const int pos = min(d_pos[z], max_seq - 1), T = pos + 1;
    const int g = blockIdx.x, c = blockIdx.y, t0 = c * tc;
    if (t0 >= T) return;  // uniform across the workgroup
    const int R = n_heads / n_kv_heads;
    const int nt = min(tc, T - t0);
    const bool has_pos = FUSED && pos < t0 + tc;  // this chunk holds the new position
    // the chunk's K and V rows of head g (cache positions; the new one is written below)
    const int q4 = head_dim / 4, n4 = nt * q4;
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
        const int t = i / q4, d = 4 * (i % q4);
        if (has_pos && t0 + t == pos) continue;
        const size_t o = (size_t)(t0 + t) * kv_dim + g * head_dim + d;
        const float4 kk = *reinterpret_cast<const float4 *>(k_cache + o);
        const float4 vv = *reinterpret_cast<const float4 *>(v_cache + o);
        float *kd = sk + t * kst + d;
        kd[0] = kk.x; kd[1] = kk.y; kd[2] = kk.z; kd[3] = kk.w;
        *reinterpret_cast<float4 *>(sv + t * head_dim + d) = vv;
    }
    if (has_pos) {
        const int tp = pos - t0;
        for (int p = threadIdx.x; p < head_dim / 2; p += blockDim.x) {
            float ka = k_new[g * head_dim + 2 * p], kb = k_new[g * head_dim + 2 * p + 1];
            rope_pair(ka, kb, p, head_dim, pos, theta);
            sk[tp * kst + 2 * p] = ka;
            sk[tp * kst + 2 * p + 1] = kb;
            const size_t o = (size_t)pos * kv_dim + g * head_dim + 2 * p;
            k_cache[o] = ka;
            k_cache[o + 1] = kb;
        }
        for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
            const float v = v_new[g * head_dim + d];
            sv[tp * head_dim + d] = v;
            v_cache[(size_t)pos * kv_dim + g * head_dim + d] = v;
        }
    }
    __syncthreads();
    for (int r = wave; r < R; r += nw) {  // wave-uniform
        const int h = g * R + r;
        for (int p = lane; p < head_dim / 2; p += 64) {
            float a = q[h * head_dim + 2 * p], b = q[h * head_dim + 2 * p + 1];
            if (FUSED) rope_pair(a, b, p, head_dim, pos, theta);
            sq[2 * p] = a;
            sq[2 * p + 1] = b;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float s = -INFINITY;
        if (lane < nt) {
            float dot = 0.f;
            for (int d = 0; d < head_dim; d++) dot += sq[d] * sk[lane * kst + d];
            s = dot * scale;
        }
        float m = s;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float e = lane < nt ? (float)exp((double)(s - m)) : 0.f;
        const float l = wave_sum(e);
        if (lane < tc) sp[lane] = e;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float *ph = part + ((size_t)h * gridDim.y + c) * (head_dim + 2);
        for (int d = lane; d < head_dim; d += 64) {
            float o = 0.f;
            for (int t = 0; t < nt; t++) o += sp[t] * sv[t * head_dim + d];
            ph[2 + d] = o;
        }
        if (lane == 0) {
            ph[0] = m;
            ph[1] = l;
        }
        // sq / sp are rewritten by this wave's next head
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// attn_chunk_k for head_dim HD in {64, 128} (Llama, TinyLlama, Qwen2): the
// same work split and results up to summation order, with the per-lane loops
// unrolled into independent chains.  K rows sit in LDS as float4 slots,
// XOR-swizzled per row (slot j of row t at j ^ (t mod HD/4)), so that a lane
// reads its row 16 bytes at a time and the 16 lanes of an LDS pass hit distinct
// banks; q . k runs in four accumulators.  For p . V each lane owns HD / 64
// adjacent output dims and alternates two accumulators over positions.
template <bool FUSED, int HD, bool VG>  // VG: p . V reads V from the cache (global) instead of LDS
__global__ __launch_bounds__(64 * kAttnWaves) void attn_chunk_hd(
    const float *__restrict__ q, const float *__restrict__ k_new, const float *__restrict__ v_new,
    float *__restrict__ k_cache, float *__restrict__ v_cache, int n_heads, int n_kv_heads, const int *__restrict__ d_pos,
    int max_seq, float theta, float scale, float *__restrict__ part, const int *__restrict__ d_slot, int n_slots) {
    constexpr int tc = attn_tc(HD), Q4 = HD / 4, M = Q4 - 1, DPL = HD / 64;
    extern __shared__ float lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    float4 *sk4 = reinterpret_cast<float4 *>(lds);  // [tc][Q4] swizzled
    float *sv = lds + tc * HD;                        // [tc][HD] (not with VG)
    float *srope = sv + (VG ? 0 : tc * HD);           // [HD / 2] (cos, sin) of this request's position
    float *sq = srope + HD + wave * (HD + tc);        // this wave's [HD] q, then [tc] weights
    float *sp = sq + HD;
    const int z = blockIdx.z, kv_dim = n_kv_heads * HD;
    q += (size_t)z * n_heads * HD;
    if (FUSED) {
        k_new += (size_t)z * kv_dim;
        v_new += (size_t)z * kv_dim;
    }
    {
        const size_t cb = d_slot ? (size_t)min(max(d_slot[z], 0), n_slots - 1) * max_seq * kv_dim : 0;
        k_cache += cb;
        v_cache += cb;
    }
    part += (size_t)z * n_heads * gridDim.y * (HD + 2);
    const int pos = min(d_pos[z], max_seq - 1), T = pos + 1;
    const int g = blockIdx.x, c = blockIdx.y, t0 = c * tc;
    if (t0 >= T) return;  // uniform across the workgroup
    const int R = n_heads / n_kv_heads;
    const int nt = min(tc, T - t0);
    const bool has_pos = FUSED && pos < t0 + tc;
    // four rows' loads in flight per thread before any is written (rows past
    // the chunk's end or the cache are clamped for the load and not written)
    for (int base = 0; base < nt * Q4; base += 4 * (int)blockDim.x) {
        float4 kk[4], vv[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + u * blockDim.x + threadIdx.x, t = i / Q4, j = i % Q4;
            const size_t o = (size_t)min(t0 + t, T - 1) * kv_dim + g * HD + 4 * j;
            kk[u] = *reinterpret_cast<const float4 *>(k_cache + o);
            if (!VG) vv[u] = *reinterpret_cast<const float4 *>(v_cache + o);
        }
        // rope's (cos, sin) for this position, once per workgroup, while the first loads are in flight
        // (rope_pair's arithmetic: the same values)
        if (FUSED && base == 0 && threadIdx.x < HD / 2) {
            const int pp = threadIdx.x;
            const double freq = 1.0 / pow((double)theta, (2.0 * pp) / HD);
            const double angle = pos * freq;
            srope[2 * pp] = (float)cos(angle);
            srope[2 * pp + 1] = (float)sin(angle);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = base + u * blockDim.x + threadIdx.x, t = i / Q4, j = i % Q4;
            if (t >= nt || (has_pos && t0 + t == pos)) continue;
            sk4[t * Q4 + (j ^ (t & M))] = kk[u];
            if (!VG) *reinterpret_cast<float4 *>(sv + t * HD + 4 * j) = vv[u];
        }
    }
    if (has_pos) {
        const int tp = pos - t0;
        float *skf = reinterpret_cast<float *>(sk4);
        for (int p = threadIdx.x; p < HD / 2; p += blockDim.x) {  // thread p wrote pair p of the table
            float ka = k_new[g * HD + 2 * p], kb = k_new[g * HD + 2 * p + 1];
            rope_rot(ka, kb, srope[2 * p], srope[2 * p + 1]);
            const int d = 2 * p, slot = tp * Q4 + ((d >> 2) ^ (tp & M));
            skf[4 * slot + (d & 3)] = ka;
            skf[4 * slot + (d & 3) + 1] = kb;
            const size_t o = (size_t)pos * kv_dim + g * HD + 2 * p;
            k_cache[o] = ka;
            k_cache[o + 1] = kb;
        }
        for (int d = threadIdx.x; d < HD; d += blockDim.x) {
            const float v = v_new[g * HD + d];
            if (!VG) sv[tp * HD + d] = v;
            v_cache[(size_t)pos * kv_dim + g * HD + d] = v;  // VG: read back below, after the barrier
        }
    }
    __syncthreads();
    for (int r = wave; r < R; r += nw) {  // wave-uniform
        const int h = g * R + r;
        for (int p = lane; p < HD / 2; p += 64) {
            float a = q[h * HD + 2 * p], b = q[h * HD + 2 * p + 1];
            if (FUSED) rope_rot(a, b, srope[2 * p], srope[2 * p + 1]);
            sq[2 * p] = a;
            sq[2 * p + 1] = b;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lanes past the chunk's end compute on whatever row lane holds and are masked
        const float4 *q4 = reinterpret_cast<const float4 *>(sq);
        const float4 *k4 = sk4 + lane * Q4;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int j = 0; j < Q4; j++) {
            const float4 qq = q4[j], kk = k4[j ^ (lane & M)];
            a0 = fmaf(qq.x, kk.x, a0);
            a1 = fmaf(qq.y, kk.y, a1);
            a2 = fmaf(qq.z, kk.z, a2);
            a3 = fmaf(qq.w, kk.w, a3);
        }
        const float s = lane < nt ? ((a0 + a1) + (a2 + a3)) * scale : -INFINITY;
        float m = s;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float e = lane < nt ? (float)exp((double)(s - m)) : 0.f;
        const float l = wave_sum(e);
        if (lane < tc) sp[lane] = e;  // one weight per position (0 past the chunk's end)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float oe[DPL], oo[DPL];
#pragma unroll
        for (int i = 0; i < DPL; i++) oe[i] = oo[i] = 0.f;
        // V rows: LDS, or the cache rows t0 .. of head g (lanes read adjacent dims: coalesced)
        const float *vcol = VG ? v_cache + (size_t)t0 * kv_dim + g * HD + DPL * lane : sv + DPL * lane;
        const int vst = VG ? kv_dim : HD;
        int t = 0;
        if (VG) {  // eight rows' loads in flight before their FMAs (global latency)
            for (; t + 7 < nt; t += 8) {
                float vv[8][DPL];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int i = 0; i < DPL; i++) vv[u][i] = vcol[(size_t)(t + u) * vst + i];
#pragma unroll
                for (int u = 0; u < 8; u += 2)
#pragma unroll
                    for (int i = 0; i < DPL; i++) {
                        oe[i] = fmaf(sp[t + u], vv[u][i], oe[i]);
                        oo[i] = fmaf(sp[t + u + 1], vv[u + 1][i], oo[i]);
                    }
            }
        }
        for (; t + 1 < nt; t += 2) {
            const float pe = sp[t], po = sp[t + 1];
#pragma unroll
            for (int i = 0; i < DPL; i++) {
                oe[i] = fmaf(pe, vcol[(size_t)t * vst + i], oe[i]);
                oo[i] = fmaf(po, vcol[(size_t)(t + 1) * vst + i], oo[i]);
            }
        }
        if (t < nt) {
            const float pe = sp[t];
#pragma unroll
            for (int i = 0; i < DPL; i++) oe[i] = fmaf(pe, vcol[(size_t)t * vst + i], oe[i]);
        }
        float *ph = part + ((size_t)h * gridDim.y + c) * (HD + 2);
#pragma unroll
        for (int i = 0; i < DPL; i++) ph[2 + DPL * lane + i] = oe[i] + oo[i];
        if (lane == 0) {
            ph[0] = m;
            ph[1] = l;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// One chunk of tc positions for all R query heads of a KV group, with K and V
// each read once per workgroup and every load issued before the first wait:
//  * K goes through LDS (as attn_chunk_hd: swizzled float4 rows, lane = row
//    for q . k); V stays in registers, thread (d4, ph) holding dims 4 d4 .. +4
//    of rows ph, ph + PH, ...;
//  * q . k and the softmax weights run one head per wave (waves loop over
//    the group's heads), the weights of all heads meeting in LDS;
//  * p . V: each thread folds its V rows into R float4 accumulators (one per
//    head), the PH row phases are summed through LDS (the K buffer, free by
//    then) in phase order.
// The new position's K (roped) and V replace the cache rows in LDS and in the
// registers and are written to the cache.  Results match attn_chunk_k up to
// the summation order of p . V.
template <bool FUSED, int HD, int R, int TC>  // TC: positions per chunk (64, or 32 for a grid of few chunks)
__global__ __launch_bounds__(256) void attn_chunk_rv(
    const float *__restrict__ q, const float *__restrict__ k_new, const float *__restrict__ v_new,
    float *__restrict__ k_cache, float *__restrict__ v_cache, int n_heads, int n_kv_heads, const int *__restrict__ d_pos,
    int max_seq, float theta, float scale, float *__restrict__ part, const int *__restrict__ d_slot, int n_slots) {
    constexpr int tc = TC, Q4 = HD / 4, M = Q4 - 1;
    constexpr int PH = 256 / Q4;         // row phases of p . V
    constexpr int VJ = tc / PH;          // V rows per thread
    constexpr int KJ = tc * Q4 / 256;    // K float4 per thread
    constexpr int KR = tc * HD > PH * R * HD ? tc * HD : PH * R * HD;  // floats: K rows, later the phase sums
    extern __shared__ float lds[];
    float4 *sk4 = reinterpret_cast<float4 *>(lds);  // [tc][Q4] swizzled
    float *red = lds;                               // [PH][R][HD] after q . k
    float *srope = lds + KR;                        // [HD / 2] (cos, sin)
    float *sq = srope + HD;                         // [R][HD]
    float *sp = sq + R * HD;                        // [R][tc]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int z = blockIdx.z, kv_dim = n_kv_heads * HD;
    q += (size_t)z * n_heads * HD;
    if (FUSED) {
        k_new += (size_t)z * kv_dim;
        v_new += (size_t)z * kv_dim;
    }
    {
        const size_t cb = d_slot ? (size_t)min(max(d_slot[z], 0), n_slots - 1) * max_seq * kv_dim : 0;
        k_cache += cb;
        v_cache += cb;
    }
    part += (size_t)z * n_heads * gridDim.y * (HD + 2);
    const int pos = min(d_pos[z], max_seq - 1), T = pos + 1;
    const int g = blockIdx.x, c = blockIdx.y, t0 = c * tc;
    if (t0 >= T) return;  // uniform across the workgroup
    const int nt = min(tc, T - t0);
    const bool has_pos = FUSED && pos < t0 + tc;
    // every K and V load of the chunk in flight at once (rows past the end clamped)
    float4 kk[KJ], vv[VJ];
#pragma unroll
    for (int u = 0; u < KJ; u++) {
        const int i = u * 256 + tid, t = i / Q4, j = i % Q4;
        kk[u] = *reinterpret_cast<const float4 *>(k_cache + (size_t)min(t0 + t, T - 1) * kv_dim + g * HD + 4 * j);
    }
    const int d4 = tid % Q4, ph = tid / Q4;
#pragma unroll
    for (int u = 0; u < VJ; u++) {
        const int t = ph + PH * u;
        vv[u] = *reinterpret_cast<const float4 *>(v_cache + (size_t)min(t0 + t, T - 1) * kv_dim + g * HD + 4 * d4);
    }
    if (FUSED) {  // rope's (cos, sin) for this position (rope_pair's arithmetic), while the loads fly
        // every thread computes (no branch for the loads above to sink into); the first HD / 2 store
        const int pp = tid & (HD / 2 - 1);
        const double freq = 1.0 / pow((double)theta, (2.0 * pp) / HD);
        const double angle = pos * freq;
        const float cs = (float)cos(angle), sn = (float)sin(angle);
        if (tid < HD / 2) {
            srope[2 * pp] = cs;
            srope[2 * pp + 1] = sn;
        }
    }
    // every thread stores every row it loaded (rows past the chunk's end and the
    // new position's row go to a dummy slot): a conditional store would let the
    // compiler sink each load into its branch and wait for them one by one
    float4 *sdummy = reinterpret_cast<float4 *>(sp + R * tc);
#pragma unroll
    for (int u = 0; u < KJ; u++) {
        const int i = u * 256 + tid, t = i / Q4, j = i % Q4;
        const bool keep = t < nt && !(has_pos && t0 + t == pos);
        *(keep ? sk4 + t * Q4 + (j ^ (t & M)) : sdummy) = kk[u];
    }
    if (has_pos) {
        const int tp = pos - t0;
        float *skf = reinterpret_cast<float *>(sk4);
        if (tid < HD / 2) {  // thread tid wrote pair tid of the table
            const int p = tid;
            float ka = k_new[g * HD + 2 * p], kb = k_new[g * HD + 2 * p + 1];
            rope_rot(ka, kb, srope[2 * p], srope[2 * p + 1]);
            const int d = 2 * p, slot = tp * Q4 + ((d >> 2) ^ (tp & M));
            skf[4 * slot + (d & 3)] = ka;
            skf[4 * slot + (d & 3) + 1] = kb;
            const size_t o = (size_t)pos * kv_dim + g * HD + 2 * p;
            k_cache[o] = ka;
            k_cache[o + 1] = kb;
        }
        if (tid < Q4)
            *reinterpret_cast<float4 *>(v_cache + (size_t)pos * kv_dim + g * HD + 4 * tid) =
                *reinterpret_cast<const float4 *>(v_new + g * HD + 4 * tid);
#pragma unroll
        for (int u = 0; u < VJ; u++)
            if (ph + PH * u == tp) vv[u] = *reinterpret_cast<const float4 *>(v_new + g * HD + 4 * d4);
    }
    __syncthreads();
    for (int r = wave; r < R; r += 4) {  // wave-uniform
        const int h = g * R + r;
        float *sqr = sq + r * HD;
        for (int p = lane; p < HD / 2; p += 64) {
            float a = q[h * HD + 2 * p], b = q[h * HD + 2 * p + 1];
            if (FUSED) rope_rot(a, b, srope[2 * p], srope[2 * p + 1]);
            sqr[2 * p] = a;
            sqr[2 * p + 1] = b;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lanes past the chunk's end compute on whatever row they hold and are masked
        const float4 *q4 = reinterpret_cast<const float4 *>(sqr);
        const int kr = min(lane, tc - 1);  // lanes past the chunk read its last row (masked below)
        const float4 *k4 = sk4 + kr * Q4;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int j = 0; j < Q4; j++) {
            const float4 qq = q4[j], kq = k4[j ^ (kr & M)];
            a0 = fmaf(qq.x, kq.x, a0);
            a1 = fmaf(qq.y, kq.y, a1);
            a2 = fmaf(qq.z, kq.z, a2);
            a3 = fmaf(qq.w, kq.w, a3);
        }
        const float sc = lane < nt ? ((a0 + a1) + (a2 + a3)) * scale : -INFINITY;
        float m = sc;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const float e = lane < nt ? (float)exp((double)(sc - m)) : 0.f;
        const float l = wave_sum(e);
        if (lane < tc) sp[r * tc + lane] = e;  // one weight per position (0 past the chunk's end)
        if (lane == 0) {
            float *hp = part + ((size_t)h * gridDim.y + c) * (HD + 2);
            hp[0] = m;
            hp[1] = l;
        }
    }
    __syncthreads();  // every head's weights are in LDS; K is no longer read
    float4 acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < VJ; u++) {
        const int t = ph + PH * u;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float pw = sp[r * tc + t];
            acc[r].x = fmaf(pw, vv[u].x, acc[r].x);
            acc[r].y = fmaf(pw, vv[u].y, acc[r].y);
            acc[r].z = fmaf(pw, vv[u].z, acc[r].z);
            acc[r].w = fmaf(pw, vv[u].w, acc[r].w);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) *reinterpret_cast<float4 *>(red + (ph * R + r) * HD + 4 * d4) = acc[r];
    __syncthreads();
    for (int i = tid; i < R * HD; i += 256) {
        const int r = i / HD, d = i % HD;
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < PH; k++) o += red[(k * R + r) * HD + d];
        part[((size_t)(g * R + r) * gridDim.y + c) * (HD + 2) + 2 + d] = o;
    }
}

template <int HD, int R, int TC>
constexpr size_t attn_rv_lds() {
    constexpr int tc = TC, PH = 256 / (HD / 4);
    constexpr int KR = tc * HD > PH * R * HD ? tc * HD : PH * R * HD;
    return sizeof(float) * (KR + HD + R * HD + R * tc + 4);
}

__global__ __launch_bounds__(256) void attn_combine_k(const float *__restrict__ part, int head_dim, int tc,
                                                      const int *__restrict__ d_pos, int max_seq, int nchmax,
                                                      float *__restrict__ out) {
    // The chunk maxima and normalisers are loaded by one thread per chunk, all at
    // once; the sums over chunks then run in chunk order from LDS (L) or with
    // eight chunks' loads in flight (o), so that the arithmetic is the plain
    // sequential one without a memory round trip per chunk.
    __shared__ float wc[1024], wl[1024], wmax[4];
    __shared__ float sL;
    const int h = blockIdx.x, z = blockIdx.y;  // head, request
    const int tid = threadIdx.x;
    d_pos += z;
    part += (size_t)z * gridDim.x * nchmax * (head_dim + 2);
    out += (size_t)z * gridDim.x * head_dim;
    const int T = min(*d_pos, max_seq - 1) + 1, nch = min((T + tc - 1) / tc, 1024);
    const float *ph = part + (size_t)h * nchmax * (head_dim + 2);
    // the first kPre chunks' o of this thread's first dimension, loaded now: they
    // do not depend on the weights, so their round trip overlaps the one of the
    // maxima instead of following it
    constexpr int kPre = 16;
    float opre[kPre];
#pragma unroll
    for (int u = 0; u < kPre; u++)
        opre[u] = (tid < head_dim && u < nch) ? ph[u * (head_dim + 2) + 2 + tid] : 0.f;
    float M = -INFINITY;
    for (int c = tid; c < nch; c += 256) {
        const float m = ph[c * (head_dim + 2)];
        wc[c] = m;
        wl[c] = ph[c * (head_dim + 2) + 1];
        M = fmaxf(M, m);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    if ((tid & 63) == 0) wmax[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));  // max: any order gives the same value
    for (int c = tid; c < nch; c += 256) wc[c] = (float)exp((double)(wc[c] - M));
    __syncthreads();
    if (tid == 0) {
        float L = 0.f;
        for (int c = 0; c < nch; c++) L = fmaf(wl[c], wc[c], L);
        sL = L;
    }
    __syncthreads();
    const float L = sL;
    for (int d = tid; d < head_dim; d += 256) {
        const float *op = ph + 2 + d;
        float o = 0.f;
        int c = 0;
        if (d == tid) {  // the prefetched chunks, in chunk order
#pragma unroll
            for (int u = 0; u < kPre; u++)
                if (u < nch) o = fmaf(opre[u], wc[u], o);
            c = min(nch, kPre);
        }
        for (; c + 8 <= nch; c += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = op[(c + u) * (head_dim + 2)];
#pragma unroll
            for (int u = 0; u < 8; u++) o = fmaf(v[u], wc[c + u], o);
        }
        for (; c < nch; c++) o = fmaf(op[c * (head_dim + 2)], wc[c], o);
        out[(size_t)h * head_dim + d] = o / L;
    }
}

// ------------------------------------------------------------------ SwiGLU
// silu, LlamaTransformerHandler.java:1733-1735, times up (ffn :796-797)
__global__ __launch_bounds__(256) void silu_mul_k(const float *__restrict__ gate, const float *__restrict__ up, int n,
                                                  float *__restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        out[i] = silu_times(g, up[i]);
    }
}

// ------------------------------------------------------------------ LoRA overlay
// LoraAdapter.forward (LoraAdapter.java:79-98): h = A x (A [rank][in]), then
// delta = (B h) * scale (B [out][rank]); applyLoraInPlace adds delta to the
// projection's output (LoraTrainableHandler.java:489-496).  One workgroup per
// (r, request) for h; one thread per (output row, request) for the update.
__global__ __launch_bounds__(256) void lora_down_k(const float *__restrict__ A, const float *__restrict__ x, int in_dim,
                                                   int rank, float *__restrict__ h) {
    __shared__ float part[4];
    const int r = blockIdx.x, b = blockIdx.y;
    const float *ar = A + (size_t)r * in_dim, *xb = x + (size_t)b * in_dim;
    float acc = 0.f;
    for (int c = threadIdx.x; c < in_dim; c += 256) acc += ar[c] * xb[c];
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) h[(size_t)b * rank + r] = (part[0] + part[1]) + (part[2] + part[3]);
}

__global__ __launch_bounds__(256) void lora_up_k(const float *__restrict__ B, const float *__restrict__ h, int rank,
                                                 int out_dim, float scale, float *__restrict__ y) {
    const int i = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
    if (i >= out_dim) return;
    const float *br = B + (size_t)i * rank, *hb = h + (size_t)b * rank;
    float acc = 0.f;
    for (int c = 0; c < rank; c++) acc += br[c] * hb[c];
    float *yp = y + (size_t)b * out_dim + i;
    *yp = *yp + acc * scale;
}

// addInPlace (LlamaTransformerHandler.java:1641-1646) on each of rows rows:
// y[r][i] += bias[i] (the Q / K / V projection biases, :758-761).
__global__ __launch_bounds__(256) void add_rows_k(float *__restrict__ y, const float *__restrict__ bias, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        float *yr = y + (size_t)blockIdx.y * n;
        yr[i] = yr[i] + bias[i];
    }
}

__global__ void pos_increment_k(int *d_pos, int delta) {
    if (threadIdx.x == 0) *d_pos += delta;
}

}  // namespace

hipError_t launch_rmsnorm(const float *x, const float *res, const float *w, int n, int rows, float eps, float *x_out,
                          float *out, hipStream_t s) {
    rmsnorm_k<<<rows, kNormThreads, 0, s>>>(x, res, w, n, eps, x_out, out);
    return hipGetLastError();
}

hipError_t launch_rope_kv(float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                          const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache,
                          hipStream_t s) {
    const int items = (n_heads + n_kv_heads) * (head_dim / 2) + n_kv_heads * head_dim;
    rope_kv_k<<<(items + 255) / 256, 256, 0, s>>>(q, k, v, n_heads, n_kv_heads, head_dim, d_pos, max_seq, theta,
                                                   k_cache, v_cache);
    return hipGetLastError();
}

// JUNO_ATTN_RV=0 selects the per-wave kernels (tuning runs)
static bool attn_rv_wanted() {
    static const bool on = [] {
        const char *v = getenv("JUNO_ATTN_RV");
        return !(v && v[0] == '0');
    }();
    return on;
}
// per-wave kernels: V read from the cache instead of LDS (measured at position
// 511, head_dim 128, B = 32: 48.2 -> 45.3 us; slower for head_dim 64, 20.6 ->
// 29.5 us, and at B = 1)
static bool attn_v_global(int head_dim, int batch) { return head_dim == 128 && batch >= 8; }

static bool attn_rv_applies(int n_heads, int n_kv_heads, int head_dim) {
    const int R = n_heads / n_kv_heads;
    return (head_dim == 64 || head_dim == 128) && (R == 1 || R == 2 || R == 4 || R == 8) && attn_rv_wanted();
}
// 32-position chunks when the grid would be small (one request): twice the workgroups, each half the rows
static bool attn_small_chunks(bool rv, int n_kv_heads, int max_seq, int batch) {
    return rv && (size_t)batch * n_kv_heads * ((max_seq + 63) / 64) < 512 &&
           (max_seq + kAttnSmallTc - 1) / kAttnSmallTc <= 1024;
}

void attention_chunking(int n_heads, int n_kv_heads, int head_dim, int max_seq, int batch, int *tc, int *nch) {
    const bool small = attn_small_chunks(attn_rv_applies(n_heads, n_kv_heads, head_dim), n_kv_heads, max_seq, batch);
    *tc = small ? kAttnSmallTc : attn_tc(head_dim);
    *nch = (max_seq + *tc - 1) / *tc;
}

size_t attention_workspace_bytes(int n_heads, int head_dim, int max_seq, int batch) {
    const int tc = head_dim <= 128 ? kAttnSmallTc : attn_tc(head_dim);  // the finest chunking the launcher may pick
    const int nch = (max_seq + tc - 1) / tc;
    return (size_t)batch * n_heads * nch * (head_dim + 2) * sizeof(float);
}

hipError_t launch_attention(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                            int n_heads, int n_kv_heads, int head_dim, const int *d_pos, int max_seq, float theta,
                            bool fused, float *out, void *workspace, hipStream_t s, int batch, const int *d_slot,
                            int n_slots, bool combine) {
    const int R = n_heads / n_kv_heads;
    const bool rv = attn_rv_applies(n_heads, n_kv_heads, head_dim);
    const bool small = attn_small_chunks(rv, n_kv_heads, max_seq, batch);
    const int tc = small ? kAttnSmallTc : attn_tc(head_dim), nch = (max_seq + tc - 1) / tc;
    if (nch > 1024) return hipErrorNotSupported;  // combine weights live in a fixed LDS array
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    float *part = static_cast<float *>(workspace);
    const dim3 grid(n_kv_heads, nch, batch);
    const int nw = min(n_heads / n_kv_heads, kAttnWaves);  // one wave per query head of a group, up to 4
    const size_t lds = sizeof(float) * ((size_t)tc * (head_dim + 1) + (size_t)tc * head_dim +
                                        (size_t)nw * (head_dim + tc));
    static const bool attr = [] {
        const void *fs[] = {reinterpret_cast<const void *>(&attn_chunk_k<true>),
                            reinterpret_cast<const void *>(&attn_chunk_k<false>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<true, 64, false>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<false, 64, false>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<true, 128, false>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<false, 128, false>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<true, 64, true>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<false, 64, true>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<true, 128, true>),
                            reinterpret_cast<const void *>(&attn_chunk_hd<false, 128, true>)};
        bool ok = true;
        for (const void *f : fs)
            ok = ok && hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        return ok;
    }();
    (void)attr;
    if (rv) {
        // (at most ~40 KB of LDS: within the default dynamic limit)
#define JH_RV_T(FU, HD, RR, T)                                                                                     \
    attn_chunk_rv<FU, HD, RR, T><<<grid, 256, attn_rv_lds<HD, RR, T>(), s>>>(                                       \
        q, FU ? k_new : nullptr, FU ? v_new : nullptr, k_cache, v_cache, n_heads, n_kv_heads, d_pos, max_seq, theta, \
        scale, part, d_slot, n_slots)
#define JH_RV(FU, HD, RR)                                                                                          \
    if (small) JH_RV_T(FU, HD, RR, kAttnSmallTc); else JH_RV_T(FU, HD, RR, 64)
#define JH_RV_R(FU, HD)                                                                                            \
    switch (R) {                                                                                                   \
    case 1: JH_RV(FU, HD, 1); break;                                                                               \
    case 2: JH_RV(FU, HD, 2); break;                                                                               \
    case 4: JH_RV(FU, HD, 4); break;                                                                               \
    default: JH_RV(FU, HD, 8); break;                                                                              \
    }
        if (head_dim == 64) {
            if (fused) { JH_RV_R(true, 64) } else { JH_RV_R(false, 64) }
        } else {
            if (fused) { JH_RV_R(true, 128) } else { JH_RV_R(false, 128) }
        }
#undef JH_RV_R
#undef JH_RV
#undef JH_RV_T
    } else if (head_dim == 64 || head_dim == 128) {
        // many workgroups (a batch): V is read from the cache, so that a workgroup's LDS holds only K and more of
        // them fit per CU
        const bool vg = attn_v_global(head_dim, batch);
        const size_t lds_hd =
            sizeof(float) * ((vg ? 1 : 2) * (size_t)tc * head_dim + head_dim + (size_t)nw * (head_dim + tc));
#define JH_ATT(FU, HD, VG)                                                                                    \
    attn_chunk_hd<FU, HD, VG><<<grid, 64 * nw, lds_hd, s>>>(q, FU ? k_new : nullptr, FU ? v_new : nullptr, k_cache,   \
                                                           v_cache, n_heads, n_kv_heads, d_pos, max_seq, theta, scale, \
                                                           part, d_slot, n_slots)
        if (head_dim == 64) {
            if (vg) {
                if (fused) JH_ATT(true, 64, true); else JH_ATT(false, 64, true);
            } else {
                if (fused) JH_ATT(true, 64, false); else JH_ATT(false, 64, false);
            }
        } else {
            if (vg) {
                if (fused) JH_ATT(true, 128, true); else JH_ATT(false, 128, true);
            } else {
                if (fused) JH_ATT(true, 128, false); else JH_ATT(false, 128, false);
            }
        }
#undef JH_ATT
    } else if (fused)
        attn_chunk_k<true><<<grid, 64 * nw, lds, s>>>(q, k_new, v_new, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos,
                                                max_seq, theta, scale, part, d_slot, n_slots);
    else
        attn_chunk_k<false><<<grid, 64 * nw, lds, s>>>(q, nullptr, nullptr, k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                                 d_pos, max_seq, theta, scale, part, d_slot, n_slots);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !combine) return e;
    attn_combine_k<<<dim3(n_heads, batch), 256, 0, s>>>(part, head_dim, tc, d_pos, max_seq, nch, out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gate, const float *up, int n, float *out, hipStream_t s) {
    silu_mul_k<<<(n + 255) / 256, 256, 0, s>>>(gate, up, n, out);
    return hipGetLastError();
}

hipError_t launch_lora(const float *a, const float *b, int rank, int in_dim, int out_dim, float scale, const float *x,
                       int batch, float *y, float *h_ws, hipStream_t s) {
    lora_down_k<<<dim3(rank, batch), 256, 0, s>>>(a, x, in_dim, rank, h_ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    lora_up_k<<<dim3((out_dim + 255) / 256, batch), 256, 0, s>>>(b, h_ws, rank, out_dim, scale, y);
    return hipGetLastError();
}

hipError_t launch_add_rows(float *y, const float *bias, int n, int rows, hipStream_t s) {
    add_rows_k<<<dim3((n + 255) / 256, rows), 256, 0, s>>>(y, bias, n);
    return hipGetLastError();
}

hipError_t launch_pos_increment(int *d_pos, int delta, hipStream_t s) {
    pos_increment_k<<<1, 64, 0, s>>>(d_pos, delta);
    return hipGetLastError();
}

}  // namespace jh
