// jh_decode.hip -- the rest of a Llama decode step on the device, around the
// quantized GEMVs: RMS normalisation (fused with the residual add), rotary
// embeddings fused with the KV-cache append, grouped-query attention over the
// cache, and the SwiGLU product.  Each kernel restates one method of
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

#include "jh_device.hpp"
#include "jh_kernels.hpp"

namespace jh {
namespace {

// ------------------------------------------------------------------ rmsNorm (+ residual)
// rmsNorm, LlamaTransformerHandler.java:818-826; the residual add of
// transformerLayer (:778, :783) is fused in front: v = x + res, x_out = v.
constexpr int kNormThreads = 1024;

// x_out may alias x (in-place residual); out must not alias x or x_out.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_k(const float *x, const float *__restrict__ res,
                                                         const float *__restrict__ w, int n, float eps, float *x_out,
                                                         float *__restrict__ out) {
    __shared__ float part[kNormThreads / 64];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kNormThreads) {
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
    for (int i = threadIdx.x; i < n; i += kNormThreads) {  // the same i as above: x_out[i] is this thread's
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
// Split over the sequence: workgroup (g, c) takes KV head g and positions
// [c*TC, c*TC + TC) for all R = n_heads / n_kv_heads query heads of g, with
// the chunk's K and V staged in LDS once.  It writes, per query head, the
// chunk's max score m, sum of exp(s - m) l, and sum of exp(s - m) v; the
// combine kernel rescales the chunks to the global max and normalises.
// Each dot product q . k runs over d in order, as the reference's does.
__global__ __launch_bounds__(256) void attn_chunk_k(const float *__restrict__ q, const float *__restrict__ k_cache,
                                                    const float *__restrict__ v_cache, int n_heads, int n_kv_heads,
                                                    int head_dim, const int *__restrict__ d_pos, int max_seq,
                                                    int tc, float scale, float *__restrict__ part) {
    extern __shared__ float lds[];
    const int T = min(*d_pos, max_seq - 1) + 1;
    const int g = blockIdx.x, c = blockIdx.y, t0 = c * tc;
    if (t0 >= T) return;  // uniform across the workgroup
    const int R = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim, nt = min(tc, T - t0);
    const int kst = head_dim + 1;  // padded K rows: consecutive positions in different banks
    float *sk = lds;                        // [tc][head_dim + 1]
    float *sv = sk + tc * kst;              // [tc][head_dim]
    float *sq = sv + tc * head_dim;         // [R][head_dim]
    float *sp = sq + R * head_dim;          // [R][tc]
    float *sm = sp + R * tc;                // [R] max, [R] sum
    for (int i = threadIdx.x; i < nt * head_dim; i += 256) {
        const int t = i / head_dim, d = i % head_dim;
        const size_t o = (size_t)(t0 + t) * kv_dim + g * head_dim + d;
        sk[t * kst + d] = k_cache[o];
        sv[t * head_dim + d] = v_cache[o];
    }
    for (int i = threadIdx.x; i < R * head_dim; i += 256) sq[i] = q[g * R * head_dim + i];
    __syncthreads();
    for (int i = threadIdx.x; i < R * nt; i += 256) {
        const int j = i / nt, t = i % nt;
        float dot = 0.f;
        for (int d = 0; d < head_dim; d++) dot += sq[j * head_dim + d] * sk[t * kst + d];
        sp[j * tc + t] = dot * scale;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int j = wave; j < R; j += 4) {
        float m = -INFINITY;
        for (int t = lane; t < nt; t += 64) m = fmaxf(m, sp[j * tc + t]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float l = 0.f;
        for (int t = lane; t < nt; t += 64) {
            const float e = (float)exp((double)(sp[j * tc + t] - m));
            sp[j * tc + t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            sm[j] = m;
            sm[R + j] = l;
        }
    }
    __syncthreads();
    const int nch = gridDim.y;
    for (int i = threadIdx.x; i < R * head_dim; i += 256) {
        const int j = i / head_dim, d = i % head_dim;
        float o = 0.f;
        for (int t = 0; t < nt; t++) o += sp[j * tc + t] * sv[t * head_dim + d];
        const int h = g * R + j;
        part[((size_t)h * nch + c) * (head_dim + 2) + 2 + d] = o;
    }
    if (threadIdx.x < R) {
        const int h = g * R + threadIdx.x;
        part[((size_t)h * nch + c) * (head_dim + 2)] = sm[threadIdx.x];
        part[((size_t)h * nch + c) * (head_dim + 2) + 1] = sm[R + threadIdx.x];
    }
}

__global__ __launch_bounds__(256) void attn_combine_k(const float *__restrict__ part, int head_dim,
                                                      const int *__restrict__ d_pos, int max_seq, int tc, int nchmax,
                                                      float *__restrict__ out) {
    const int h = blockIdx.x;
    const int T = min(*d_pos, max_seq - 1) + 1, nch = (T + tc - 1) / tc;
    const float *ph = part + (size_t)h * nchmax * (head_dim + 2);
    float M = -INFINITY;
    for (int c = 0; c < nch; c++) M = fmaxf(M, ph[c * (head_dim + 2)]);
    float L = 0.f;
    for (int c = 0; c < nch; c++) L += ph[c * (head_dim + 2) + 1] * (float)exp((double)(ph[c * (head_dim + 2)] - M));
    for (int d = threadIdx.x; d < head_dim; d += 256) {
        float o = 0.f;
        for (int c = 0; c < nch; c++)
            o += ph[c * (head_dim + 2) + 2 + d] * (float)exp((double)(ph[c * (head_dim + 2)] - M));
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
        out[i] = g / (1.f + (float)exp(-(double)g)) * up[i];
    }
}

__global__ void pos_increment_k(int *d_pos, int delta) {
    if (threadIdx.x == 0) *d_pos += delta;
}

}  // namespace

hipError_t launch_rmsnorm(const float *x, const float *res, const float *w, int n, float eps, float *x_out,
                          float *out, hipStream_t s) {
    rmsnorm_k<<<1, kNormThreads, 0, s>>>(x, res, w, n, eps, x_out, out);
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

int attention_chunk(int head_dim) { return head_dim >= 256 ? 32 : 8192 / head_dim; }

size_t attention_workspace_bytes(int n_heads, int head_dim, int max_seq) {
    const int tc = attention_chunk(head_dim), nch = (max_seq + tc - 1) / tc;
    return (size_t)n_heads * nch * (head_dim + 2) * sizeof(float);
}

size_t attention_lds_bytes(int n_heads, int n_kv_heads, int head_dim) {
    const int tc = attention_chunk(head_dim), R = n_heads / n_kv_heads;
    return sizeof(float) * ((size_t)tc * (head_dim + 1) + (size_t)tc * head_dim + (size_t)R * head_dim +
                            (size_t)R * tc + 2 * (size_t)R);
}

hipError_t launch_attention(const float *q, const float *k_cache, const float *v_cache, int n_heads, int n_kv_heads,
                            int head_dim, const int *d_pos, int max_seq, float *out, void *workspace,
                            hipStream_t s) {
    const int tc = attention_chunk(head_dim), nch = (max_seq + tc - 1) / tc;
    const size_t lds = attention_lds_bytes(n_heads, n_kv_heads, head_dim);
    static bool attr = hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_chunk_k),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    (void)attr;
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    float *part = static_cast<float *>(workspace);
    attn_chunk_k<<<dim3(n_kv_heads, nch), 256, lds, s>>>(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, d_pos,
                                                         max_seq, tc, scale, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    attn_combine_k<<<n_heads, 256, 0, s>>>(part, head_dim, d_pos, max_seq, tc, nch, out);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gate, const float *up, int n, float *out, hipStream_t s) {
    silu_mul_k<<<(n + 255) / 256, 256, 0, s>>>(gate, up, n, out);
    return hipGetLastError();
}

hipError_t launch_pos_increment(int *d_pos, int delta, hipStream_t s) {
    pos_increment_k<<<1, 64, 0, s>>>(d_pos, delta);
    return hipGetLastError();
}

}  // namespace jh
