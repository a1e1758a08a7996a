/*
 * juno_oracle_decode.c -- CPU restatement of the rest of Juno's Llama decode
 * step around the quantized matvec: RMS normalisation, rotary embeddings,
 * grouped-query attention with its softmax, SwiGLU and the residual adds,
 * composed into one transformer layer exactly as the reference composes them.
 *
 * TEST INFRASTRUCTURE ONLY (see juno_oracle.h).  Java semantics kept: strict
 * fp32 without contraction (-ffp-contract=off), sequential loops in the
 * reference's order, double precision exactly where the reference computes in
 * double (Math.sqrt / Math.pow / Math.cos / Math.sin / Math.exp, each result
 * cast to float where the Java code casts it).  libm's double routines stand
 * in for java.lang.Math's: both are faithfully rounded, so individual values
 * may differ in the last double bit, far below the fp32 results' resolution.
 *
 * Citations relative to /root/reference/node/src/main/java/cab/ml/juno/node/.
 */
#include "juno_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* rmsNorm, LlamaTransformerHandler.java:818-826 */
void or_rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float scale = 1.0f / (float)sqrt((double)(ss / (float)n + eps));
    for (int i = 0; i < n; i++) out[i] = w[i] * x[i] * scale;
}

/* rope, LlamaTransformerHandler.java:1657-1671 (adjacent pairs, in place) */
void or_rope(float *x, int pos, int n_heads, int head_dim, float theta) {
    for (int h = 0; h < n_heads; h++) {
        const int base = h * head_dim;
        for (int i = 0; i < head_dim / 2; i++) {
            const double freq = 1.0 / pow((double)theta, (2.0 * i) / head_dim);
            const double angle = pos * freq;
            const float c = (float)cos(angle), s = (float)sin(angle);
            const float x0 = x[base + 2 * i], x1 = x[base + 2 * i + 1];
            x[base + 2 * i] = x0 * c - x1 * s;
            x[base + 2 * i + 1] = x0 * s + x1 * c;
        }
    }
}

/* softmax, LlamaTransformerHandler.java:1718-1731 (in place over n) */
void or_softmax(float *s, int n) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++)
        if (s[i] > mx) mx = s[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        s[i] = (float)exp((double)(s[i] - mx));
        sum += s[i];
    }
    for (int i = 0; i < n; i++) s[i] /= sum;
}

/* gqa, LlamaTransformerHandler.java:1678-1715.  k_cache / v_cache rows are
 * kv_dim = n_kv_heads * head_dim floats per position; out has n_heads * head_dim. */
void or_gqa(const float *q, const float *k_cache, const float *v_cache, int n_heads, int n_kv_heads,
            int head_dim, int seq_len, float *out) {
    const int ratio = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
    const float scale = (float)(1.0 / sqrt((double)head_dim));
    float *scores = (float *)malloc(sizeof(float) * (size_t)(seq_len > 0 ? seq_len : 1));
    memset(out, 0, sizeof(float) * (size_t)n_heads * head_dim);
    for (int h = 0; h < n_heads; h++) {
        const int kbase = (h / ratio) * head_dim, qbase = h * head_dim;
        for (int t = 0; t < seq_len; t++) {
            float dot = 0.0f;
            const float *kr = k_cache + (size_t)t * kv_dim + kbase;
            for (int d = 0; d < head_dim; d++) dot += q[qbase + d] * kr[d];
            scores[t] = dot * scale;
        }
        or_softmax(scores, seq_len);
        for (int t = 0; t < seq_len; t++) {
            const float *vr = v_cache + (size_t)t * kv_dim + kbase;
            const float wt = scores[t];
            for (int d = 0; d < head_dim; d++) out[qbase + d] += wt * vr[d];
        }
    }
    free(scores);
}

/* silu, LlamaTransformerHandler.java:1733-1735, and the SwiGLU product of ffn :796-797 */
float or_silu(float x) { return x / (1.0f + (float)exp((double)-x)); }

void or_silu_mul(const float *gate, const float *up, int n, float *out) {
    for (int i = 0; i < n; i++) out[i] = or_silu(gate[i]) * up[i];
}

/* add, LlamaTransformerHandler.java:1737-1742 */
/* LoraAdapter.forward (lora/src/main/java/cab/ml/juno/lora/LoraAdapter.java:79-98):
 * h[r] = sum_c a[r*in + c] * x[c] in c order; delta[o] = (sum_r b[o*rank + r] * h[r]) * scale. */
void or_lora_forward(const float *a, const float *b, int rank, int in_dim, int out_dim, float scale, const float *x,
                     float *delta) {
    float h[4096];
    if (rank > 4096) return;
    for (int r = 0; r < rank; r++) {
        float acc = 0.0f;
        for (int c = 0; c < in_dim; c++) acc += a[(size_t)r * in_dim + c] * x[c];
        h[r] = acc;
    }
    for (int o = 0; o < out_dim; o++) {
        float acc = 0.0f;
        for (int c = 0; c < rank; c++) acc += b[(size_t)o * rank + c] * h[c];
        delta[o] = acc * scale;
    }
}

void or_add(const float *a, const float *b, int n, float *out) {
    for (int i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* transformerLayer, LlamaTransformerHandler.java:743-784, with ffn :787-800.
 * Matrices are packed rows x cols (GGML type per matrix); k_cache / v_cache
 * hold at least pos + 1 positions and receive this position's k and v.
 * x is updated in place.  Returns 0, or -1 on an unsupported matrix type. */
int or_llama_layer(const OrLlamaLayer *L, const OrLlamaDims *D, float *x, int pos, float *k_cache,
                   float *v_cache, int nthreads) {
    const int H = D->hidden, KV = D->n_kv_heads * D->head_dim, I = D->ffn;
    float *xn = (float *)malloc(sizeof(float) * (size_t)H);
    float *q = (float *)malloc(sizeof(float) * (size_t)H);
    float *k = (float *)malloc(sizeof(float) * (size_t)KV);
    float *v = (float *)malloc(sizeof(float) * (size_t)KV);
    float *att = (float *)malloc(sizeof(float) * (size_t)H);
    float *proj = (float *)malloc(sizeof(float) * (size_t)H);
    float *g = (float *)malloc(sizeof(float) * (size_t)I);
    float *u = (float *)malloc(sizeof(float) * (size_t)I);
    float *hid = (float *)malloc(sizeof(float) * (size_t)I);
    int rc = 0;
    or_rmsnorm(x, L->attn_norm, H, D->eps, xn);
    rc |= or_matvec(L->type_q, L->wq, xn, 0, H, H, q, nthreads);
    rc |= or_matvec(L->type_k, L->wk, xn, 0, KV, H, k, nthreads);
    rc |= or_matvec(L->type_v, L->wv, xn, 0, KV, H, v, nthreads);
    or_rope(q, pos, D->n_heads, D->head_dim, D->theta);
    or_rope(k, pos, D->n_kv_heads, D->head_dim, D->theta);
    memcpy(k_cache + (size_t)pos * KV, k, sizeof(float) * (size_t)KV);
    memcpy(v_cache + (size_t)pos * KV, v, sizeof(float) * (size_t)KV);
    or_gqa(q, k_cache, v_cache, D->n_heads, D->n_kv_heads, D->head_dim, pos + 1, att);
    rc |= or_matvec(L->type_o, L->wo, att, 0, H, H, proj, nthreads);
    or_add(x, proj, H, x); /* x2 = x + attnProj */
    or_rmsnorm(x, L->ffn_norm, H, D->eps, xn);
    rc |= or_matvec(L->type_gate, L->wgate, xn, 0, I, H, g, nthreads);
    rc |= or_matvec(L->type_up, L->wup, xn, 0, I, H, u, nthreads);
    or_silu_mul(g, u, I, hid);
    rc |= or_matvec(L->type_down, L->wdown, hid, 0, H, I, proj, nthreads);
    or_add(x, proj, H, x);
    free(xn); free(q); free(k); free(v); free(att); free(proj); free(g); free(u); free(hid);
    return rc ? -1 : 0;
}
