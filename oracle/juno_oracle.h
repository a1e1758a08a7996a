/*
 * juno_oracle.h -- CPU restatement of Juno's Java quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP library
 * (libjunohip.so).  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load it.  No product code path may call it.
 *
 * Every function restates one Java routine of the reference with the Java
 * semantics kept: strict IEEE fp32 with no contraction (built with
 * -ffp-contract=off), signed bytes masked explicitly, Math.round as
 * floor(x + 0.5) evaluated exactly, sequential per-row accumulation in
 * block -> group -> element order.  Citations are given per function in
 * juno_oracle.c, relative to /root/reference/node/src/main/java/cab/ml/juno/node/.
 */
#ifndef JUNO_ORACLE_H
#define JUNO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids used by Juno (GgufReader.java constants). */
enum {
    OR_TYPE_F32 = 0,
    OR_TYPE_Q8_0 = 8,
    OR_TYPE_Q2_K = 10,
    OR_TYPE_Q3_K = 11,
    OR_TYPE_Q4_K = 12,
    OR_TYPE_Q5_K = 13,
    OR_TYPE_Q6_K = 14,
};

float    or_f16_to_f32(uint16_t bits);
uint32_t or_f16_to_f32_bits(uint16_t bits);
uint16_t or_f32_to_f16(float value);
int32_t  or_java_round(float a);
int64_t  or_raw_byte_count(int type, int64_t nelems);

/* Q4_K 6-bit scale / min unpack for sub-block j (0..7) of the 12 scale bytes. */
int or_q4k_scale(const uint8_t *sc, int j);
int or_q4k_min(const uint8_t *sc, int j);
/* The 16 signed Q3_K sub-block scales (dequantizeQ3K, LlamaTransformerHandler.java:969-985). */
void or_q3k_scales(const uint8_t *sc12, int sc[16]);

/* Dequantize rows*cols elements of a packed tensor to fp32 (row-major).
 * Returns 0, or -1 for an unsupported type / cols not a block multiple. */
int or_dequantize(int type, const uint8_t *raw, int rows, int cols, float *out);

/* y[r - row_start] = sum_c deq(W[r, c]) * x[c] for r in [row_start, row_end),
 * with the Java per-row summation order.  nthreads <= 0 uses one thread per
 * online CPU (the ForkJoinPool.commonPool() parallelism plus the caller). */
int or_matvec(int type, const uint8_t *raw, const float *x, int row_start, int row_end,
              int cols, float *y, int nthreads);

/* fp32 -> packed blocks with LoraMerge's quantizers.  n must be a block
 * multiple.  out must hold or_raw_byte_count(type, n) bytes. */
int or_quantize(int type, const float *data, int64_t n, uint8_t *out);

/* ---- the rest of the decode step (juno_oracle_decode.c) ---- */
void  or_rmsnorm(const float *x, const float *w, int n, float eps, float *out);
void  or_rope(float *x, int pos, int n_heads, int head_dim, float theta);
void  or_softmax(float *s, int n);
void  or_gqa(const float *q, const float *k_cache, const float *v_cache, int n_heads, int n_kv_heads,
             int head_dim, int seq_len, float *out);
float or_silu(float x);
void  or_silu_mul(const float *gate, const float *up, int n, float *out);
/* LoraAdapter.forward: delta = (B (A x)) * scale, rank <= 4096. */
void  or_lora_forward(const float *a, const float *b, int rank, int in_dim, int out_dim, float scale, const float *x,
                      float *delta);
void  or_add(const float *a, const float *b, int n, float *out);

typedef struct {
    int hidden, n_heads, n_kv_heads, head_dim, ffn;
    float eps, theta;
} OrLlamaDims;

typedef struct {
    const float *attn_norm, *ffn_norm;                               /* [hidden] */
    const uint8_t *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;           /* packed rows x cols */
    int type_q, type_k, type_v, type_o, type_gate, type_up, type_down;
} OrLlamaLayer;

/* One transformer layer at position pos (x updated in place; k / v of this
 * position written into the caches, which hold kv_dim floats per position). */
int or_llama_layer(const OrLlamaLayer *L, const OrLlamaDims *D, float *x, int pos, float *k_cache,
                   float *v_cache, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
