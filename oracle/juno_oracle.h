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

#ifdef __cplusplus
}
#endif
#endif
