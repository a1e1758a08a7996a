/*
 * junohip.h -- C ABI of libjunohip.so, the MI355X (gfx950) quantized matvec
 * library that replaces the GPU side of Juno's matvec boundary.
 *
 * Reference interfaces replaced (paths under /root/reference/node/src/main/java/cab/ml/juno/node/):
 *   MatVec.sgemv(...)                        MatVec.java:56-90
 *   GpuMatVec.upload/uploadHalf/...          GpuMatVec.java:38-70
 *   RocmMatVec (rocBLAS sgemv / hssgemv)     RocmMatVec.java:52-452
 *   RocmBindings / GpuContext / Device*Matrix RocmBindings.java:61-287, GpuContext.java:58-268,
 *                                            DeviceFloatMatrix.java:39-111, DeviceHalfMatrix.java:41-115
 *   RocmAvailability                         RocmAvailability.java:32-128
 *   static matVec(QuantizedTensor, x, rowStart, rowEnd, cols)
 *                                            LlamaTransformerHandler.java:1200-1254
 *   LlamaTransformerHandler.dequantize       LlamaTransformerHandler.java:873-885
 *   LoraMerge.requantize                     LoraMerge.java:226-241
 *
 * Conventions
 *   - Every function returns an int status: JH_OK (0) or a JH_E* code.  The
 *     message of the last failure on the calling thread is jh_last_error().
 *   - Messages follow the reference: dimension errors name "rows*cols" or
 *     "cols" (MatVecBackendContractTest.java:196-212); HIP failures read
 *     "<op> failed: rc=N" (GpuBindings.java:180-183); out-of-memory errors
 *     contain "hipMalloc" so the handlers' CPU fallback keeps working
 *     (LlamaTransformerHandler.java:340-357).
 *   - Weight matrices are W[rows][cols] row-major in GGUF packed blocks along
 *     cols, exactly the bytes of GgufReader.QuantizedTensor.data()
 *     (GgufReader.java:319-339).  Supported ggml types: 0 (F32), 8 (Q8_0),
 *     12 (Q4_K), 13 (Q5_K), 14 (Q6_K).
 *   - Host-pointer entry points are synchronous and thread-safe: each host
 *     thread has its own HIP stream and staging buffers per device.
 *   - Device-pointer entry points (*_dev) enqueue on the given stream
 *     (NULL = the default stream) and return without synchronising.
 *   - Some *_dev calls use a library workspace of the stream they are given
 *     (batched MFMA GEMVs, attention, LoRA, the small-matrix SwiGLU path).
 *     It is allocated, or grown, only outside graph capture: before capturing
 *     such calls, make each of them once eagerly on the same stream with the
 *     same sizes, or the captured call fails with JH_EINVAL.  A workspace that
 *     grows is replaced, never freed, so graphs captured earlier stay valid.
 *     A captured graph uses its stream's workspace: do not replay it while
 *     other work on that workspace (the same stream's calls or another replay)
 *     is running on another stream.
 */
#ifndef JUNOHIP_H
#define JUNOHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    JH_OK = 0,
    JH_EINVAL = 1,       /* IllegalArgumentException in the reference */
    JH_ENOMEM = 2,       /* device allocation failed ("hipMalloc failed ...") */
    JH_EHIP = 3,         /* IllegalStateException("<op> failed: rc=N") */
    JH_EUNSUPPORTED = 4, /* UnsupportedOperationException (ggml type) */
    JH_ECLOSED = 5,      /* IllegalStateException("... is closed") */
    JH_ENODEV = 6,       /* no usable gfx950 device */
    JH_EFORMAT = 7,      /* IOException: not a GGUF / llamafile, bad header or metadata */
    JH_EIO = 8,          /* IOException: open / read failed or file truncated */
};

enum {
    JH_TYPE_F32 = 0,
    JH_TYPE_Q8_0 = 8,
    JH_TYPE_Q2_K = 10,
    JH_TYPE_Q3_K = 11,
    JH_TYPE_Q4_K = 12,
    JH_TYPE_Q5_K = 13,
    JH_TYPE_Q6_K = 14,
};

typedef struct jh_ctx jh_ctx;
typedef struct jh_qmat jh_qmat;

/* Thread-local message of the last failing call on this thread ("" if none).
 * Replaces GpuBindings.check's exception text (GpuBindings.java:180-183). */
const char *jh_last_error(void);

/* Library version string, e.g. "junohip 0.1 gfx950". */
const char *jh_version(void);

/* Device discovery; replaces RocmAvailability.isAvailable / device queries
 * (RocmAvailability.java:32-128, RocmBindings.java:208-238). */
int jh_device_count(int *count);
int jh_device_info(int device, char name[256], uint64_t *vram_bytes, char arch[64]);

/* Process-wide shared context per device, reference counted; replaces
 * GpuContext.shared(dev) (GpuContext.java:109-120). */
int jh_ctx_create(int device, jh_ctx **out);
int jh_ctx_destroy(jh_ctx *ctx);

/* GgufReader.rawByteCount (GgufReader.java:347-360) for the supported types. */
int jh_raw_byte_count(int ggml_type, int64_t nelems, int64_t *out);

/* Copy packed bytes host->device unchanged and keep them resident; replaces
 * GpuMatVec.upload / uploadHalf (GpuMatVec.java:38-58) and the dequantize->fp16
 * upload of LlamaTransformerHandler.java:296-358.  nbytes must equal
 * rawByteCount(type, rows*cols) and cols must be a multiple of the block size. */
int jh_qmat_upload(jh_ctx *ctx, int ggml_type, const void *raw, size_t nbytes, int rows, int cols,
                   jh_qmat **out);

/* Quantize a device fp32 matrix [rows][cols] into a new resident packed matrix
 * with LoraMerge's quantizers (LoraMerge.java:226-469), on the device. */
int jh_qmat_quantize_dev(jh_ctx *ctx, int ggml_type, const float *d_src, int rows, int cols,
                         void *stream, jh_qmat **out);

/* Release the device memory and the handle (DeviceHalfMatrix.close(),
 * DeviceHalfMatrix.java:107-114).  NULL is accepted; the handle is invalid
 * afterwards, so idempotent close() lives in the binding, which clears its
 * pointer. */
int jh_qmat_free(jh_qmat *m);

/* Shape, type, size and device address of the packed bytes. */
int jh_qmat_info(const jh_qmat *m, int *ggml_type, int *rows, int *cols, size_t *nbytes,
                 const void **d_raw);

/* y[r - row_start] = sum_c deq(W[r][c]) * x[c] for r in [row_start, row_end).
 * Host x[cols] in, host y[row_end-row_start] out, synchronous; x is not
 * mutated.  Replaces sgemv(DeviceHalfMatrix, x) (RocmMatVec.java:272-329) and
 * matVec(QuantizedTensor, x, rowStart, rowEnd, cols)
 * (LlamaTransformerHandler.java:1200-1212). */
int jh_qmatvec(jh_ctx *ctx, const jh_qmat *m, const float *x, float *y, int row_start, int row_end);

/* B right-hand sides at once: X[B][cols] in, Y[B][row_end-row_start] out,
 * row-major, host pointers, synchronous.  Equal, to the GEMV tolerance, to B
 * independent jh_qmatvec calls.  This is the batched entry point the
 * reference's InferencePipeline.forwardBatch lacks (InferencePipeline.java:62-69). */
int jh_qmatvec_batched(jh_ctx *ctx, const jh_qmat *m, const float *X, int B, float *Y, int row_start,
                       int row_end);

/* Full fp32 dequantization W[rows][cols] to host memory, bit-exact with
 * LlamaTransformerHandler.dequantize (LlamaTransformerHandler.java:873-1135). */
int jh_qmat_dequant(jh_ctx *ctx, const jh_qmat *m, float *out);

/* Plain fp32 GEMV with host operands, A[rows][cols] row-major; replaces
 * MatVec.sgemv(float[] A, float[] x, rows, cols) (MatVec.java:56-66,
 * RocmMatVec.java:138-197). */
int jh_sgemv(jh_ctx *ctx, const float *A, const float *x, int rows, int cols, float *y);

/* Device-pointer variants: operands already in HBM, enqueued on `stream`. */
int jh_qmatvec_dev(const jh_qmat *m, const float *d_x, float *d_y, int row_start, int row_end,
                   void *stream);
int jh_qmatvec_batched_dev(const jh_qmat *m, const float *d_X, int B, float *d_Y, int row_start,
                           int row_end, void *stream);
int jh_qmat_dequant_dev(const jh_qmat *m, float *d_out, void *stream);

/* jh_qmatvec_batched_dev without any device allocation.  No counterpart in
 * the reference: for callers that cannot allocate (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).  The scratch
 * of the batched MFMA path (split-K partials, prepared x, arrival counters)
 * is a library-static device array of 8 MiB of workspace per device instead
 * of the stream workspace; a call that would need more fails with JH_EINVAL
 * and says how much (jh_qmatvec_batched_dev has no such limit).  Every call
 * on a device shares that device's array, which keeps the last call's
 * contents: calls that overlap on one device (two streams, or a graph replay
 * beside an eager call) race and must be ordered by the caller.  Results are
 * those of jh_qmatvec_batched_dev, bit for bit. */
int jh_qmatvec_batched_noalloc_dev(const jh_qmat *m, const float *d_X, int B, float *d_Y, int row_start,
                                   int row_end, void *stream);

/* n <= 8 independent GEMVs, y_i = W_i x_i over all rows of W_i, B = 1, device
 * pointers, enqueued on one stream in as few kernel launches as possible:
 * large matrices of one format that share an x (gate and up) go through one
 * staged launch, all other matrices through one one-shot launch.  Equal to n
 * jh_qmatvec_dev calls.  The handlers issue such independent matVecs back to
 * back on one input (Q, K, V and gate, up: LlamaTransformerHandler.java:751-800;
 * the fused-QKV row ranges of Phi3TransformerHandler.java:329-334). */
int jh_qmatvec_group_dev(int n, const jh_qmat *const *mats, const float *const *d_x, float *const *d_y,
                         void *stream);

/* out[r] = silu(gate_r . x) * (up_r . x) at B = 1 for every row r of the two
 * matrices (same shape and format): the FFN's gate / up projections and the
 * SwiGLU product of LlamaTransformerHandler.java:796-797 (silu: :1733-1735),
 * which the reference runs as two matVecs and a host loop.  Large matrices
 * take one staged launch that pairs row r of gate with row r of up, so the
 * product is formed where both dot products end and neither projection is
 * written out; otherwise a grouped GEMV into the stream's workspace and
 * jh_silu_mul_dev's kernel.  Equal to that pair of calls. */
int jh_qmatvec_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_x, float *d_out, void *stream);

/* The FFN input norm fused into the gate / up launch: h = x + res (res may be
 * NULL: h = x), x_out = h (when not NULL; it must not alias x or res),
 * out[r] = silu(gate_r . xn) * (up_r . xn) with xn = rmsNorm(h, norm_w, eps).
 * transformerLayer's x2 = x + attnProj, rmsNorm(x2) and the SwiGLU
 * (LlamaTransformerHandler.java:778-797, rmsNorm :818-826).  Where the staged
 * kernel applies (large matrices, cols <= 4096) one launch converts the norm's
 * output as its input and never writes xn; otherwise jh_rmsnorm_dev into the
 * caller's xn scratch (n floats, contents unspecified afterwards) and
 * jh_qmatvec_swiglu_dev.  The two differ only in the summation order of
 * mean(h^2). */
int jh_rmsnorm_qmatvec_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_x, const float *d_res,
                                  const float *d_norm_w, float eps, float *d_x_out, float *d_xn, float *d_out,
                                  void *stream);

/* The same fusion for one GEMV over all rows at B = 1: y = W rmsNorm(x + res)
 * (the final norm and the output projection, LlamaTransformerHandler.java:803-810). */
int jh_rmsnorm_qmatvec_dev(const jh_qmat *m, const float *d_x, const float *d_res, const float *d_norm_w, float eps,
                           float *d_x_out, float *d_xn, float *d_y, void *stream);

/* Device-side waits that gave up since the last call on this device (a
 * column-tile ring cell of the staged kernel past its spin bound: that launch's
 * results are then wrong); the count is cleared.  No counterpart in the
 * reference (its matVecs have no cross-wave waits): for tests and health checks. */
int jh_sync_faults(int device, unsigned int *count);

/* Timeline builds only (compiled with -DJH_TIMELINE by juno_amd/timeline.py,
 * never the shipped library; JH_EUNSUPPORTED otherwise): n entries of the
 * per-wave s_memrealtime stamps (100 MHz) of the last launch.  kernel 0: the
 * staged B = 1 walk, 4 per wave at (workgroup * 16 + wave) * 4: entry, after
 * the x prologue, first row group landed, end of the walk.  kernel 1: the
 * batched MFMA walk at B <= 32, 68 per wave at (workgroup * 8 + wave) * 68:
 * entry, then per super-block step (up to 16) after the barrier, weights
 * parked, next x staged, MFMAs folded; then the split-K epilogue's partials
 * acknowledged, arrival counted, end of the last split's sums and stores.  No counterpart in the reference; a
 * profiling aid. */
int jh_debug_timeline(int device, int kernel, uint64_t *out, size_t n);

/* The attention input norm fused into the grouped GEMV of the matrices that
 * read it: h = x + res, x_out = h (when not NULL; it must not alias x or res),
 * y_i = W_i rmsNorm(h, norm_w, eps) for n <= 8 matrices of one column count
 * (q, k, v: transformerLayer's rmsNorm and three matVecs,
 * LlamaTransformerHandler.java:749-757, rmsNorm :818-826).  With res given and
 * quantized matrices one one-shot launch forms w_n * h in each workgroup's LDS,
 * applies the norm's scale to its sums and never writes xn (cols <= 8192);
 * otherwise jh_rmsnorm_dev into the caller's xn scratch (cols floats) and
 * jh_qmatvec_group_dev.  The two differ only in where the scale is applied
 * and the summation order of mean(h^2). */
int jh_rmsnorm_qmatvec_group_dev(int n, const jh_qmat *const *mats, const float *d_x, const float *d_res,
                                 const float *d_norm_w, float eps, float *d_x_out, float *d_xn, float *const *d_y,
                                 void *stream);

/* Batched form: out[b][r] = silu(gate_r . X_b) * (up_r . X_b) for B rows of X.
 * For 3 <= B <= 32 (Q4_K, Q5_K, Q6_K, Q8_0) one MFMA launch whose workgroups
 * take 128 rows of gate and the same rows of up and store the product; B = 1
 * is jh_qmatvec_swiglu_dev; otherwise jh_qmatvec_batched_group_dev into the
 * caller's d_gate / d_up scratch ([B][rows] each, used only on that path) and
 * jh_silu_mul_dev.  Equal to that pair of calls, bit for bit. */
int jh_qmatvec_batched_swiglu_dev(const jh_qmat *gate, const jh_qmat *up, const float *d_X, int B, float *d_out,
                                  float *d_gate, float *d_up, void *stream);

/* Batched form of jh_qmatvec_group_dev: Y_i[B][rows_i] = X_i[B][cols] W_i^T
 * for n <= 4 matrices, full row ranges, one launch when B >= 3 and the
 * matrices share cols (the MFMA path; formats may differ, e.g. the Q4_K q / k
 * and Q6_K v of a Q4_K_M layer), else one call per matrix.  Same results as
 * n calls of jh_qmatvec_batched_dev.  The reference's forwardBatch runs the
 * requests one by one (InferencePipeline.java:62-69); this is the grouped
 * projection step of its batched replacement. */
int jh_qmatvec_batched_group_dev(int n, const jh_qmat *const *mats, const float *const *d_X, int B,
                                 float *const *d_Y, void *stream);

/* Diagnostics: the kernel jh_qmatvec_batched_group_dev takes for these n
 * matrices (full row ranges) at batch B: *kernel = 0 for the VALU kernels,
 * 1 for the grouped MFMA kernel with K split *ksplit ways, 2 for the
 * prepared-x MFMA kernel (one matrix with enough row tiles to fill the GPU
 * unsplit, B <= 32: the output projection).  No counterpart in the reference;
 * for tests that must reach a given kernel. */
int jh_qmatvec_batched_plan(int n, const jh_qmat *const *mats, int B, int *kernel, int *ksplit);
/* The same plan for one matrix of a given format and shape, rows [row_start,
 * row_end), without a device or a matrix (host-only arithmetic): for CPU
 * checks of the kernels' address arithmetic. */
int jh_qmatvec_batched_plan_shape(int ggml_type, int cols, int row_start, int row_end, int B, int *kernel,
                                  int *ksplit);

/* Diagnostics of the per-stream library workspace (see Conventions): the
 * scratch bytes the stream `stream` on `device` currently has (0 before its
 * first use) and the base address of its live allocation, which changes when
 * the workspace grows.  No counterpart in the reference; for tests and tools
 * that check that captured graphs survive growth. */
int jh_stream_workspace_info(int device, void *stream, size_t *scratch_bytes, void **base);

/* Raw-pointer variant of the quantizer: n fp32 values -> packed bytes in a
 * caller-provided device buffer of rawByteCount(type, n) bytes. */
int jh_quantize_dev(int ggml_type, const float *d_src, int64_t n, void *d_dst, void *stream);

/* ---- The rest of a Llama decode step, device-resident.  All pointers are
 * device pointers; the device is the caller's current device; work is
 * enqueued on `stream` (NULL: the null stream).  The decode position is a
 * device int (d_pos) so that a captured graph of a step can be replayed with
 * the position advanced on the device (jh_pos_increment_dev).  These have no
 * C counterpart in the reference: each restates one Java method of
 * LlamaTransformerHandler, cited per function, for a device-activation path
 * beside the MatVec interface. */

/* out = rmsNorm(v, w, eps) with v = x + res (res may be NULL: v = x); when
 * x_out is not NULL it receives v (x_out may equal x: in-place residual).
 * rmsNorm: LlamaTransformerHandler.java:818-826; the residual adds of
 * transformerLayer :778, :783.  n <= 1 << 20. */
int jh_rmsnorm_dev(const float *x, const float *res, const float *w, int n, float eps, float *x_out, float *out,
                   void *stream);

/* jh_rmsnorm_dev over each row of [rows][n] (a batch of requests, one row
 * each): forwardBatch's stacked activations (InferencePipeline.java:62-69). */
int jh_rmsnorm_rows_dev(const float *x, const float *res, const float *w, int n, int rows, float eps, float *x_out,
                        float *out, void *stream);

/* Rotary embedding at position *d_pos (adjacent pairs) of q in place and of
 * k into k_cache[pos], and v copied into v_cache[pos]; caches hold max_seq
 * rows of n_kv_heads * head_dim floats.  rope: LlamaTransformerHandler.java:
 * 1657-1671; the cache stores of transformerLayer :769-770. */
int jh_rope_kv_dev(float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                   const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache, void *stream);

/* Grouped-query attention of q over cache positions 0 .. *d_pos, output
 * [n_heads * head_dim].  gqa + softmax: LlamaTransformerHandler.java:1678-1731.
 * Uses a per-stream library workspace (allocated on first use, JH_ENOMEM
 * with "hipMalloc" in the message on failure). */
int jh_attention_dev(const float *q, const float *k_cache, const float *v_cache, int n_heads, int n_kv_heads,
                     int head_dim, const int *d_pos, int max_seq, float *out, void *stream);

/* The attention sub-layer of one position in one launch pair: rope of the raw
 * projections q and k at *d_pos, k and v appended to the caches, and the
 * attention output (q is not modified).  transformerLayer :765-773 with rope
 * :1657-1671 and gqa :1678-1731.  Same workspace as jh_attention_dev. */
int jh_rope_attention_dev(const float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                          const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache, float *out,
                          void *stream);

/* jh_rope_attention_dev followed by the output projection y = wo . att
 * (transformerLayer :765-776: rope, KV append, gqa, then wo): the pair of
 * calls (jh_rope_attention_dev, then jh_qmatvec_group_dev of wo).  With
 * JUNO_ATTN_FUSE=1, where the staged GEMV applies (B = 1, at most 64 heads and
 * 64 chunks of the cache), attention's combine of its chunk partials runs in
 * the GEMV's input conversion instead of a launch of its own and one of its
 * workgroups stores att (one launch fewer, but slower at the shapes measured:
 * each workgroup reads every partial).  att is the attention output either
 * way, equal bit for bit; y is within the GEMV tolerance of the pair's (the
 * same bits as the staged kernel on att).  wo has n_heads * head_dim columns.
 * Same workspace as jh_rope_attention_dev. */
int jh_rope_attention_qmatvec_dev(const float *q, const float *k, const float *v, int n_heads, int n_kv_heads,
                                  int head_dim, const int *d_pos, int max_seq, float theta, float *k_cache,
                                  float *v_cache, const jh_qmat *wo, float *att, float *y, void *stream);
/* jh_rope_attention_dev for `batch` requests in one launch pair: q [batch][n_heads*head_dim], k and v
 * [batch][n_kv_heads*head_dim], out like q; request z is at position d_pos[z] and uses KV-cache slot
 * d_slot[z] of caches laid out [n_slots][max_seq][n_kv_heads*head_dim] (one slot per request, the
 * per-requestId caches of LlamaTransformerHandler.java:670-679).  forwardBatch, InferencePipeline.java:62-69. */
int jh_rope_attention_batched_dev(const float *q, const float *k, const float *v, int batch, int n_heads,
                                  int n_kv_heads, int head_dim, const int *d_pos, const int *d_slot, int n_slots,
                                  int max_seq, float theta, float *k_cache, float *v_cache, float *out, void *stream);

/* out = silu(gate) * up.  silu and ffn: LlamaTransformerHandler.java:1733-1735,
 * 796-797. */
int jh_silu_mul_dev(const float *gate, const float *up, int n, float *out, void *stream);

/* The embedding row of token clamp(*d_token, 0, rows - 1), dequantized into
 * d_out[cols]: getInitialActivation (LlamaTransformerHandler.java:651-660) over
 * the packed token_embd matrix kept resident instead of a host float[] copy.
 * The token is read on the device, so a captured step can be replayed. */
int jh_embed_dev(const jh_qmat *m, const int *d_token, float *d_out, void *stream);

/* jh_embed_dev for n tokens d_tokens[0..n) into d_out[n][cols] (a batch of requests). */
int jh_embed_rows_dev(const jh_qmat *m, const int *d_tokens, int n, float *d_out, void *stream);

/* d_y[r][i] += d_bias[i] for each of rows rows of n: the Q / K / V projection biases of
 * Qwen2-style models, added right after the projections (addInPlace,
 * LlamaTransformerHandler.java:758-761, 1641-1646). */
int jh_add_rows_dev(float *d_y, const float *d_bias, int n, int rows, void *stream);

/* LoRA overlay: for each of `batch` rows, d_y[b][0..out_dim) += scale * B (A d_x[b]), with
 * A [rank][in_dim] and B [out_dim][rank] fp32 in HBM.  LoraAdapter.forward
 * (lora/.../LoraAdapter.java:79-98) added to a projection's output as
 * LoraTrainableHandler.applyLoraInPlace does (LoraTrainableHandler.java:475-476, 489-496);
 * scale = alpha / rank.  Uses the stream workspace for the rank-r intermediate. */
int jh_lora_apply_dev(const float *d_a, const float *d_b, int rank, int in_dim, int out_dim, float scale,
                      const float *d_x, int batch, float *d_y, void *stream);

/* *d_pos += delta, on the device (for replaying a captured decode step). */
int jh_pos_increment_dev(int *d_pos, int delta, void *stream);

/* ---------------------------------------------------------------- GGUF files
 *
 * GgufReader (GgufReader.java) behind plain handles.  A file that does not
 * start with the GGUF magic is read as a llamafile: a ZIP whose *.gguf entry is
 * stored uncompressed (findGgufOffsetInZip, :808-1025, with the forward-scan
 * fallback :1027-1134 and ZIP64 offsets :1136-1154).  Metadata keeps the
 * reference's Java typing (readMetadataValue, :1189-1246): 8- and 16-bit
 * integers sign-extended to int, 32-bit to int, 64-bit to long. */
typedef struct jh_gguf jh_gguf;

enum {
    JH_GGUF_UINT8 = 0, JH_GGUF_INT8 = 1, JH_GGUF_UINT16 = 2, JH_GGUF_INT16 = 3, JH_GGUF_UINT32 = 4,
    JH_GGUF_INT32 = 5, JH_GGUF_FLOAT32 = 6, JH_GGUF_BOOL = 7, JH_GGUF_STRING = 8, JH_GGUF_ARRAY = 9,
    JH_GGUF_UINT64 = 10, JH_GGUF_INT64 = 11, JH_GGUF_FLOAT64 = 12,
};

/* GgufReader.open (:102-183): header, metadata, tensor infos, data offset
 * (aligned to 32 bytes from the start of the GGUF image).  JH_EFORMAT carries
 * the reference's IOException messages. */
int jh_gguf_open(const char *path, jh_gguf **out);

/* GgufReader.close (:382-385).  NULL is accepted. */
int jh_gguf_close(jh_gguf *g);

/* GGUF version, header tensor / metadata counts, ggufFileOffset (:293),
 * the data-section offset and metadataSectionEnd (:284).  Any out may be NULL. */
int jh_gguf_info(const jh_gguf *g, int *version, int64_t *tensor_count, int64_t *kv_count, int64_t *gguf_offset,
                 int64_t *data_offset, int64_t *metadata_end);

/* meta(key) (:185): the value type (-1 when absent); for arrays the element
 * type and count. */
int jh_gguf_meta_type(const jh_gguf *g, const char *key, int *vtype, int *elem_type, int64_t *count);

/* metaLong / metaInt / metaFloat (:194-207): present = the value is a Number;
 * as_long = Number.longValue(), as_double = the exact value (a FLOAT32 value
 * is exact in double, so floatValue() is (float)as_double). */
int jh_gguf_meta_number(const jh_gguf *g, const char *key, int *present, int64_t *as_long, double *as_double);

/* A BOOL entry (readMetadataValue :1220-1226): present = the key holds a bool. */
int jh_gguf_meta_bool(const jh_gguf *g, const char *key, int *present, int *value);

/* metaString (:189-192): *len = the UTF-8 byte length, or (size_t)-1 when the
 * key is absent or not a string; up to cap-1 bytes and a NUL go to buf. */
int jh_gguf_meta_string(const jh_gguf *g, const char *key, char *buf, size_t cap, size_t *len);

/* Index of a tensor in file order (tensorOrder, :275), -1 when absent
 * (hasTensor, :209).  A repeated name maps to its last entry. */
int jh_gguf_tensor_index(const jh_gguf *g, const char *name, int64_t *index);

/* tensorType / tensorDims / tensorNelems / tensorAbsoluteOffset (:225-270).
 * dims receives ndims (<= 8) entries; *name stays valid until close. */
int jh_gguf_tensor_info(const jh_gguf *g, int64_t index, const char **name, int *ggml_type, int *ndims,
                        int64_t dims[8], int64_t *nelems, int64_t *abs_offset);

/* tensorRaw (:329-345): the packed bytes, rawByteCount (:347-360) of them,
 * into dst (cap bytes); *nbytes receives the size even when cap is short, and
 * dst = NULL with cap = 0 only queries it. */
int jh_gguf_tensor_read(const jh_gguf *g, int64_t index, void *dst, size_t cap, size_t *nbytes);

/* tensorRaw + jh_qmat_upload in one pass: the tensor's bytes are streamed from
 * the file through pinned staging into a new resident matrix with cols =
 * dims[0] and rows = nelems / dims[0] (the ggml layout the reference's handlers
 * use, LlamaTransformerHandler.java:296-358).  No host copy of the whole
 * tensor is made. */
int jh_gguf_upload(jh_ctx *ctx, const jh_gguf *g, int64_t index, jh_qmat **out);

#ifdef __cplusplus
}
#endif
#endif /* JUNOHIP_H */
