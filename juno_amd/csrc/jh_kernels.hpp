// jh_kernels.hpp -- host-side launch interface of the libjunohip kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jh {

// Bytes of zero padding after every packed matrix: the kernels read whole
// aligned dwords around 2-byte-aligned Q6_K / Q8_0 fields, which can reach up
// to 6 bytes past the last block.
constexpr size_t kTailPad = 256;

struct GemvArgs {
    int type;        // ggml type: 0, 8, 12, 14
    const uint8_t *w;  // packed matrix base (row 0)
    size_t pitch;    // bytes per row
    int cols;
    int row_start, row_end;
    int batch;       // 1, 2, 4 or 8 right-hand sides
    const float *x;  // x[j][cols], j < batch, stride ldx floats
    int ldx;
    float *y;        // y[j][row_end-row_start], stride ldy floats
    int ldy;
};

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s);

// Independent B = 1 GEMVs over full row ranges, one launch for all.
constexpr int kMaxGroup = 8;
struct GroupProblem {
    int type;
    const uint8_t *w;
    size_t pitch;
    int cols, nrows;
    const float *x;
    float *y;
    int rows_per_wave, wg_begin;  // set by the launcher
};
struct GroupArgs {
    int n;
    GroupProblem p[kMaxGroup];
    // optional residual add + rmsnorm of the (shared) input: x = w_n * (x + res) * scale,
    // h = x + res stored to x_out; hipErrorNotSupported where it does not apply
    const float *res = nullptr, *norm_w = nullptr;
    float eps = 0.f;
    float *x_out = nullptr;
};
constexpr int kNormGroupMaxCols = 8192;  // the LDS image of the normalised input
hipError_t launch_gemv_group(GroupArgs g, hipStream_t s);

// Large same-format matrices sharing one x (e.g. gate and up) through the
// staged kernel, as one launch over their concatenated rows.  Returns
// hipErrorNotSupported when the problems do not qualify.
constexpr int kMaxStagedGroup = 4;
hipError_t launch_gemv_staged_group(int n, const GroupProblem *p, hipStream_t s);
// out[r] = silu(gate_r . x) * (up_r . x) for every row r, B = 1, one staged
// launch that takes a row of gate and the same row of up into one row group
// (hipErrorNotSupported where the staged kernel does not apply)
// The residual add and rmsnorm a staged launch can apply to its input while it
// converts it: x_gemv = w * h * scale, h = x + res, scale = 1 / sqrt(mean(h^2)
// + eps); workgroup 0 stores h to x_out (which aliases neither x nor res).
struct NormSpec {
    const float *res, *w;
    float eps;
    float *x_out;
};
hipError_t launch_gemv_swiglu(const GroupProblem &gate, const GroupProblem &up, float *out, hipStream_t s,
                              const NormSpec *norm = nullptr);

// Bounded device-side waits that gave up (the staged kernel's column-tile ring
// cells) since the last call, on the current device; the count is cleared.
hipError_t sync_faults(unsigned *count);
// Timeline builds only (-DJH_TIMELINE): the staged walk's per-wave timestamps.
hipError_t timeline_read(unsigned long long *out, size_t n);
hipError_t mfma_timeline_read(unsigned long long *out, size_t n);

// B = 1 coalesced, pipelined, int8-x kernel (jh_gemv_staged.hip); returns
// hipErrorNotSupported for shapes it does not cover.
bool staged_supported(int type, int cols);
hipError_t launch_gemv_staged(const GemvArgs &a, hipStream_t s, const NormSpec *norm = nullptr);
// The input of a B = 1 GEMV formed in the staged kernel's prologue as attention's
// combine of its chunk partials (launch_attention with combine = false): part
// holds [head][nchmax][m, l, o[head_dim]] for heads = cols / head_dim, over the
// chunks of tc positions that hold 0 .. *pos.  Workgroup 0 stores the merged x
// to x_out (may be null).  hipErrorNotSupported where it does not apply.
struct CombineSpec {
    const float *part;
    const int *pos;
    int head_dim, tc, max_seq, nchmax;
    float *x_out;
};
// check_only: hipSuccess when it applies, nothing launched
hipError_t launch_gemv_staged_combine(const GemvArgs &a, const CombineSpec &c, hipStream_t s, bool check_only = false);

// Batched decode through the LDS-staged, fp16-MFMA path (kMfmaMinBatch <= B <= 64).
// Batched GEMVs (kMfmaMinBatch <= B <= 64) on fp16 MFMA: up to kMaxMfmaGroup matrices
// with the same cols, each with its own x [B][cols] and y [B][row_end -
// row_start], in one launch.  mfma_group_workspace_bytes returns 0 when the
// path does not apply (types, shapes, alignment); otherwise launch_mfma_group
// needs that many bytes of device workspace and 1024 ints of counters that
// are zero before the first launch and that every launch leaves zero (the
// split-K hand-off counts a tile's splits there).
struct MfmaDesc {
    int type;
    const uint8_t *w;
    size_t pitch;
    int cols, row_start, row_end;
    const float *x;
    float *y;
};
constexpr int kMaxMfmaGroup = 4;
// Smallest batch that takes the MFMA path.  The x tile is padded to 32 columns, so a launch costs about the same from
// B = 3 to 32.  Measured 8B GEMV step: B = 2 3.24 ms (VALU kernels) vs 3.78 ms (MFMA); B = 3 5.54 vs 3.80 ms; B = 8
// 15.4 vs 3.88 ms.
constexpr int kMfmaMinBatch = 3;
size_t mfma_group_workspace_bytes(int n, const MfmaDesc *d, int B);
hipError_t launch_mfma_group(int n, const MfmaDesc *d, int B, void *workspace, int *counters, hipStream_t s);
// Which kernel launch_mfma_group takes: 0 none (the path does not apply),
// 1 mfma_group (K split *ksplit ways), 2 x_prep + mfma_px (one unsplit matrix).
int mfma_group_plan(int n, const MfmaDesc *d, int B, int *ksplit);
// The file-scope device scratch of the MFMA path for callers that cannot
// allocate (jh_qmatvec_batched_noalloc_dev): kStaticScratchBytes of workspace
// plus the split-K counters, one copy per device.  static_scratch returns this
// device's addresses (hipGetSymbolAddress once per device) and, on the first
// call on a device, zeroes the counters with a kernel on stream s.
constexpr size_t kStaticScratchBytes = 8u << 20;
hipError_t static_scratch(int device, hipStream_t s, void **workspace, int **counters);
// out[b][r] = silu(gate_r . x_b) * (up_r . x_b) for 3 <= B <= 32: one MFMA
// launch whose workgroups take 128 rows of gate and the same 128 rows of up
// (Q4_K, Q5_K, Q6_K, Q8_0; full row ranges, same shape and x).
bool mfma_swiglu_applies(const MfmaDesc &gate, const MfmaDesc &up, int B);
size_t mfma_swiglu_workspace_bytes(const MfmaDesc &gate, int B);
hipError_t launch_mfma_swiglu(const MfmaDesc &gate, const MfmaDesc &up, int B, float *out, void *workspace,
                              int *counters, hipStream_t s);

// out[rows][cols] fp32, bit-exact with the reference dequantizers.
hipError_t launch_dequant(int type, const uint8_t *w, int rows, int cols, float *out, hipStream_t s);
// Rows clamp(d_tokens[y], 0, rows - 1), y < n_out, of a packed matrix with row
// pitch `pitch`, dequantized into out[y][cols].
hipError_t launch_dequant_row(int type, const uint8_t *w, int rows, int cols, size_t pitch, const int *d_tokens,
                              int n_out, float *out, hipStream_t s);

// n fp32 values -> packed blocks with the LoraMerge quantizers.
hipError_t launch_quantize(int type, const float *src, int64_t n, uint8_t *dst, hipStream_t s);

// ---- the rest of a Llama decode step (jh_decode.hip); d_pos is a device int
hipError_t launch_rmsnorm(const float *x, const float *res, const float *w, int n, int rows, float eps, float *x_out,
                          float *out, hipStream_t s);
hipError_t launch_rope_kv(float *q, const float *k, const float *v, int n_heads, int n_kv_heads, int head_dim,
                          const int *d_pos, int max_seq, float theta, float *k_cache, float *v_cache, hipStream_t s);
size_t attention_workspace_bytes(int n_heads, int head_dim, int max_seq, int batch);
// fused: q, k_new, v_new are this position's raw projections (rope + append
// inside); otherwise q is rotated and the cache already holds the position
// batch requests: q / k / v / out rows per request, d_pos[batch]; with d_slot the
// caches are [n_slots][max_seq][kv_dim] and request z uses slot d_slot[z].
hipError_t launch_attention(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                            int n_heads, int n_kv_heads, int head_dim, const int *d_pos, int max_seq, float theta,
                            bool fused, float *out, void *workspace, hipStream_t s, int batch = 1,
                            const int *d_slot = nullptr, int n_slots = 1, bool combine = true);
// the chunking launch_attention picks: chunk length *tc, *nch chunks per head
// cover max_seq (the partials' stride)
void attention_chunking(int n_heads, int n_kv_heads, int head_dim, int max_seq, int batch, int *tc, int *nch);
// Arrival counters of the MFMA split-K hand-off: kCounterSlots per stream, one
// 128-byte line each, so that workgroups arriving at different counters never
// queue on one line's atomics.  Every launch leaves the counters it used at zero.
constexpr int kCounterSlots = 1024;
constexpr int kCounterStride = 32;  // ints
hipError_t launch_silu_mul(const float *gate, const float *up, int n, float *out, hipStream_t s);
// y[b] += scale * B (A x[b]) for b < batch; h_ws holds batch * rank floats.
hipError_t launch_lora(const float *a, const float *b, int rank, int in_dim, int out_dim, float scale, const float *x,
                       int batch, float *y, float *h_ws, hipStream_t s);
// y[r][i] += bias[i] for r < rows, i < n.
hipError_t launch_add_rows(float *y, const float *bias, int n, int rows, hipStream_t s);
hipError_t launch_pos_increment(int *d_pos, int delta, hipStream_t s);

}  // namespace jh
