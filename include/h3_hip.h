/* h3_hip.h - entry points of the MI355X HIP backend that the reference
 * device API (h3_gpu.h) does not have.
 *
 * None of these replaces a reference symbol.  They exist for three reasons:
 *   1. the backend probe that the engine selects per build
 *      (h3_hip_probe, counterpart of h3_cuda_probe, reference
 *      h3_cuda.h:6-8 and h3_gpu_cuda.cu:47-79);
 *   2. the ops a Wan-style DiT block needs and h3_gpu.h lacks: attention
 *      with q_rows != kv_rows, LayerNorm adaLN, a GELU-tanh FFN
 *      (the GELU formula is the reference's h3_cuda_core.cu:139-158);
 *   3. device-side seeded initialisation and per-op timing for the
 *      benchmark harness.
 * Same conventions as h3_gpu.h: 1 = success, 0 = failure + h3_gpu_error().
 */
#ifndef H3_HIP_H
#define H3_HIP_H

#include "h3_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Field-for-field layout of the engine's h3_device_info
 * (reference h3.h:137-146), so a build can alias the two. */
struct h3_hip_device_info {
    char name[128];
    char architecture[128];
    uint64_t physical_memory;
    uint64_t recommended_working_set;
    uint64_t max_buffer_length;
    int apple_gpu_family;
    int metal4;
    int unified_memory;
};

int h3_hip_probe(struct h3_hip_device_info *info, char *error,
                 size_t error_size);

/* Cross attention: Q [q_rows][heads][head_dim] against K/V
 * [kv_rows][heads][head_dim]; output [q_rows][heads][head_dim].  Same
 * numerics as h3_gpu_sdpa_bf16 (F32 online softmax, P rounded to bf16
 * before P.V). */
int h3_gpu_sdpa_cross_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *query,
                           const h3_gpu_tensor *key,
                           const h3_gpu_tensor *value, uint32_t q_rows,
                           uint32_t kv_rows, uint32_t heads,
                           uint32_t head_dim, float scale);

/* Self-attention with the 3D RoPE applied by the call: Q and K arrive
 * unrotated ([sequence][heads][head_dim] bf16, already normalised where the
 * model normalises them) and the pairs (d, d + rope_half), d < rope_half,
 * are rotated with the bf16 cos / sin tables [sequence][rope_half] -- Q
 * inside the attention kernel as its fragments are loaded, K once per key
 * row by a pre-pass into the context's scratch -- before the same
 * online-softmax attention as h3_gpu_sdpa_bf16 (the registered block-sparse
 * mask applies as there).
 * The rotation is the reference's RoPE step (h3_cuda_attention.cu:218-233)
 * rounded to bf16, so the result equals rotating Q and K first and calling
 * h3_gpu_sdpa_bf16.  Needs head_dim 128 and rope_half 48 (the 3 x 16
 * frequency tables of the H3 and Wan models).  No reference counterpart. */
int h3_hip_sdpa_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *query,
                          const h3_gpu_tensor *key,
                          const h3_gpu_tensor *value,
                          const h3_gpu_tensor *rope_cos,
                          const h3_gpu_tensor *rope_sin, uint32_t sequence,
                          uint32_t heads, uint32_t head_dim,
                          uint32_t rope_half, float scale);

/* The QKV projection output [sequence][3][heads][head_dim] (Q, K, V
 * thirds of each row, h3_gpu_qkv_rope_bf16's non-grouped layout), with Q
 * and K normalised per head and rotated in place: the arithmetic and
 * rounding of h3_gpu_qkv_rope_bf16 (the reference's qkv_rope_bf16 op,
 * h3_cuda_attention.cu:190-245), written over Q and K instead of into
 * separate tensors, and V left where it is.  Needs head_dim 128, rope_half
 * a multiple of 8 and 16-byte aligned tensors.  With h3_hip_sdpa_qkv_bf16
 * it saves the copy of Q, K and V out of the fused rows.  No reference
 * counterpart; used by this backend's Wan-shaped block. */
int h3_hip_qk_norm_rope_inplace_bf16(h3_gpu *gpu, h3_gpu_tensor *qkv,
                                     const h3_gpu_tensor *q_norm,
                                     const h3_gpu_tensor *k_norm,
                                     const h3_gpu_tensor *rope_cos,
                                     const h3_gpu_tensor *rope_sin,
                                     uint32_t sequence, uint32_t heads,
                                     uint32_t head_dim, uint32_t rope_half,
                                     float epsilon, int keys_only);

/* The same over K alone (keys_only != 0) leaves Q as the projection wrote
 * it, for h3_hip_sdpa_qkv_norm_rope_bf16. */

/* h3_gpu_sdpa_bf16 with Q, K and V read from the fused rows
 * [sequence][3][heads][head_dim] (as left by
 * h3_hip_qk_norm_rope_inplace_bf16); same kernel, same result as on the
 * three separate tensors.  Needs head_dim 128 and 16-byte aligned rows.
 * No reference counterpart; used by this backend's Wan-shaped block. */
int h3_hip_sdpa_qkv_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         const h3_gpu_tensor *qkv, uint32_t sequence,
                         uint32_t heads, uint32_t head_dim, float scale);

/* h3_hip_sdpa_qkv_bf16 on fused rows whose Q is still as the projection
 * wrote it (K normalised and rotated, e.g. by the keys-only in-place
 * pass): the attention kernel applies Q's per-head RMS norm (weight
 * q_norm, epsilon) and, with rope_cos / rope_sin ([sequence][48] bf16, or
 * both NULL), the RoPE pairs (d, d + 48) as it loads Q -- the arithmetic
 * and rounding of h3_gpu_qkv_rope_bf16 (reference h3_cuda_attention.cu:
 * 190-245), so the result equals normalising and rotating Q first.  Needs
 * head_dim 128 and 16-byte aligned tensors.  No reference counterpart;
 * used by this backend's Wan-shaped block. */
int h3_hip_sdpa_qkv_norm_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                   const h3_gpu_tensor *qkv,
                                   const h3_gpu_tensor *q_norm,
                                   const h3_gpu_tensor *rope_cos,
                                   const h3_gpu_tensor *rope_sin,
                                   uint32_t sequence, uint32_t heads,
                                   uint32_t head_dim, uint32_t rope_half,
                                   float epsilon, float scale);

/* h3_gpu_sdpa_cross_bf16 with the per-head RMS norm of Q (weight q_norm,
 * epsilon) applied by the attention kernel as it loads Q: the arithmetic
 * and rounding of h3_gpu_head_rms_norm_bf16, so the result equals
 * normalising Q first.  Needs head_dim 128 and 16-byte aligned tensors.
 * No reference counterpart (the reference has no cross-attention); used
 * by this backend's Wan-shaped block. */
int h3_hip_sdpa_cross_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                const h3_gpu_tensor *query,
                                const h3_gpu_tensor *key,
                                const h3_gpu_tensor *value,
                                const h3_gpu_tensor *q_norm, uint32_t q_rows,
                                uint32_t kv_rows, uint32_t heads,
                                uint32_t head_dim, float epsilon,
                                float scale);

/* LayerNorm adaLN:
 *   n = (x - mean) * rsqrt(var + eps) [* w + b]      (w, b may be NULL)
 *   y = bf16(n * (1 + mod[scale]) + mod[shift])
 * with the modulation row chosen per token by row_map, as in
 * h3_gpu_adaln_bf16.  A NULL modulation (and row_map) gives a plain
 * LayerNorm. */
int h3_gpu_layer_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *norm_weight,
                            const h3_gpu_tensor *norm_bias,
                            const h3_gpu_tensor *modulation,
                            const h3_gpu_tensor *row_map, uint32_t rows,
                            uint32_t width, uint32_t slots,
                            uint32_t shift_slot, uint32_t scale_slot,
                            float epsilon);

/* Residual update and LayerNorm adaLN in one row pass, for pre-norm blocks
 * whose residual update feeds the next norm:
 *   gated_residual = bf16(residual + branch * mod[gate_slot])
 *                    (a NULL gate_modulation gives bf16(residual + branch))
 *   output = h3_gpu_layer_adaln_bf16 of gated_residual
 * Bit-identical to h3_gpu_gate_bf16 (or h3_gpu_add_bf16) followed by
 * h3_gpu_layer_adaln_bf16; gated_residual may alias residual.  No reference
 * counterpart: the reference fuses the gate only with its RMS adaLN
 * (h3_gpu_gate_adaln_bf16). */
int h3_gpu_gate_layer_adaln_bf16(
    h3_gpu *gpu, h3_gpu_tensor *gated_residual, h3_gpu_tensor *output,
    const h3_gpu_tensor *residual, const h3_gpu_tensor *branch,
    const h3_gpu_tensor *gate_modulation, const h3_gpu_tensor *norm_weight,
    const h3_gpu_tensor *norm_bias, const h3_gpu_tensor *norm_modulation,
    const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width,
    uint32_t slots, uint32_t gate_slot, uint32_t shift_slot,
    uint32_t scale_slot, float epsilon);

/* A group of projections of one input and one shape, output_p = X .
 * weight_p^T + bias_p for p < count, as one launch: the table
 * h3_hip_linear_group_table builds holds the problems' device addresses
 * (free it with h3_gpu_tensor_free; it stays valid while the tensors
 * live), and h3_hip_linear_group_bf16 runs problems [first, first + count)
 * of it on `input`, with the rows, input_dim and output_dim the table was
 * built with (another shape, or problems past the table's count, fail with
 * an error: the table's addresses were validated for that shape only).
 * Tensors must meet the MFMA kernel's alignment (16-byte
 * weights, 8-byte outputs and biases), which the table checks.  Each
 * output is exactly what h3_gpu_linear_bf16 computes with the data-
 * parallel kernel.  Biases may be NULL (or the array NULL).  No reference
 * counterpart: the Wan-shaped driver projects the text into every block's
 * cross-attention K and V with one launch. */
h3_gpu_tensor *h3_hip_linear_group_table(h3_gpu *gpu,
                                         h3_gpu_tensor *const *outputs,
                                         const h3_gpu_tensor *const *weights,
                                         const h3_gpu_tensor *const *biases,
                                         uint32_t count, uint32_t rows,
                                         uint32_t input_dim,
                                         uint32_t output_dim);
int h3_hip_linear_group_bf16(h3_gpu *gpu, const h3_gpu_tensor *table,
                             uint32_t first, uint32_t count,
                             const h3_gpu_tensor *input, uint32_t rows,
                             uint32_t input_dim, uint32_t output_dim);

/* A group of per-head RMS norms of one shape (rows x heads x head_dim, in
 * place), each tensor with its own weight, as one launch: the table
 * h3_hip_head_norm_group_table builds holds the problems' device addresses
 * (free it with h3_gpu_tensor_free), and h3_hip_head_rms_norm_group_bf16
 * normalises problems [first, first + count) of it, at the shape the table
 * was built with (another shape fails with an error).  head_dim 128 and
 * 16-byte aligned tensors only.  Each result is bit-identical to
 * h3_gpu_head_rms_norm_bf16 on that tensor.  No reference counterpart: the
 * Wan-shaped driver normalises every block's text keys with one launch. */
h3_gpu_tensor *h3_hip_head_norm_group_table(
    h3_gpu *gpu, h3_gpu_tensor *const *tensors,
    const h3_gpu_tensor *const *weights, uint32_t count, uint32_t rows,
    uint32_t heads, uint32_t head_dim);
int h3_hip_head_rms_norm_group_bf16(h3_gpu *gpu, const h3_gpu_tensor *table,
                                    uint32_t first, uint32_t count,
                                    uint32_t rows, uint32_t heads,
                                    uint32_t head_dim, float epsilon);

/* Two projections of one input, output0 = X . weight0^T + bias0 and
 * output1 = X . weight1^T + bias1, each exactly as h3_gpu_linear_bf16
 * computes it (f32 accumulation, one bf16 rounding).  Small launches
 * (together at most half the CUs' worth of 256x256 tiles, such as the
 * text's cross-attention K and V) share one split-K launch; others run as
 * two linears.  Biases may be NULL.  No reference counterpart: the
 * reference has no cross-attention. */
int h3_hip_linear_pair_bf16(h3_gpu *gpu, h3_gpu_tensor *output0,
                            h3_gpu_tensor *output1,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *weight0,
                            const h3_gpu_tensor *bias0,
                            const h3_gpu_tensor *weight1,
                            const h3_gpu_tensor *bias1, uint32_t rows,
                            uint32_t input_dim, uint32_t output_dim);

/* h3_gpu_linear_bf16 that allocates nothing: the same kernels and the same
 * results, with the split-K partial tiles (used when the last round of
 * 256x256 tiles would leave over half the CUs idle) in a static 64 MiB
 * device array per GPU instead of the context's on-demand scratch.  A
 * launch whose split would need more fails with an error naming the size.
 * The array (256 CUs x one 256x256 f32 tile) is resident on every GPU the
 * library loads on, whether or not this entry is called.  Calls that
 * overlap on one GPU share that array and race.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory
 * (fixed-footprint serving loops, harnesses that forbid hipMalloc); it
 * makes no device allocation, but recording it into a HIP graph is not
 * tested. */
int h3_hip_linear_bf16_noalloc(h3_gpu *gpu, h3_gpu_tensor *output,
                               const h3_gpu_tensor *input,
                               const h3_gpu_tensor *weight,
                               const h3_gpu_tensor *bias, uint32_t rows,
                               uint32_t input_dim, uint32_t output_dim);

/* output = bf16(gelu_tanh(bf16(X . W^T + b))): GEMM with the activation in
 * its epilogue. */
int h3_gpu_linear_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *weight,
                            const h3_gpu_tensor *bias, uint32_t rows,
                            uint32_t input_dim, uint32_t output_dim);

/* h3_gpu_patch_linear_bf16_offset / _map (h3_gpu.h:116-135) without the
 * reference's fixed checkpoint shape (5376 outputs from 32 or 96 inputs):
 * any output width and up to 4096 inputs, for reduced-width test models.
 * The h3_gpu_ entries keep the reference's check. */
int h3_hip_patch_linear_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output,
                                    size_t output_offset,
                                    const h3_gpu_tensor *input,
                                    size_t input_offset,
                                    const h3_gpu_tensor *weight,
                                    const h3_gpu_tensor *bias, uint32_t rows,
                                    uint32_t input_dim, uint32_t output_dim);
int h3_hip_patch_linear_bf16_map(h3_gpu *gpu, h3_gpu_tensor *output,
                                 const h3_gpu_tensor *input,
                                 const h3_gpu_tensor *weight,
                                 const h3_gpu_tensor *bias,
                                 const h3_gpu_tensor *row_map,
                                 uint32_t output_rows, uint32_t rows,
                                 uint32_t input_dim, uint32_t output_dim);

/* Non-gated GELU-tanh FFN: fc2(gelu(fc1(x) + b1)) + b2.  activated is
 * caller-owned scratch of rows*hidden_dim bf16, or NULL to use the
 * context's workspace.  Biases may be NULL. */
int h3_gpu_ffn_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         h3_gpu_tensor *activated,
                         const h3_gpu_tensor *input,
                         const h3_gpu_tensor *fc1_weight,
                         const h3_gpu_tensor *fc1_bias,
                         const h3_gpu_tensor *fc2_weight,
                         const h3_gpu_tensor *fc2_bias, uint32_t rows,
                         uint32_t input_dim, uint32_t hidden_dim,
                         uint32_t output_dim);

/* Seeded N(mean, stddev^2) fill of elements values starting at offset,
 * generated on the device (counter-based: value i depends only on seed and
 * i).  Used to initialise resident random weights without host uploads. */
int h3_gpu_fill_normal_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor,
                            size_t offset, size_t elements, uint64_t seed,
                            float mean, float stddev);
int h3_gpu_fill_normal_f32(h3_gpu *gpu, h3_gpu_tensor *tensor,
                           size_t offset, size_t elements, uint64_t seed,
                           float mean, float stddev);

/* Per-op device timing.  While enabled, every launch is bracketed by a pair
 * of HIP events on the context's stream; h3_hip_op_timing_read() waits for
 * the stream and returns the number of launches and their summed device
 * milliseconds for the ops whose name starts with prefix ("" = all). */
int h3_hip_op_timing_enable(h3_gpu *gpu, int enable);
int h3_hip_op_timing_reset(h3_gpu *gpu);
int h3_hip_op_timing_read(h3_gpu *gpu, const char *prefix,
                          uint64_t *count, double *milliseconds);
/* Names of the distinct timed ops, '\n'-separated, into buffer. */
int h3_hip_op_timing_names(h3_gpu *gpu, char *buffer, size_t buffer_size);

/* Launches the measured-peak kernel: one workgroup of four waves per CU,
 * each wave issuing `iterations` x 16 bf16 MFMAs (32x32x16) from registers
 * with no LDS or memory traffic; `sink` (F32, at least CUs x 256
 * elements) receives the sums.  *flops is the launch's FLOP count, so a
 * caller timing it between two markers gets the sustained MFMA rate.  No
 * reference counterpart: the benchmark reports it beside the vendor peak. */
int h3_hip_mfma_loop(h3_gpu *gpu, h3_gpu_tensor *sink, uint32_t iterations,
                     double *flops);

/* Device milliseconds between two markers recorded on the context stream. */
int h3_hip_marker(h3_gpu *gpu, int slot);
int h3_hip_marker_elapsed(h3_gpu *gpu, int from_slot, int to_slot,
                          double *milliseconds);

/* Number of device allocations (hipMalloc calls: tensors, op scratch,
 * sparse masks) this context has made so far, cached-block reuse not
 * counted.  Lets a caller that must not allocate inside a loop check that
 * it did not. */
uint64_t h3_hip_device_allocations(const h3_gpu *gpu);

#ifdef __cplusplus
}
#endif

#endif
