/* Internal definitions of the MI355X HIP backend of h3_gpu.h.
 *
 * Execution model: one context owns one HIP stream (default priority) on
 * device 0.  Every op enqueues its kernels on that stream, so the stream's
 * order is the program order; h3_gpu_submit() waits for the stream.  This
 * is the same ordering contract as the reference's single in-order queue
 * (reference h3_cuda_internal.h:1-5, h3_gpu_cuda.cu:890-905).
 */
#ifndef HK_INTERNAL_H
#define HK_INTERNAL_H

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/h3_gpu.h"
#include "../../include/h3_hip.h"

struct h3_gpu_tensor {
    void *data;
    size_t elements;
    size_t bytes;
    h3_gpu_dtype dtype;
    struct h3_gpu *owner;
    /* host-side record of a grouped-linear table: the (rows, input_dim,
     * output_dim, problems) it was built and validated for; all zero for
     * every other tensor */
    uint32_t group_shape[4];
};

struct hk_cache_block;
struct hk_timing;

struct h3_gpu {
    int device;
    hipStream_t stream;
    int active;
    char error[512];
    h3_gpu_stats stats;
    double batch_start;
    char profile_label[128];
    h3_gpu_stats profile_mark_stats;
    double profile_mark_wall;
    /* exact-size cache of freed device blocks */
    struct hk_cache_block *cache;
    size_t cache_bytes;
    size_t cache_limit;
    /* grow-only device scratch for op intermediates */
    void *workspace;
    size_t workspace_bytes;
    void *splitk; /* f32 partial tiles of split-K GEMMs */
    size_t splitk_bytes;
    /* H3_HIP_REFERENCE=1: route GEMM and attention through the simple
     * (sequential-k / two-pass) reference kernels */
    int reference_kernels;
    /* per-op event timing */
    struct hk_timing *timing;
    hipEvent_t markers[16];
    int marker_valid[16];
    int num_cus;
    /* block-sparse joint attention mask (h3_gpu_sdpa_set_sparse): CSR over
     * 128-row query blocks of 64-row key tiles, each list sorted */
    uint32_t *sparse_ptr, *sparse_idx; /* device */
    uint32_t sparse_rows;
    /* file loader: pinned staging slots, copy stream, serialising lock */
    struct hk_loader *loader;
    /* hipMalloc calls made for this context (tensors, scratch, masks) */
    uint64_t device_mallocs;
};

/* stats kinds, mirroring the reference counters (h3_cuda_internal.h:142-160) */
enum { HK_KIND_DIRECT = 0, HK_KIND_LINEAR = 1, HK_KIND_CONV = 2,
       HK_KIND_SDPA = 3 };

static inline size_t hk_item_size(h3_gpu_dtype dtype) {
    return dtype == H3_GPU_BF16 ? 2 : dtype == H3_GPU_I8 ? 1 : 4;
}

static inline int hk_fail(struct h3_gpu *gpu, const char *format, ...) {
    if (gpu) {
        va_list arguments;
        va_start(arguments, format);
        vsnprintf(gpu->error, sizeof(gpu->error), format, arguments);
        va_end(arguments);
    }
    return 0;
}

static inline int hk_fail_hip(struct h3_gpu *gpu, const char *what,
                              hipError_t status) {
    return hk_fail(gpu, "HIP %s failed: %s", what, hipGetErrorString(status));
}

static inline int hk_require_active(struct h3_gpu *gpu) {
    if (!gpu || !gpu->active) return hk_fail(gpu, "no active command buffer");
    return 1;
}

static inline int hk_require(struct h3_gpu *gpu, const h3_gpu_tensor *tensor,
                             size_t elements, h3_gpu_dtype dtype,
                             const char *label) {
    if (!tensor || tensor->elements < elements)
        return hk_fail(gpu, "%s tensor is too small", label);
    if (tensor->dtype != dtype)
        return hk_fail(gpu, "%s tensor has the wrong dtype", label);
    return 1;
}

#define HK_BF16(t) ((uint16_t *)(t)->data)
#define HK_CBF16(t) ((const uint16_t *)(t)->data)
#define HK_F32(t) ((float *)(t)->data)
#define HK_CF32(t) ((const float *)(t)->data)
#define HK_CU32(t) ((const uint32_t *)(t)->data)

/* Op bracket: hk_op_begin() records a start event when timing is on;
 * hk_op_end() checks the launch, records the stop event and bumps the
 * stats counter of the given kind.  Returns 1/0 like the public ops. */
void hk_op_begin(struct h3_gpu *gpu, const char *name);
int hk_op_end(struct h3_gpu *gpu, const char *name, int kind);

/* Grow-only device scratch shared by ops of one context. */
void *hk_workspace(struct h3_gpu *gpu, size_t bytes);
/* Grow-only scratch for split-K partials, separate from the workspace
 * (which may hold a GEMM's input, e.g. the MLP activation). */
void *hk_splitk_space(struct h3_gpu *gpu, size_t bytes);

double hk_now(void);

/* ---------------------------------------------------------------- launch
 * helpers implemented in the kernel translation units.  All take device
 * pointers and enqueue on gpu->stream; shapes are validated by the caller.
 */

/* GEMM epilogues */
enum { HK_EPI_STORE = 0, HK_EPI_SWIGLU = 1, HK_EPI_GELU = 2,
       HK_EPI_PARTIAL = 3, /* internal: f32 split-K partial tiles */
       HK_EPI_PARTIAL_SWIGLU = 4 /* internal: the same, SwiGLU W rows */ };

/* C[M,N] = epi(A[M,K] . W[N,K]^T + bias).  For HK_EPI_SWIGLU the weight has
 * 2*N rows (gate rows [0,N), up rows [N,2N)) and C is the [M,N] activation.
 * Split-K partials go to the context's scratch (grown on demand), or, when
 * `scratch` is given, to that caller-owned device buffer of scratch_bytes:
 * then nothing is allocated, and a split that needs more fails. */
int hk_gemm_bf16(struct h3_gpu *gpu, const uint16_t *a, const uint16_t *w,
                 const uint16_t *bias, uint16_t *c, uint32_t m, uint32_t n,
                 uint32_t k, int epilogue, float *scratch = nullptr,
                 size_t scratch_bytes = 0);
int hk_gemm_bf16_pair(struct h3_gpu *gpu, const uint16_t *x,
                      const uint16_t *w0, const uint16_t *b0, uint16_t *c0,
                      const uint16_t *w1, const uint16_t *b1, uint16_t *c1,
                      uint32_t m, uint32_t n, uint32_t k);

/* Flash attention; q rows [q_rows][heads][hd], k/v [kv_rows][heads][hd].
 * head_major selects [heads][q_rows][hd] output. */
/* sparse: apply the registered block-sparse mask (joint attention whose
 * row count matches the registration).  rope_cos / rope_sin (bf16
 * [rows][48], self-attention only): Q and K arrive unrotated and the
 * kernel applies the RoPE pair rotation (d, d + 48), d < 48. */
int hk_attention_bf16(struct h3_gpu *gpu, const uint16_t *q,
                      const uint16_t *k, const uint16_t *v, uint16_t *o,
                      uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                      uint32_t head_dim, float scale, int head_major,
                      int sparse, const uint16_t *rope_cos = nullptr,
                      const uint16_t *rope_sin = nullptr, int fused_qkv = 0,
                      const uint16_t *q_norm = nullptr,
                      const uint16_t *q_cos = nullptr,
                      const uint16_t *q_sin = nullptr, float q_eps = 0.0f);
/* The two-pass reference attention (any head size up to 16384 keys). */
int hk_attention_reference(struct h3_gpu *gpu, const uint16_t *q,
                           const uint16_t *k, const uint16_t *v, uint16_t *o,
                           uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                           uint32_t head_dim, float scale, int head_major);

#endif
