/* Two-pass attention: the reference's naive SDPA (h3_cuda_attention.cu:
 * 488-549), one workgroup per (query row, head), scores in LDS, normalised
 * F32 probabilities, P.V as sequential fmaf.  It serves head sizes other
 * than 128, H3_HIP_REFERENCE=1 and the naive-SDPA knob
 * (H3_CUDA_SDPA_NAIVE / H3_HIP_SDPA_NAIVE).  This file is built with the
 * default floating-point semantics (IEEE sums and division, NaNs honoured),
 * unlike the flash kernel's file, so the debugging path stays the plain
 * f32 evaluation. */
#include "hk_common.h"
#include "hk_internal.h"

#include <math.h>

/* Two-pass reference: one workgroup per (query row, head); scores in LDS. */
__global__ void __launch_bounds__(256)
hk_attn_reference(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                  uint16_t *o, uint32_t q_rows, uint32_t kv_rows,
                  uint32_t heads, uint32_t head_dim, float scale,
                  int head_major) {
    extern __shared__ float scores[];
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x, head = blockIdx.y;
    const size_t q_base = ((size_t)row * heads + head) * head_dim;
    float local_max = -INFINITY;
    for (uint32_t key = threadIdx.x; key < kv_rows; key += blockDim.x) {
        const size_t k_base = ((size_t)key * heads + head) * head_dim;
        float dot = 0.0f;
        for (uint32_t d = 0; d < head_dim; d++)
            dot = fmaf(hk_bf2f(q[q_base + d]), hk_bf2f(k[k_base + d]), dot);
        dot *= scale;
        scores[key] = dot;
        local_max = fmaxf(local_max, dot);
    }
    /* block max through the sum helper's pattern */
    local_max = hk_wave_max(local_max);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = local_max;
    __syncthreads();
    float maximum = -INFINITY;
    for (uint32_t w = 0; w < (blockDim.x >> 6); w++)
        maximum = fmaxf(maximum, scratch[w]);
    float local_sum = 0.0f;
    for (uint32_t key = threadIdx.x; key < kv_rows; key += blockDim.x) {
        float p = expf(scores[key] - maximum);
        scores[key] = p;
        local_sum += p;
    }
    const float inverse = 1.0f / hk_block_sum(local_sum, scratch);
    for (uint32_t d = threadIdx.x; d < head_dim; d += blockDim.x) {
        float sum = 0.0f;
        for (uint32_t key = 0; key < kv_rows; key++)
            sum = fmaf(scores[key] * inverse,
                       hk_bf2f(v[((size_t)key * heads + head) * head_dim + d]),
                       sum);
        const size_t out = head_major
            ? ((size_t)head * q_rows + row) * head_dim + d
            : q_base + d;
        o[out] = hk_f2bf(sum);
    }
}

int hk_attention_reference(struct h3_gpu *gpu, const uint16_t *q,
                           const uint16_t *k, const uint16_t *v, uint16_t *o,
                           uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                           uint32_t head_dim, float scale, int head_major) {
    if ((size_t)kv_rows * sizeof(float) > 64 * 1024)
        return hk_fail(gpu, "reference attention supports at most 16384 keys");
    hipLaunchKernelGGL(hk_attn_reference, dim3(q_rows, heads), dim3(256),
                       (size_t)(kv_rows ? kv_rows : 1) * sizeof(float),
                       gpu->stream, q, k, v, o, q_rows, kv_rows, heads,
                       head_dim, scale, head_major);
    return 1;
}
