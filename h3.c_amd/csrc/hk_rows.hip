/* Memory-bound kernels of the DiT path for gfx950: adaLN / gated residual /
 * fused gate+adaLN rows, RMS and Layer norms, Q/K norm + 3D RoPE, SwiGLU,
 * GELU, casts, residual add/sub, the Euler sampler step, patch projection,
 * the fused final adaLN head and seeded device initialisation.
 *
 * Layout choices (MI355X-first): one workgroup of 256 threads per token row,
 * 16-byte loads/stores (8 bf16 per thread per chunk), the whole row kept in
 * registers between the reduction and the output pass (a 5376-wide row is
 * 2.6 chunks per thread), wave64 shuffles for the reductions.  The
 * modulation rows are addressed as mod[row_map[r]][slot][width] exactly as
 * the reference kernels do (h3_cuda_dit.cu:141-332).
 *
 * Numerics: F32 math on exactly-widened bf16, one RNE rounding per output,
 * 1/sqrtf(mean + eps) as the inverse RMS (reference h3_cuda_dit.cu:160-161).
 * Reductions run in wave-tree order, which is within one bf16 ulp of the
 * reference's block-tree order (reference tests' contract,
 * tests/test_cuda_dit.c:57-71).
 */
#include "hk_common.h"
#include "hk_internal.h"

#include <math.h>

#define HK_ROW_THREADS 256
#define HK_ROW_CHUNKS 4 /* register-resident rows up to 256*4*8 = 8192 */
#ifndef HK_K_ITEMS
#define HK_K_ITEMS 2 /* (row, head) vectors per lane group, in-place K: 2 beat 1, 4 and 8 */
#endif

/* ------------------------------------------------------------ row kernel */

enum {
    HK_ROW_GATE = 1,    /* x = bf16(residual + branch * mod[gate]) first */
    HK_ROW_LAYER = 2,   /* LayerNorm statistics instead of RMS */
    HK_ROW_WEIGHT = 4,  /* multiply by the norm weight */
    HK_ROW_BIAS = 8,    /* add the norm bias (LayerNorm) */
    HK_ROW_MOD = 16,    /* y = n * (1 + mod[scale]) + mod[shift] */
    HK_ROW_NORM = 32,   /* produce a normalised output at all */
};

struct hk_row_args {
    const uint16_t *input;      /* residual for GATE */
    const uint16_t *branch;
    const uint16_t *weight;
    const uint16_t *bias;
    const uint16_t *gate_mod;
    const uint16_t *norm_mod;
    const uint32_t *row_map;
    uint16_t *gated;            /* GATE output (may alias input) */
    uint16_t *output;
    uint32_t rows, width, slots, gate_slot, shift_slot, scale_slot;
    float epsilon;
};

/* Vectorised row op: width % 8 == 0 and width <= 8192. */
template <int MODE>
__global__ void __launch_bounds__(HK_ROW_THREADS)
hk_row_vec(hk_row_args a) {
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const size_t row_off = (size_t)row * a.width;
    /* GATE with a null gate modulation is a plain residual add */
    const bool gated = (MODE & HK_ROW_GATE) && a.gate_mod;
    size_t mod_base = 0;
    if ((MODE & HK_ROW_MOD) || gated)
        mod_base = (size_t)a.row_map[row] * a.slots * a.width;
    float v[HK_ROW_CHUNKS][8];
    float local = 0.0f;
#pragma unroll
    for (int c = 0; c < HK_ROW_CHUNKS; c++) {
        const uint32_t col = (tid + (uint32_t)c * HK_ROW_THREADS) * 8;
        if (col < a.width) {
            hk_unpack8(*(const uint4 *)(a.input + row_off + col), v[c]);
            if (MODE & HK_ROW_GATE) {
                float b[8], g[8];
                hk_unpack8(*(const uint4 *)(a.branch + row_off + col), b);
                if (gated) {
                    hk_unpack8(*(const uint4 *)(a.gate_mod + mod_base +
                                                (size_t)a.gate_slot * a.width +
                                                col), g);
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        v[c][i] = v[c][i] + b[i] * g[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[c][i] = v[c][i] + b[i];
                }
                uint4 packed = hk_pack8(v[c]);
                *(uint4 *)(a.gated + row_off + col) = packed;
                hk_unpack8(packed, v[c]); /* continue from the rounded row */
            }
#pragma unroll
            for (int i = 0; i < 8; i++)
                local = (MODE & HK_ROW_LAYER) ? local + v[c][i]
                                              : fmaf(v[c][i], v[c][i], local);
        }
    }
    if (!(MODE & HK_ROW_NORM)) return;
    float mean = 0.0f, inverse;
    if (MODE & HK_ROW_LAYER) {
        mean = hk_block_sum(local, scratch) / (float)a.width;
        float square = 0.0f;
#pragma unroll
        for (int c = 0; c < HK_ROW_CHUNKS; c++) {
            const uint32_t col = (tid + (uint32_t)c * HK_ROW_THREADS) * 8;
            if (col < a.width) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float centered = v[c][i] - mean;
                    square = fmaf(centered, centered, square);
                }
            }
        }
        inverse = 1.0f / sqrtf(hk_block_sum(square, scratch) /
                               (float)a.width + a.epsilon);
    } else {
        inverse = 1.0f / sqrtf(hk_block_sum(local, scratch) /
                               (float)a.width + a.epsilon);
    }
#pragma unroll
    for (int c = 0; c < HK_ROW_CHUNKS; c++) {
        const uint32_t col = (tid + (uint32_t)c * HK_ROW_THREADS) * 8;
        if (col < a.width) {
            float w[8], b[8], shift[8], scale[8], y[8];
            if (MODE & HK_ROW_WEIGHT)
                hk_unpack8(*(const uint4 *)(a.weight + col), w);
            if (MODE & HK_ROW_BIAS)
                hk_unpack8(*(const uint4 *)(a.bias + col), b);
            if (MODE & HK_ROW_MOD) {
                hk_unpack8(*(const uint4 *)(a.norm_mod + mod_base +
                                            (size_t)a.shift_slot * a.width +
                                            col), shift);
                hk_unpack8(*(const uint4 *)(a.norm_mod + mod_base +
                                            (size_t)a.scale_slot * a.width +
                                            col), scale);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float n = (MODE & HK_ROW_LAYER) ? (v[c][i] - mean) * inverse
                                                : v[c][i] * inverse;
                if ((MODE & HK_ROW_WEIGHT) && (MODE & HK_ROW_BIAS))
                    n = fmaf(n, w[i], b[i]);
                else if (MODE & HK_ROW_WEIGHT)
                    n = n * w[i];
                else if (MODE & HK_ROW_BIAS)
                    n = n + b[i];
                if (MODE & HK_ROW_MOD) n = n * (1.0f + scale[i]) + shift[i];
                y[i] = n;
            }
            *(uint4 *)(a.output + row_off + col) = hk_pack8(y);
        }
    }
}

/* Scalar row op for any width (two passes over global memory). */
template <int MODE>
__global__ void __launch_bounds__(HK_ROW_THREADS)
hk_row_scalar(hk_row_args a) {
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x;
    const size_t row_off = (size_t)row * a.width;
    const bool gated = (MODE & HK_ROW_GATE) && a.gate_mod;
    size_t mod_base = 0;
    if ((MODE & HK_ROW_MOD) || gated)
        mod_base = (size_t)a.row_map[row] * a.slots * a.width;
    const uint16_t *x = (MODE & HK_ROW_GATE) ? a.gated : a.input;
    float local = 0.0f;
    for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x) {
        float value = hk_bf2f(a.input[row_off + col]);
        if (MODE & HK_ROW_GATE) {
            const float b = hk_bf2f(a.branch[row_off + col]);
            uint16_t rounded;
            if (gated) {
                float g = hk_bf2f(a.gate_mod[mod_base +
                                  (size_t)a.gate_slot * a.width + col]);
                rounded = hk_f2bf(value + b * g);
            } else {
                rounded = hk_f2bf(value + b);
            }
            a.gated[row_off + col] = rounded;
            value = hk_bf2f(rounded);
        }
        local = (MODE & HK_ROW_LAYER) ? local + value
                                      : fmaf(value, value, local);
    }
    if (!(MODE & HK_ROW_NORM)) return;
    float mean = 0.0f, inverse;
    if (MODE & HK_ROW_LAYER) {
        mean = hk_block_sum(local, scratch) / (float)a.width;
        float square = 0.0f;
        for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x) {
            float centered = hk_bf2f(x[row_off + col]) - mean;
            square = fmaf(centered, centered, square);
        }
        inverse = 1.0f / sqrtf(hk_block_sum(square, scratch) /
                               (float)a.width + a.epsilon);
    } else {
        inverse = 1.0f / sqrtf(hk_block_sum(local, scratch) /
                               (float)a.width + a.epsilon);
    }
    for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x) {
        float value = hk_bf2f(x[row_off + col]);
        float n = (MODE & HK_ROW_LAYER) ? (value - mean) * inverse
                                        : value * inverse;
        if ((MODE & HK_ROW_WEIGHT) && (MODE & HK_ROW_BIAS))
            n = fmaf(n, hk_bf2f(a.weight[col]), hk_bf2f(a.bias[col]));
        else if (MODE & HK_ROW_WEIGHT)
            n = n * hk_bf2f(a.weight[col]);
        else if (MODE & HK_ROW_BIAS)
            n = n + hk_bf2f(a.bias[col]);
        if (MODE & HK_ROW_MOD) {
            float shift = hk_bf2f(a.norm_mod[mod_base +
                                  (size_t)a.shift_slot * a.width + col]);
            float scale = hk_bf2f(a.norm_mod[mod_base +
                                  (size_t)a.scale_slot * a.width + col]);
            n = n * (1.0f + scale) + shift;
        }
        a.output[row_off + col] = hk_f2bf(n);
    }
}

template <int MODE>
static void hk_row_launch(struct h3_gpu *gpu, const hk_row_args &args) {
    if (!args.rows || !args.width) return;
    const bool aligned =
        args.width % 8 == 0 && args.width <= HK_ROW_THREADS * HK_ROW_CHUNKS * 8 &&
        ((uintptr_t)args.input & 15) == 0 && ((uintptr_t)args.output & 15) == 0;
    if (aligned)
        hipLaunchKernelGGL(hk_row_vec<MODE>, dim3(args.rows),
                           dim3(HK_ROW_THREADS), 0, gpu->stream, args);
    else
        hipLaunchKernelGGL(hk_row_scalar<MODE>, dim3(args.rows),
                           dim3(HK_ROW_THREADS), 0, gpu->stream, args);
}

/* --------------------------------------------------------- F32 row ops */

struct hk_row32_args {
    const float *input, *branch, *weight, *bias, *modulation;
    const uint32_t *row_map;
    float *output;
    uint32_t rows, width, slots, shift_slot, scale_slot, gate_slot;
    float epsilon;
    int mode; /* 0 rms(w), 1 adaLN, 2 layer norm (w,b) */
};

__global__ void __launch_bounds__(HK_ROW_THREADS)
hk_row_f32(hk_row32_args a) {
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x;
    const float *x = a.input + (size_t)row * a.width;
    float local = 0.0f;
    for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x)
        local = a.mode == 2 ? local + x[col] : fmaf(x[col], x[col], local);
    float mean = 0.0f, inverse;
    if (a.mode == 2) {
        mean = hk_block_sum(local, scratch) / (float)a.width;
        float square = 0.0f;
        for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x) {
            float centered = x[col] - mean;
            square = fmaf(centered, centered, square);
        }
        inverse = 1.0f / sqrtf(hk_block_sum(square, scratch) /
                               (float)a.width + a.epsilon);
    } else {
        inverse = 1.0f / sqrtf(hk_block_sum(local, scratch) /
                               (float)a.width + a.epsilon);
    }
    size_t base = a.mode == 1 ? (size_t)a.row_map[row] * a.slots * a.width : 0;
    for (uint32_t col = threadIdx.x; col < a.width; col += blockDim.x) {
        float y;
        if (a.mode == 2) {
            y = (x[col] - mean) * inverse * a.weight[col] + a.bias[col];
        } else {
            y = x[col] * inverse * a.weight[col];
            if (a.mode == 1)
                y = y * (1.0f + a.modulation[base +
                                 (size_t)a.scale_slot * a.width + col]) +
                    a.modulation[base + (size_t)a.shift_slot * a.width + col];
        }
        a.output[(size_t)row * a.width + col] = y;
    }
}

__global__ void hk_gate_f32_kernel(const float *residual, const float *branch,
                                   const float *modulation,
                                   const uint32_t *row_map, float *output,
                                   uint32_t rows, uint32_t width,
                                   uint32_t slots, uint32_t gate_slot) {
    size_t index = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (index >= (size_t)rows * width) return;
    uint32_t row = (uint32_t)(index / width), col = (uint32_t)(index % width);
    float gate = modulation[(size_t)row_map[row] * slots * width +
                            (size_t)gate_slot * width + col];
    output[index] = residual[index] + branch[index] * gate;
}

/* ------------------------------------------------------ elementwise ops */

enum {
    HK_EW_SILU_BF16, HK_EW_SILU_F32, HK_EW_ADD_BF16, HK_EW_SUB_BF16,
    HK_EW_SILU_MUL_BF16, HK_EW_CAST_F2B, HK_EW_CAST_B2F, HK_EW_GELU_TANH,
    HK_EW_GELU_ERF
};

__device__ __forceinline__ float hk_silu(float x) {
    return x / (1.0f + expf(-x));
}

/* GELU, tanh form and erf form, with the reference's +-10 saturation
 * (reference h3_cuda_core.cu:139-158).  The erf form uses the
 * Abramowitz-Stegun 7.1.26 polynomial, as the reference does. */
__device__ __forceinline__ float hk_gelu_tanh(float x) {
    float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return inner <= -10.0f ? 0.0f
         : inner >= 10.0f  ? x
                           : 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float hk_erf_as(float value) {
    float sign = value < 0.0f ? -1.0f : 1.0f;
    float x = fabsf(value);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float poly = (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) *
                   t - 0.284496736f) * t + 0.254829592f) * t;
    return sign * (1.0f - poly * expf(-x * x));
}

__device__ __forceinline__ float hk_gelu_erf(float x) {
    return x <= -10.0f ? 0.0f
         : x >= 10.0f  ? x
                       : 0.5f * x * (1.0f + hk_erf_as(x * 0.7071067811865475f));
}

template <int OP>
__global__ void hk_elementwise(const void *left, const void *right, void *out,
                               size_t count) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        if (OP == HK_EW_SILU_F32) {
            ((float *)out)[i] = hk_silu(((const float *)left)[i]);
        } else if (OP == HK_EW_CAST_F2B) {
            ((uint16_t *)out)[i] = hk_f2bf(((const float *)left)[i]);
        } else if (OP == HK_EW_CAST_B2F) {
            ((float *)out)[i] = hk_bf2f(((const uint16_t *)left)[i]);
        } else {
            float x = hk_bf2f(((const uint16_t *)left)[i]);
            float y = 0.0f;
            if (OP == HK_EW_SILU_BF16) y = hk_silu(x);
            if (OP == HK_EW_GELU_TANH) y = hk_gelu_tanh(x);
            if (OP == HK_EW_GELU_ERF) y = hk_gelu_erf(x);
            if (OP == HK_EW_ADD_BF16)
                y = x + hk_bf2f(((const uint16_t *)right)[i]);
            if (OP == HK_EW_SUB_BF16)
                y = x - hk_bf2f(((const uint16_t *)right)[i]);
            if (OP == HK_EW_SILU_MUL_BF16)
                y = hk_silu(x) * hk_bf2f(((const uint16_t *)right)[i]);
            ((uint16_t *)out)[i] = hk_f2bf(y);
        }
    }
}

/* bf16 -> bf16 ops, 8 elements (16 bytes) per thread and step; the last
 * count % 8 elements go to the first threads of the grid. */
template <int OP>
__device__ __forceinline__ float hk_ew_bf16(float x, float y) {
    if (OP == HK_EW_SILU_BF16) return hk_silu(x);
    if (OP == HK_EW_GELU_TANH) return hk_gelu_tanh(x);
    if (OP == HK_EW_GELU_ERF) return hk_gelu_erf(x);
    if (OP == HK_EW_ADD_BF16) return x + y;
    if (OP == HK_EW_SUB_BF16) return x - y;
    return hk_silu(x) * y; /* HK_EW_SILU_MUL_BF16 */
}

template <int OP>
__global__ void __launch_bounds__(256)
hk_elementwise8(const uint16_t *left, const uint16_t *right, uint16_t *out,
                size_t count) {
    constexpr bool binary = OP == HK_EW_ADD_BF16 || OP == HK_EW_SUB_BF16 ||
                            OP == HK_EW_SILU_MUL_BF16;
    const size_t chunks = count / 8;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const size_t first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (size_t c = first; c < chunks; c += stride) {
        const uint4 a = ((const uint4 *)left)[c];
        uint4 b = make_uint4(0, 0, 0, 0);
        if (binary) b = ((const uint4 *)right)[c];
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
        const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
        uint32_t ow[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            ow[e] = hk_pack2(
                hk_ew_bf16<OP>(hk_bf2f(aw[e] & 0xffffu),
                               hk_bf2f(bw[e] & 0xffffu)),
                hk_ew_bf16<OP>(hk_bf2f(aw[e] >> 16), hk_bf2f(bw[e] >> 16)));
        ((uint4 *)out)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
    const size_t tail = chunks * 8 + first;
    if (tail < count)
        out[tail] = hk_f2bf(
            hk_ew_bf16<OP>(hk_bf2f(left[tail]),
                           binary ? hk_bf2f(right[tail]) : 0.0f));
}

template <int OP>
static void hk_ew_launch(struct h3_gpu *gpu, const void *left,
                         const void *right, void *out, size_t count) {
    if (!count) return;
    constexpr bool bf16_out = OP == HK_EW_SILU_BF16 ||
                              OP == HK_EW_GELU_TANH ||
                              OP == HK_EW_GELU_ERF || OP == HK_EW_ADD_BF16 ||
                              OP == HK_EW_SUB_BF16 ||
                              OP == HK_EW_SILU_MUL_BF16;
    const uintptr_t bases = (uintptr_t)left | (uintptr_t)right |
                            (uintptr_t)out;
    if (bf16_out && (bases & 15u) == 0) {
        size_t blocks = (count / 8 + 255) / 256;
        const size_t cap = (size_t)gpu->num_cus * 8;
        if (blocks > cap) blocks = cap;
        if (blocks == 0) blocks = 1;
        hipLaunchKernelGGL(hk_elementwise8<OP>, dim3((unsigned)blocks),
                           dim3(256), 0, gpu->stream,
                           (const uint16_t *)left, (const uint16_t *)right,
                           (uint16_t *)out, count);
        return;
    }
    size_t blocks = (count + 255) / 256;
    size_t cap = (size_t)gpu->num_cus * 16;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(hk_elementwise<OP>, dim3((unsigned)blocks), dim3(256),
                       0, gpu->stream, left, right, out, count);
}

/* SwiGLU over a fused [rows, 2*width] tensor: gate columns first. */
template <typename T>
__global__ void hk_swiglu_kernel(const T *fused, T *out, uint32_t rows,
                                 uint32_t width) {
    size_t index = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (index >= (size_t)rows * width) return;
    size_t row = index / width, col = index % width;
    size_t base = row * width * 2;
    if constexpr (sizeof(T) == 2) {
        float g = hk_bf2f(fused[base + col]);
        float u = hk_bf2f(fused[base + width + col]);
        out[index] = hk_f2bf(hk_silu(g) * u);
    } else {
        float g = fused[base + col], u = fused[base + width + col];
        out[index] = hk_silu(g) * u;
    }
}

/* Euler step from bf16 velocity caches into an f32 sample range
 * (reference h3_cuda_dit.cu:536-548). */
__global__ void hk_euler_kernel(float *sample, const uint16_t *last,
                                const uint16_t *previous, uint32_t count,
                                float delta, float ratio) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float v = hk_bf2f(last[i]);
    float velocity = fmaf(ratio, v - hk_bf2f(previous[i]), v);
    sample[i] = fmaf(delta, velocity, sample[i]);
}

/* ------------------------------------------------- Q/K norm + 3D RoPE */

/* One wave64 per (row, head) for head_dim 128: lane l owns dims 2l, 2l+1 of
 * q, k and v.  Per-head RMS over the 128 dims (wave reduction), weight,
 * then rotate-half RoPE on dims [0, 2*rope_half): d < rope_half pairs with
 * d + rope_half (x*c - x'*s), the next rope_half dims pair back
 * (x*c + x'*s), the rest pass through (reference
 * h3_cuda_attention.cu:175-237).  The partner lives rope_half/2 lanes
 * away. */
__global__ void __launch_bounds__(256)
hk_qk_norm_rope128(const uint16_t *__restrict__ qkv,
                   const uint16_t *__restrict__ q_weight,
                   const uint16_t *__restrict__ k_weight,
                   const uint16_t *__restrict__ rope_cos,
                   const uint16_t *__restrict__ rope_sin,
                   uint16_t *__restrict__ query, uint16_t *__restrict__ key,
                   uint16_t *__restrict__ value, uint32_t sequence,
                   uint32_t heads, uint32_t rope_half, uint32_t grouped,
                   float epsilon) {
    const uint32_t HD = 128;
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= sequence * heads) return;
    const uint32_t row = wave / heads, head = wave % heads;
    const size_t inner = (size_t)heads * HD;
    const size_t row_base = (size_t)row * inner * 3;
    size_t q_base, k_base, v_base;
    if (grouped) {
        q_base = row_base + (size_t)head * HD * 3;
        k_base = q_base + HD;
        v_base = k_base + HD;
    } else {
        q_base = row_base + (size_t)head * HD;
        k_base = q_base + inner;
        v_base = k_base + inner;
    }
    const uint32_t d0 = lane * 2;
    uint32_t qr = *(const uint32_t *)(qkv + q_base + d0);
    uint32_t kr = *(const uint32_t *)(qkv + k_base + d0);
    uint32_t vr = *(const uint32_t *)(qkv + v_base + d0);
    uint32_t qw = *(const uint32_t *)(q_weight + d0);
    uint32_t kw = *(const uint32_t *)(k_weight + d0);
    float q0 = hk_bf2f(qr & 0xffffu), q1 = hk_bf2f(qr >> 16);
    float k0 = hk_bf2f(kr & 0xffffu), k1 = hk_bf2f(kr >> 16);
    float q_sum = hk_wave_sum(fmaf(q0, q0, q1 * q1));
    float k_sum = hk_wave_sum(fmaf(k0, k0, k1 * k1));
    float q_inv = 1.0f / sqrtf(q_sum / (float)HD + epsilon);
    float k_inv = 1.0f / sqrtf(k_sum / (float)HD + epsilon);
    float qn0 = q0 * q_inv * hk_bf2f(qw & 0xffffu);
    float qn1 = q1 * q_inv * hk_bf2f(qw >> 16);
    float kn0 = k0 * k_inv * hk_bf2f(kw & 0xffffu);
    float kn1 = k1 * k_inv * hk_bf2f(kw >> 16);
    const uint32_t shift = rope_half / 2;
    int src = (int)lane;
    if (d0 < rope_half) src = (int)(lane + shift);
    else if (d0 < rope_half * 2) src = (int)(lane - shift);
    float qp0 = __shfl(qn0, src, 64), qp1 = __shfl(qn1, src, 64);
    float kp0 = __shfl(kn0, src, 64), kp1 = __shfl(kn1, src, 64);
    float qo0 = qn0, qo1 = qn1, ko0 = kn0, ko1 = kn1;
    if (d0 < rope_half * 2) {
        const bool first = d0 < rope_half;
        const uint32_t pair = first ? d0 : d0 - rope_half;
        const size_t table = (size_t)row * rope_half + pair;
        uint32_t cr = *(const uint32_t *)(rope_cos + table);
        uint32_t sr = *(const uint32_t *)(rope_sin + table);
        float c0 = hk_bf2f(cr & 0xffffu), c1 = hk_bf2f(cr >> 16);
        float s0 = hk_bf2f(sr & 0xffffu), s1 = hk_bf2f(sr >> 16);
        if (first) {
            qo0 = qn0 * c0 - qp0 * s0; qo1 = qn1 * c1 - qp1 * s1;
            ko0 = kn0 * c0 - kp0 * s0; ko1 = kn1 * c1 - kp1 * s1;
        } else {
            qo0 = qn0 * c0 + qp0 * s0; qo1 = qn1 * c1 + qp1 * s1;
            ko0 = kn0 * c0 + kp0 * s0; ko1 = kn1 * c1 + kp1 * s1;
        }
    }
    const size_t out = ((size_t)row * heads + head) * HD + d0;
    *(uint32_t *)(query + out) = hk_pack2(qo0, qo1);
    *(uint32_t *)(key + out) = hk_pack2(ko0, ko1);
    *(uint32_t *)(value + out) = vr;
}

/* The same with DPL dims (2·DPL bytes) per lane and 128 / DPL lanes per
 * (row, head), for rope_half % DPL == 0: the dims of a lane then sit on one
 * side of the rotate-half split and their partners rope_half / DPL lanes
 * away. */
template <int DPL> struct hk_vec_of;
template <> struct hk_vec_of<4> { typedef uint2 type; };
template <> struct hk_vec_of<8> { typedef uint4 type; };

template <int DPL>
__device__ __forceinline__ void hk_unpack(const uint16_t *p, float v[DPL]) {
    const typename hk_vec_of<DPL>::type raw =
        *(const typename hk_vec_of<DPL>::type *)p;
    const uint32_t *w = (const uint32_t *)&raw;
#pragma unroll
    for (int e = 0; e < DPL / 2; e++) {
        v[2 * e] = hk_bf2f(w[e] & 0xffffu);
        v[2 * e + 1] = hk_bf2f(w[e] >> 16);
    }
}

template <int DPL>
__device__ __forceinline__ void hk_pack_store(uint16_t *p, const float v[DPL]) {
    typename hk_vec_of<DPL>::type raw;
    uint32_t *w = (uint32_t *)&raw;
#pragma unroll
    for (int e = 0; e < DPL / 2; e++) w[e] = hk_pack2(v[2 * e], v[2 * e + 1]);
    *(typename hk_vec_of<DPL>::type *)p = raw;
}

/* IN_PLACE: the normalised, rotated Q and K go back over their own
 * elements of qkv (query must be qkv itself; key and value are unused), and
 * V stays where it is: attention then reads all three from the fused
 * buffer (h3_hip_sdpa_qkv_bf16).  Each thread reads its elements before any
 * thread of its row group writes.  K_ONLY (with IN_PLACE): K alone, for
 * attention that normalises and rotates Q itself as it loads it
 * (h3_hip_sdpa_qkv_norm_rope_bf16). */
template <int DPL, bool IN_PLACE = false, bool K_ONLY = false>
__global__ void __launch_bounds__(256)
hk_qk_norm_rope128v(const uint16_t *qkv,
                    const uint16_t *__restrict__ q_weight,
                    const uint16_t *__restrict__ k_weight,
                    const uint16_t *__restrict__ rope_cos,
                    const uint16_t *__restrict__ rope_sin,
                    uint16_t *query, uint16_t *key,
                    uint16_t *value, uint32_t sequence,
                    uint32_t heads, uint32_t rope_half, uint32_t grouped,
                    float epsilon) {
    constexpr uint32_t HD = 128, LANES = HD / DPL;
    typedef typename hk_vec_of<DPL>::type vec_t;
    const uint32_t vec = (blockIdx.x * blockDim.x + threadIdx.x) / LANES;
    const uint32_t part = threadIdx.x % LANES;
    const bool live = vec < sequence * heads;
    const uint32_t row = live ? vec / heads : 0, head = live ? vec % heads : 0;
    const size_t inner = (size_t)heads * HD;
    const size_t row_base = (size_t)row * inner * 3;
    size_t q_base, k_base, v_base;
    if (grouped) {
        q_base = row_base + (size_t)head * HD * 3;
        k_base = q_base + HD;
        v_base = k_base + HD;
    } else {
        q_base = row_base + (size_t)head * HD;
        k_base = q_base + inner;
        v_base = k_base + inner;
    }
    const uint32_t d0 = part * DPL;
    float q[DPL], k[DPL], qw[DPL], kw[DPL];
    if (K_ONLY) {
#pragma unroll
        for (int e = 0; e < DPL; e++) q[e] = 0.0f;
    } else {
        hk_unpack<DPL>(qkv + q_base + d0, q);
    }
    hk_unpack<DPL>(qkv + k_base + d0, k);
    vec_t vr;
    if (!IN_PLACE) vr = *(const vec_t *)(qkv + v_base + d0);
    hk_unpack<DPL>(q_weight + d0, qw);
    hk_unpack<DPL>(k_weight + d0, kw);
    float q_sum = 0.0f, k_sum = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        q_sum = fmaf(q[e], q[e], q_sum);
        k_sum = fmaf(k[e], k[e], k_sum);
    }
#pragma unroll
    for (int offset = LANES / 2; offset; offset >>= 1) {
        q_sum += __shfl_xor(q_sum, offset, LANES);
        k_sum += __shfl_xor(k_sum, offset, LANES);
    }
    const float q_inv = 1.0f / sqrtf(q_sum / (float)HD + epsilon);
    const float k_inv = 1.0f / sqrtf(k_sum / (float)HD + epsilon);
    float qn[DPL], kn[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        qn[e] = q[e] * q_inv * qw[e];
        kn[e] = k[e] * k_inv * kw[e];
    }
    const uint32_t shift = rope_half / DPL;
    int src = (int)part;
    if (d0 < rope_half) src = (int)(part + shift);
    else if (d0 < rope_half * 2) src = (int)(part - shift);
    float qp[DPL], kp[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        qp[e] = __shfl(qn[e], src, LANES);
        kp[e] = __shfl(kn[e], src, LANES);
    }
    if (!live) return;
    float qo[DPL], ko[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        qo[e] = qn[e];
        ko[e] = kn[e];
    }
    if (d0 < rope_half * 2) {
        const bool first = d0 < rope_half;
        const uint32_t pair = first ? d0 : d0 - rope_half;
        const size_t table = (size_t)row * rope_half + pair;
        float c[DPL], sn[DPL];
        hk_unpack<DPL>(rope_cos + table, c);
        hk_unpack<DPL>(rope_sin + table, sn);
#pragma unroll
        for (int e = 0; e < DPL; e++) {
            if (first) {
                qo[e] = qn[e] * c[e] - qp[e] * sn[e];
                ko[e] = kn[e] * c[e] - kp[e] * sn[e];
            } else {
                qo[e] = qn[e] * c[e] + qp[e] * sn[e];
                ko[e] = kn[e] * c[e] + kp[e] * sn[e];
            }
        }
    }
    const size_t out = ((size_t)row * heads + head) * HD + d0;
    if (IN_PLACE) {
        if (!K_ONLY) hk_pack_store<DPL>(query + q_base + d0, qo);
        hk_pack_store<DPL>(query + k_base + d0, ko);
        return;
    }
    hk_pack_store<DPL>(query + out, qo);
    hk_pack_store<DPL>(key + out, ko);
    *(vec_t *)(value + out) = vr;
}

/* K alone, in place over the fused QKV rows (the K_ONLY case of
 * hk_qk_norm_rope128v<8, true, true>, with the same arithmetic in the same
 * order): each 16-lane group handles ITEMS consecutive (row, head) vectors
 * and issues all of their loads before any arithmetic.  With one vector
 * per group a wave has 1 KiB of K in flight, too little to stream HBM at
 * full rate. */
template <int ITEMS>
__global__ void __launch_bounds__(256)
hk_k_norm_rope128_inplace(uint16_t *qkv, const uint16_t *__restrict__ k_weight,
                          const uint16_t *__restrict__ rope_cos,
                          const uint16_t *__restrict__ rope_sin,
                          uint32_t sequence, uint32_t heads,
                          uint32_t rope_half, float epsilon) {
    constexpr uint32_t HD = 128, DPL = 8, LANES = HD / DPL;
    const uint32_t group = (blockIdx.x * blockDim.x + threadIdx.x) / LANES;
    const uint32_t part = threadIdx.x % LANES;
    const uint32_t d0 = part * DPL;
    const uint32_t vectors = sequence * heads;
    const size_t inner = (size_t)heads * HD;
    uint4 kr[ITEMS], cr[ITEMS], sr[ITEMS];
    size_t k_base[ITEMS];
    uint32_t row[ITEMS];
    const bool roped = d0 < rope_half * 2;
    const bool first = d0 < rope_half;
    const uint32_t pair = first ? d0 : d0 - rope_half;
#pragma unroll
    for (int it = 0; it < ITEMS; it++) {
        const uint32_t vec = min(group * ITEMS + it, vectors - 1);
        row[it] = vec / heads;
        const uint32_t head = vec % heads;
        k_base[it] = (size_t)row[it] * inner * 3 + inner + (size_t)head * HD;
        kr[it] = *(const uint4 *)(qkv + k_base[it] + d0);
        if (roped) {
            const size_t table = (size_t)row[it] * rope_half + pair;
            cr[it] = *(const uint4 *)(rope_cos + table);
            sr[it] = *(const uint4 *)(rope_sin + table);
        }
    }
    float kw[DPL];
    hk_unpack8(*(const uint4 *)(k_weight + d0), kw);
    const uint32_t shift = rope_half / DPL;
    int src = (int)part;
    if (d0 < rope_half) src = (int)(part + shift);
    else if (d0 < rope_half * 2) src = (int)(part - shift);
#pragma unroll
    for (int it = 0; it < ITEMS; it++) {
        float k[DPL];
        hk_unpack8(kr[it], k);
        float k_sum = 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; e++) k_sum = fmaf(k[e], k[e], k_sum);
#pragma unroll
        for (int offset = LANES / 2; offset; offset >>= 1)
            k_sum += __shfl_xor(k_sum, offset, LANES);
        const float k_inv = 1.0f / sqrtf(k_sum / (float)HD + epsilon);
        float kn[DPL], kp[DPL], ko[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) kn[e] = k[e] * k_inv * kw[e];
#pragma unroll
        for (int e = 0; e < DPL; e++) kp[e] = __shfl(kn[e], src, LANES);
#pragma unroll
        for (int e = 0; e < DPL; e++) ko[e] = kn[e];
        if (roped) {
            float c[DPL], sn[DPL];
            hk_unpack8(cr[it], c);
            hk_unpack8(sr[it], sn);
#pragma unroll
            for (int e = 0; e < DPL; e++)
                ko[e] = first ? kn[e] * c[e] - kp[e] * sn[e]
                              : kn[e] * c[e] + kp[e] * sn[e];
        }
        if (group * ITEMS + it < vectors)
            *(uint4 *)(qkv + k_base[it] + d0) = hk_pack8(ko);
    }
}

/* Generic per-element variant for other head sizes (any rope_half with
 * 2*rope_half <= head_dim). */
template <typename T>
__device__ __forceinline__ float hk_ld(const T *p, size_t i) {
    if constexpr (sizeof(T) == 2) return hk_bf2f(p[i]);
    else return p[i];
}
template <typename T>
__device__ __forceinline__ void hk_st(T *p, size_t i, float v) {
    if constexpr (sizeof(T) == 2) p[i] = hk_f2bf(v);
    else p[i] = v;
}

template <typename T>
__global__ void hk_qk_norm_rope_any(const T *qkv, const T *q_weight,
                                    const T *k_weight, const T *rope_cos,
                                    const T *rope_sin, T *query, T *key,
                                    T *value, uint32_t sequence,
                                    uint32_t heads, uint32_t head_dim,
                                    uint32_t rope_half, uint32_t grouped,
                                    float epsilon, uint32_t use_norm) {
    size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (size_t)head_dim * heads * sequence) return;
    uint32_t d = (uint32_t)(gid % head_dim);
    uint32_t head = (uint32_t)((gid / head_dim) % heads);
    uint32_t row = (uint32_t)(gid / ((size_t)head_dim * heads));
    size_t inner = (size_t)heads * head_dim;
    size_t row_base = (size_t)row * inner * 3;
    size_t q_base = row_base + (size_t)head * head_dim;
    size_t k_base = q_base + inner, v_base = q_base + 2 * inner;
    if (grouped) {
        q_base = row_base + (size_t)head * head_dim * 3;
        k_base = q_base + head_dim;
        v_base = k_base + head_dim;
    }
    float q_inv = 1.0f, k_inv = 1.0f;
    if (use_norm) {
        float qs = 0.0f, ks = 0.0f;
        for (uint32_t i = 0; i < head_dim; i++) {
            float q = hk_ld(qkv, q_base + i), k = hk_ld(qkv, k_base + i);
            qs = fmaf(q, q, qs);
            ks = fmaf(k, k, ks);
        }
        q_inv = 1.0f / sqrtf(qs / (float)head_dim + epsilon);
        k_inv = 1.0f / sqrtf(ks / (float)head_dim + epsilon);
    }
    auto qn = [&](uint32_t i) {
        float x = hk_ld(qkv, q_base + i) * q_inv;
        return use_norm ? x * hk_ld(q_weight, i) : x;
    };
    auto kn = [&](uint32_t i) {
        float x = hk_ld(qkv, k_base + i) * k_inv;
        return use_norm ? x * hk_ld(k_weight, i) : x;
    };
    float q0 = qn(d), k0 = kn(d);
    if (d < rope_half) {
        float c = hk_ld(rope_cos, (size_t)row * rope_half + d);
        float s = hk_ld(rope_sin, (size_t)row * rope_half + d);
        float q1 = qn(d + rope_half), k1 = kn(d + rope_half);
        q0 = q0 * c - q1 * s;
        k0 = k0 * c - k1 * s;
    } else if (d < rope_half * 2) {
        uint32_t pair = d - rope_half;
        float c = hk_ld(rope_cos, (size_t)row * rope_half + pair);
        float s = hk_ld(rope_sin, (size_t)row * rope_half + pair);
        float q1 = qn(pair), k1 = kn(pair);
        q0 = q0 * c + q1 * s;
        k0 = k0 * c + k1 * s;
    }
    size_t out = ((size_t)row * heads + head) * head_dim + d;
    hk_st(query, out, q0);
    hk_st(key, out, k0);
    value[out] = qkv[v_base + d];
}

/* In-place per-head RMS norm, [sequence][heads][head_dim]
 * (reference h3_cuda_core.cu:322-341).  One wave64 per (row, head). */
__global__ void __launch_bounds__(256)
hk_head_rms_kernel(uint16_t *tensor, const uint16_t *weight,
                   uint32_t sequence, uint32_t heads, uint32_t head_dim,
                   float epsilon) {
    const uint32_t wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63;
    if (wave >= sequence * heads) return;
    uint16_t *x = tensor + (size_t)wave * head_dim;
    float sum = 0.0f;
    for (uint32_t d = lane; d < head_dim; d += 64) {
        float v = hk_bf2f(x[d]);
        sum = fmaf(v, v, sum);
    }
    const float inverse =
        1.0f / sqrtf(hk_wave_sum(sum) / (float)head_dim + epsilon);
    for (uint32_t d = lane; d < head_dim; d += 64)
        x[d] = hk_f2bf(hk_bf2f(x[d]) * inverse * hk_bf2f(weight[d]));
}

/* The same for head_dim 128: 16 lanes per (row, head), 8 dims (16 bytes)
 * per lane, four heads per wave.  hk_head_rms128_vec is one lane's part of
 * one vector, shared with the grouped form below so both round alike. */
__device__ __forceinline__ void hk_head_rms128_vec(uint16_t *vector,
                                                   const uint16_t *weight,
                                                   uint32_t part, bool live,
                                                   float epsilon) {
    uint4 *x = (uint4 *)vector + part;
    const uint4 raw = live ? *x : make_uint4(0, 0, 0, 0);
    const uint4 wraw = ((const uint4 *)weight)[part];
    const uint32_t xw[4] = {raw.x, raw.y, raw.z, raw.w};
    const uint32_t ww[4] = {wraw.x, wraw.y, wraw.z, wraw.w};
    float v[8], sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[2 * e] = hk_bf2f(xw[e] & 0xffffu);
        v[2 * e + 1] = hk_bf2f(xw[e] >> 16);
    }
#pragma unroll
    for (int e = 0; e < 8; e++) sum = fmaf(v[e], v[e], sum);
#pragma unroll
    for (int offset = 8; offset; offset >>= 1)
        sum += __shfl_xor(sum, offset, 16);
    const float inverse = 1.0f / sqrtf(sum / 128.0f + epsilon);
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
        ow[e] = hk_pack2(v[2 * e] * inverse * hk_bf2f(ww[e] & 0xffffu),
                         v[2 * e + 1] * inverse * hk_bf2f(ww[e] >> 16));
    if (live) *x = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

__global__ void __launch_bounds__(256)
hk_head_rms128(uint16_t *tensor, const uint16_t *weight, uint32_t vectors,
               float epsilon) {
    const uint32_t vec = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const bool live = vec < vectors;
    hk_head_rms128_vec(tensor + (size_t)(live ? vec : 0) * 128u, weight,
                       threadIdx.x & 15u, live, epsilon);
}

/* Many tensors of one shape, each with its own weight, in one launch:
 * vector v belongs to problem v / per_problem, whose tensor and weight
 * addresses are table[2 p] and table[2 p + 1]. */
__global__ void __launch_bounds__(256)
hk_head_rms128_group(const uint64_t *table, uint32_t per_problem,
                     uint32_t vectors, float epsilon) {
    const uint32_t vec = (blockIdx.x * blockDim.x + threadIdx.x) >> 4;
    const bool live = vec < vectors;
    const uint32_t v = live ? vec : 0;
    const uint32_t p = v / per_problem;
    uint16_t *tensor = (uint16_t *)(uintptr_t)table[2 * p];
    const uint16_t *weight = (const uint16_t *)(uintptr_t)table[2 * p + 1];
    hk_head_rms128_vec(tensor + (size_t)(v - p * per_problem) * 128u, weight,
                       threadIdx.x & 15u, live, epsilon);
}

/* ------------------------------------------------- small projections */

/* F32 patch projection, one thread per output, sequential-k fmaf from the
 * bias (the reference's exact hand-kernel order, h3_cuda_core.cu:374-403);
 * rounded to bf16 into output row map[r] (or r + 0 for the offset form). */
__global__ void hk_patch_linear_kernel(const float *input, const float *weight,
                                       const float *bias, uint16_t *output,
                                       const uint32_t *row_map, uint32_t rows,
                                       uint32_t input_dim,
                                       uint32_t output_dim) {
    uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t row = blockIdx.y; /* grid.y == rows */
    extern __shared__ float x_row[];
    for (uint32_t k = threadIdx.x; k < input_dim; k += blockDim.x)
        x_row[k] = input[(size_t)row * input_dim + k];
    __syncthreads();
    if (col >= output_dim) return;
    float sum = bias ? bias[col] : 0.0f;
    const float *w = weight + (size_t)col * input_dim;
    for (uint32_t k = 0; k < input_dim; k++) sum = fmaf(x_row[k], w[k], sum);
    size_t out_row = row_map ? row_map[row] : row;
    output[out_row * output_dim + col] = hk_f2bf(sum);
}

/* F32 linear, one thread per output, sequential k (timestep MLP and the
 * F32 final heads; small row counts). */
__global__ void hk_linear_f32_kernel(const float *input, const float *weight,
                                     const float *bias, float *output,
                                     uint32_t rows, uint32_t input_dim,
                                     uint32_t output_dim) {
    uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t row = blockIdx.y;
    if (row >= rows || col >= output_dim) return;
    float sum = bias ? bias[col] : 0.0f;
    const float *x = input + (size_t)row * input_dim;
    const float *w = weight + (size_t)col * input_dim;
    for (uint32_t k = 0; k < input_dim; k++) sum = fmaf(x[k], w[k], sum);
    output[(size_t)row * output_dim + col] = sum;
}

/* Final adaLN head: one workgroup per row.  The inverse RMS is reduced over
 * the row, the adaLN output is rounded to bf16 (the reference's boundary,
 * h3_cuda_dit.cu:183-234) and kept in LDS, then each wave computes dot
 * products against output columns of the [output_dim, width] weight. */
__global__ void __launch_bounds__(256)
hk_adaln_head_kernel(const uint16_t *input, float *inverse_out,
                     const uint16_t *norm_weight, const uint16_t *modulation,
                     const uint32_t *row_map, const uint16_t *weight,
                     const uint16_t *bias, uint16_t *output, uint32_t width,
                     uint32_t output_dim, uint32_t slots, uint32_t shift_slot,
                     uint32_t scale_slot, float epsilon) {
    extern __shared__ float normed[];
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x;
    const uint16_t *x = input + (size_t)row * width;
    float local = 0.0f;
    for (uint32_t k = threadIdx.x; k < width; k += blockDim.x) {
        float v = hk_bf2f(x[k]);
        local = fmaf(v, v, local);
    }
    float inverse = 1.0f / sqrtf(hk_block_sum(local, scratch) / (float)width +
                                 epsilon);
    if (threadIdx.x == 0) inverse_out[row] = inverse;
    size_t base = (size_t)row_map[row] * slots * width;
    for (uint32_t k = threadIdx.x; k < width; k += blockDim.x) {
        float shift = hk_bf2f(modulation[base + (size_t)shift_slot * width + k]);
        float scale = hk_bf2f(modulation[base + (size_t)scale_slot * width + k]);
        float n = hk_bf2f(x[k]) * inverse * hk_bf2f(norm_weight[k]);
        normed[k] = hk_bf2f(hk_f2bf(n * (1.0f + scale) + shift));
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t col = wave; col < output_dim; col += blockDim.x >> 6) {
        const uint16_t *w = weight + (size_t)col * width;
        float sum = 0.0f;
        for (uint32_t k = lane; k < width; k += 64)
            sum = fmaf(normed[k], hk_bf2f(w[k]), sum);
        sum = hk_wave_sum(sum);
        if (lane == 0) {
            if (bias) sum += hk_bf2f(bias[col]);
            output[(size_t)row * output_dim + col] = hk_f2bf(sum);
        }
    }
}

/* ------------------------------------------------------ seeded fill */

/* Counter-based N(mean, std^2): value i hashes (seed, i) through the
 * splitmix64 finaliser into two uniforms and takes one Box-Muller branch. */
__device__ __forceinline__ uint64_t hk_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float hk_normal_at(uint64_t seed, uint64_t i) {
    uint64_t bits = hk_mix64(seed * 0x9e3779b97f4a7c15ull + i * 2 + 1);
    uint32_t a = (uint32_t)(bits >> 32), b = (uint32_t)bits;
    float u1 = ((float)(a >> 8) + 1.0f) * (1.0f / 16777217.0f);
    float u2 = (float)(b >> 8) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

template <typename T>
__global__ void hk_fill_normal_kernel(T *out, size_t count, uint64_t seed,
                                      float mean, float stddev) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        float v = mean + stddev * hk_normal_at(seed, i);
        if constexpr (sizeof(T) == 2) out[i] = hk_f2bf(v);
        else out[i] = v;
    }
}

/* =============================================================== host */

/* ---------------------------------------------------------------------
 * Token reduction (reference h3_cuda_dit.cu:336-535): pool pairs of rows of
 * the full token grid into one reduced row, snapshot the pre-pool rows
 * ("original") and the pooled rows the reduced stack starts from
 * ("baseline"); later expand back, each full row taking its parent's update
 * relative to that baseline.  The _adaln variants fuse the next attention
 * RMS adaLN.  One workgroup per output row; rows are moved in 16-byte
 * chunks when the width allows.  Every row addressed through a device-side
 * index (pairs, parents, baseline rows) goes through a buffer resource
 * bounded by its tensor, so a bad index reads zeros and drops its writes
 * instead of faulting.
 * ------------------------------------------------------------------- */
struct hk_token_args {
    const uint16_t *input;     /* pool: full grid; expand: reduced stack */
    uint16_t *original;        /* full-grid snapshot */
    uint16_t *baseline;        /* pooled snapshot rows */
    const uint32_t *baseline_indices;
    const uint32_t *index;     /* pool: pairs (2 per row); expand: parents */
    uint16_t *residual;        /* pool: reduced rows; expand: full rows */
    uint16_t *adaln;           /* fused adaLN output or null */
    const uint16_t *norm_weight, *modulation;
    const uint32_t *row_map;
    uint32_t input_bytes, original_bytes, baseline_bytes, index_bytes,
        baseline_index_bytes;
    uint32_t input_offset, original_offset, baseline_offset; /* elements */
    uint32_t rows, width, exact_prefix_rows;
    uint32_t slots, shift_slot, scale_slot;
    float update_scale, epsilon;
};

typedef int hk_v4i __attribute__((ext_vector_type(4)));

#define HK_TOKEN_CHUNKS 3 /* 16-byte chunks per thread: width <= 6144 */

__device__ __forceinline__ __amdgpu_buffer_rsrc_t hk_tok_rsrc(const void *p,
                                                              uint32_t n) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)n, 0x00020000);
}

/* EXPAND = false: pool; true: expand.  ADALN: fuse the RMS adaLN. */
template <bool EXPAND, bool ADALN>
__global__ void __launch_bounds__(256)
hk_token_kernel(hk_token_args a) {
    __shared__ float scratch[16];
    const uint32_t row = blockIdx.x;
    const uint32_t width = a.width, chunks = width >> 3;
    const auto in_r = hk_tok_rsrc(a.input, a.input_bytes);
    const auto org_r = hk_tok_rsrc(a.original, a.original_bytes);
    const auto base_r = hk_tok_rsrc(a.baseline, a.baseline_bytes);
    const auto idx_r = hk_tok_rsrc(a.index, a.index_bytes);
    const auto bidx_r = hk_tok_rsrc(a.baseline_indices, a.baseline_index_bytes);
    uint32_t first, second, baseline_row;
    bool direct = false;
    if (!EXPAND) {
        first = __builtin_amdgcn_raw_buffer_load_b32(idx_r, row * 8u, 0, 0);
        second = __builtin_amdgcn_raw_buffer_load_b32(idx_r, row * 8u + 4u,
                                                      0, 0);
        baseline_row = __builtin_amdgcn_raw_buffer_load_b32(bidx_r, row * 4u,
                                                            0, 0);
    } else {
        first = __builtin_amdgcn_raw_buffer_load_b32(idx_r, row * 4u, 0, 0);
        second = first;
        baseline_row = __builtin_amdgcn_raw_buffer_load_b32(bidx_r, first * 4u,
                                                            0, 0);
        direct = row < a.exact_prefix_rows || baseline_row == 0xffffffffu;
    }
    /* byte offsets of the rows this workgroup touches */
    const uint32_t in1 = (a.input_offset + first * width) * 2u;
    const uint32_t in2 = (a.input_offset + second * width) * 2u;
    const uint32_t org1 = (a.original_offset +
                           (EXPAND ? row : first) * width) * 2u;
    const uint32_t org2 = (a.original_offset + second * width) * 2u;
    const uint32_t bas = baseline_row == 0xffffffffu
        ? 0xfffffff0u
        : (a.baseline_offset + baseline_row * width) * 2u;
    uint16_t *dst = a.residual + (size_t)row * width;

    float local = 0.0f;
    hk_v4i kept[HK_TOKEN_CHUNKS];
#pragma unroll
    for (int j = 0; j < HK_TOKEN_CHUNKS; j++) {
        const uint32_t c = threadIdx.x + j * 256u;
        if (c >= chunks) break;
        const uint32_t cb = c * 16u;
        hk_v4i value;
        if (!EXPAND) {
            hk_v4i x = __builtin_amdgcn_raw_buffer_load_b128(in_r, in1 + cb,
                                                              0, 0);
            __builtin_amdgcn_raw_buffer_store_b128(x, org_r, org1 + cb, 0, 0);
            value = x;
            if (first != second) {
                hk_v4i y = __builtin_amdgcn_raw_buffer_load_b128(
                    in_r, in2 + cb, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(y, org_r, org2 + cb, 0,
                                                       0);
                const uint16_t *xs = (const uint16_t *)&x;
                const uint16_t *ys = (const uint16_t *)&y;
                uint16_t *vs = (uint16_t *)&value;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    vs[e] = hk_f2bf((hk_bf2f(xs[e]) + hk_bf2f(ys[e])) * 0.5f);
            }
            if (baseline_row != 0xffffffffu)
                __builtin_amdgcn_raw_buffer_store_b128(value, base_r,
                                                       bas + cb, 0, 0);
        } else {
            value = __builtin_amdgcn_raw_buffer_load_b128(in_r, in1 + cb, 0,
                                                          0);
            if (!direct) {
                hk_v4i o = __builtin_amdgcn_raw_buffer_load_b128(
                    org_r, org1 + cb, 0, 0);
                hk_v4i b = __builtin_amdgcn_raw_buffer_load_b128(
                    base_r, bas + cb, 0, 0);
                const uint16_t *os = (const uint16_t *)&o;
                const uint16_t *bs = (const uint16_t *)&b;
                uint16_t *vs = (uint16_t *)&value;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float update = hk_bf2f(vs[e]) - hk_bf2f(bs[e]);
                    vs[e] = hk_f2bf(hk_bf2f(os[e]) + a.update_scale * update);
                }
            }
        }
        *(hk_v4i *)(dst + c * 8u) = value;
        if (ADALN) {
            kept[j] = value;
            const uint16_t *vs = (const uint16_t *)&value;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float f = hk_bf2f(vs[e]);
                local = fmaf(f, f, local);
            }
        }
    }
    if (!ADALN) return;
    const float total = hk_block_sum(local, scratch);
    const float inverse = 1.0f / sqrtf(total / (float)width + a.epsilon);
    const size_t base = (size_t)a.row_map[row] * a.slots * width;
    const uint16_t *shift = a.modulation + base + (size_t)a.shift_slot * width;
    const uint16_t *scale = a.modulation + base + (size_t)a.scale_slot * width;
    uint16_t *out = a.adaln + (size_t)row * width;
#pragma unroll
    for (int j = 0; j < HK_TOKEN_CHUNKS; j++) {
        const uint32_t c = threadIdx.x + j * 256u;
        if (c >= chunks) break;
        const uint16_t *vs = (const uint16_t *)&kept[j];
        const hk_v4i w = *(const hk_v4i *)(a.norm_weight + c * 8u);
        const hk_v4i sh = *(const hk_v4i *)(shift + c * 8u);
        const hk_v4i sc = *(const hk_v4i *)(scale + c * 8u);
        const uint16_t *ws = (const uint16_t *)&w;
        const uint16_t *shs = (const uint16_t *)&sh;
        const uint16_t *scs = (const uint16_t *)&sc;
        hk_v4i result;
        uint16_t *rs = (uint16_t *)&result;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float normalized = hk_bf2f(vs[e]) * inverse * hk_bf2f(ws[e]);
            rs[e] = hk_f2bf(normalized * (1.0f + hk_bf2f(scs[e])) +
                            hk_bf2f(shs[e]));
        }
        *(hk_v4i *)(out + c * 8u) = result;
    }
}

#define HK_REQ_BF16(t, n, label) hk_require(gpu, t, n, H3_GPU_BF16, label)
#define HK_REQ_F32(t, n, label) hk_require(gpu, t, n, H3_GPU_F32, label)
#define HK_REQ_U32(t, n, label) hk_require(gpu, t, n, H3_GPU_U32, label)

extern "C" {

int h3_gpu_adaln_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output,
                             const h3_gpu_tensor *input, size_t input_offset,
                             const h3_gpu_tensor *norm_weight,
                             const h3_gpu_tensor *modulation,
                             const h3_gpu_tensor *row_map, uint32_t rows,
                             uint32_t width, uint32_t slots,
                             uint32_t shift_slot, uint32_t scale_slot,
                             float epsilon) {
    size_t count = (size_t)rows * width;
    if (input_offset > SIZE_MAX - count)
        return hk_fail(gpu, "AdaLN input offset is out of range");
    if (!HK_REQ_BF16(input, input_offset + count, "AdaLN input") ||
        !HK_REQ_BF16(norm_weight, width, "AdaLN norm") ||
        !HK_REQ_BF16(modulation, 1, "AdaLN modulation") ||
        !HK_REQ_U32(row_map, rows, "AdaLN row map") ||
        !HK_REQ_BF16(output, count, "AdaLN output") ||
        !hk_require_active(gpu))
        return 0;
    if (shift_slot >= slots || scale_slot >= slots)
        return hk_fail(gpu, "AdaLN modulation slot is out of range");
    hk_op_begin(gpu, "adaln");
    hk_row_args a = {};
    a.input = HK_CBF16(input) + input_offset;
    a.weight = HK_CBF16(norm_weight);
    a.norm_mod = HK_CBF16(modulation);
    a.row_map = HK_CU32(row_map);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.slots = slots;
    a.shift_slot = shift_slot; a.scale_slot = scale_slot;
    a.epsilon = epsilon;
    hk_row_launch<HK_ROW_NORM | HK_ROW_WEIGHT | HK_ROW_MOD>(gpu, a);
    return hk_op_end(gpu, "adaln", HK_KIND_DIRECT);
}

int h3_gpu_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                      const h3_gpu_tensor *input,
                      const h3_gpu_tensor *norm_weight,
                      const h3_gpu_tensor *modulation,
                      const h3_gpu_tensor *row_map, uint32_t rows,
                      uint32_t width, uint32_t slots, uint32_t shift_slot,
                      uint32_t scale_slot, float epsilon) {
    return h3_gpu_adaln_bf16_offset(gpu, output, input, 0, norm_weight,
                                    modulation, row_map, rows, width, slots,
                                    shift_slot, scale_slot, epsilon);
}

int h3_gpu_gate_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *residual,
                     const h3_gpu_tensor *branch,
                     const h3_gpu_tensor *modulation,
                     const h3_gpu_tensor *row_map, uint32_t rows,
                     uint32_t width, uint32_t slots, uint32_t gate_slot) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_BF16(residual, count, "gate residual") ||
        !HK_REQ_BF16(branch, count, "gate branch") ||
        !HK_REQ_BF16(modulation, 1, "gate modulation") ||
        !HK_REQ_U32(row_map, rows, "gate row map") ||
        !HK_REQ_BF16(output, count, "gate output") ||
        !hk_require_active(gpu))
        return 0;
    if (gate_slot >= slots)
        return hk_fail(gpu, "gate modulation slot is out of range");
    hk_op_begin(gpu, "gate");
    hk_row_args a = {};
    a.input = HK_CBF16(residual);
    a.branch = HK_CBF16(branch);
    a.gate_mod = HK_CBF16(modulation);
    a.row_map = HK_CU32(row_map);
    a.gated = HK_BF16(output);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.slots = slots; a.gate_slot = gate_slot;
    hk_row_launch<HK_ROW_GATE>(gpu, a);
    return hk_op_end(gpu, "gate", HK_KIND_DIRECT);
}

int h3_gpu_gate_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *gated_residual,
                           h3_gpu_tensor *output,
                           const h3_gpu_tensor *residual,
                           const h3_gpu_tensor *branch,
                           const h3_gpu_tensor *norm_weight,
                           const h3_gpu_tensor *gate_modulation,
                           const h3_gpu_tensor *norm_modulation,
                           const h3_gpu_tensor *row_map, uint32_t rows,
                           uint32_t width, uint32_t slots, uint32_t gate_slot,
                           uint32_t shift_slot, uint32_t scale_slot,
                           float epsilon) {
    size_t count = (size_t)rows * width;
    /* the reference keeps the gated row in shared memory and caps the width
     * at 5376 (h3_cuda_dit.cu:769-770); the same limit is kept so callers
     * see identical validation */
    if (!rows || !width || width > 5376 || count > UINT32_MAX)
        return hk_fail(gpu, "fused gate AdaLN shape is out of range");
    if (gate_slot >= slots || shift_slot >= slots || scale_slot >= slots)
        return hk_fail(gpu, "fused gate AdaLN modulation slot out of range");
    if (!HK_REQ_BF16(residual, count, "fused gate AdaLN residual") ||
        !HK_REQ_BF16(branch, count, "fused gate AdaLN branch") ||
        !HK_REQ_BF16(norm_weight, width, "fused gate AdaLN norm") ||
        !HK_REQ_BF16(gate_modulation, 1, "fused gate AdaLN gate modulation") ||
        !HK_REQ_BF16(norm_modulation, 1, "fused gate AdaLN norm modulation") ||
        !HK_REQ_U32(row_map, rows, "fused gate AdaLN row map") ||
        !HK_REQ_BF16(gated_residual, count, "fused gate AdaLN gated residual") ||
        !HK_REQ_BF16(output, count, "fused gate AdaLN output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "gate_adaln");
    hk_row_args a = {};
    a.input = HK_CBF16(residual);
    a.branch = HK_CBF16(branch);
    a.weight = HK_CBF16(norm_weight);
    a.gate_mod = HK_CBF16(gate_modulation);
    a.norm_mod = HK_CBF16(norm_modulation);
    a.row_map = HK_CU32(row_map);
    a.gated = HK_BF16(gated_residual);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.slots = slots;
    a.gate_slot = gate_slot; a.shift_slot = shift_slot;
    a.scale_slot = scale_slot; a.epsilon = epsilon;
    hk_row_launch<HK_ROW_GATE | HK_ROW_NORM | HK_ROW_WEIGHT | HK_ROW_MOD>(gpu,
                                                                         a);
    return hk_op_end(gpu, "gate_adaln", HK_KIND_DIRECT);
}

int h3_gpu_layer_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *norm_weight,
                            const h3_gpu_tensor *norm_bias,
                            const h3_gpu_tensor *modulation,
                            const h3_gpu_tensor *row_map, uint32_t rows,
                            uint32_t width, uint32_t slots,
                            uint32_t shift_slot, uint32_t scale_slot,
                            float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_BF16(input, count, "LayerNorm AdaLN input") ||
        (norm_weight && !HK_REQ_BF16(norm_weight, width, "LayerNorm weight")) ||
        (norm_bias && !HK_REQ_BF16(norm_bias, width, "LayerNorm bias")) ||
        (modulation && !HK_REQ_BF16(modulation, 1, "LayerNorm modulation")) ||
        (modulation && !HK_REQ_U32(row_map, rows, "LayerNorm row map")) ||
        !HK_REQ_BF16(output, count, "LayerNorm AdaLN output") ||
        !hk_require_active(gpu))
        return 0;
    if (modulation && (shift_slot >= slots || scale_slot >= slots))
        return hk_fail(gpu, "LayerNorm AdaLN modulation slot out of range");
    hk_op_begin(gpu, "layer_adaln");
    hk_row_args a = {};
    a.input = HK_CBF16(input);
    a.weight = norm_weight ? HK_CBF16(norm_weight) : NULL;
    a.bias = norm_bias ? HK_CBF16(norm_bias) : NULL;
    a.norm_mod = modulation ? HK_CBF16(modulation) : NULL;
    a.row_map = modulation ? HK_CU32(row_map) : NULL;
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.slots = slots;
    a.shift_slot = shift_slot; a.scale_slot = scale_slot; a.epsilon = epsilon;
    const int base = HK_ROW_NORM | HK_ROW_LAYER;
    int key = (norm_weight ? 1 : 0) | (norm_bias ? 2 : 0) | (modulation ? 4 : 0);
    switch (key) {
    case 0: hk_row_launch<base>(gpu, a); break;
    case 1: hk_row_launch<base | HK_ROW_WEIGHT>(gpu, a); break;
    case 2: hk_row_launch<base | HK_ROW_BIAS>(gpu, a); break;
    case 3: hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_BIAS>(gpu, a); break;
    case 4: hk_row_launch<base | HK_ROW_MOD>(gpu, a); break;
    case 5: hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_MOD>(gpu, a); break;
    case 6: hk_row_launch<base | HK_ROW_BIAS | HK_ROW_MOD>(gpu, a); break;
    default:
        hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_BIAS | HK_ROW_MOD>(gpu, a);
    }
    return hk_op_end(gpu, "layer_adaln", HK_KIND_DIRECT);
}

int h3_gpu_gate_layer_adaln_bf16(
    h3_gpu *gpu, h3_gpu_tensor *gated_residual, h3_gpu_tensor *output,
    const h3_gpu_tensor *residual, const h3_gpu_tensor *branch,
    const h3_gpu_tensor *gate_modulation, const h3_gpu_tensor *norm_weight,
    const h3_gpu_tensor *norm_bias, const h3_gpu_tensor *norm_modulation,
    const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width,
    uint32_t slots, uint32_t gate_slot, uint32_t shift_slot,
    uint32_t scale_slot, float epsilon) {
    size_t count = (size_t)rows * width;
    const bool need_map = gate_modulation || norm_modulation;
    if ((gate_modulation && gate_slot >= slots) ||
        (norm_modulation && (shift_slot >= slots || scale_slot >= slots)))
        return hk_fail(gpu, "gate LayerNorm AdaLN modulation slot out of range");
    if (!HK_REQ_BF16(residual, count, "gate LayerNorm AdaLN residual") ||
        !HK_REQ_BF16(branch, count, "gate LayerNorm AdaLN branch") ||
        (gate_modulation &&
         !HK_REQ_BF16(gate_modulation, 1,
                      "gate LayerNorm AdaLN gate modulation")) ||
        (norm_weight && !HK_REQ_BF16(norm_weight, width, "LayerNorm weight")) ||
        (norm_bias && !HK_REQ_BF16(norm_bias, width, "LayerNorm bias")) ||
        (norm_modulation &&
         !HK_REQ_BF16(norm_modulation, 1, "LayerNorm modulation")) ||
        (need_map && !HK_REQ_U32(row_map, rows, "gate LayerNorm AdaLN row map")) ||
        !HK_REQ_BF16(gated_residual, count,
                     "gate LayerNorm AdaLN gated residual") ||
        !HK_REQ_BF16(output, count, "gate LayerNorm AdaLN output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "gate_layer_adaln");
    hk_row_args a = {};
    a.input = HK_CBF16(residual);
    a.branch = HK_CBF16(branch);
    a.gate_mod = gate_modulation ? HK_CBF16(gate_modulation) : NULL;
    a.weight = norm_weight ? HK_CBF16(norm_weight) : NULL;
    a.bias = norm_bias ? HK_CBF16(norm_bias) : NULL;
    a.norm_mod = norm_modulation ? HK_CBF16(norm_modulation) : NULL;
    a.row_map = need_map ? HK_CU32(row_map) : NULL;
    a.gated = HK_BF16(gated_residual);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.slots = slots;
    a.gate_slot = gate_slot; a.shift_slot = shift_slot;
    a.scale_slot = scale_slot; a.epsilon = epsilon;
    const int base = HK_ROW_GATE | HK_ROW_NORM | HK_ROW_LAYER;
    int key = (norm_weight ? 1 : 0) | (norm_bias ? 2 : 0) |
              (norm_modulation ? 4 : 0);
    switch (key) {
    case 0: hk_row_launch<base>(gpu, a); break;
    case 1: hk_row_launch<base | HK_ROW_WEIGHT>(gpu, a); break;
    case 2: hk_row_launch<base | HK_ROW_BIAS>(gpu, a); break;
    case 3: hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_BIAS>(gpu, a); break;
    case 4: hk_row_launch<base | HK_ROW_MOD>(gpu, a); break;
    case 5: hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_MOD>(gpu, a); break;
    case 6: hk_row_launch<base | HK_ROW_BIAS | HK_ROW_MOD>(gpu, a); break;
    default:
        hk_row_launch<base | HK_ROW_WEIGHT | HK_ROW_BIAS | HK_ROW_MOD>(gpu, a);
    }
    return hk_op_end(gpu, "gate_layer_adaln", HK_KIND_DIRECT);
}

int h3_gpu_rms_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         const h3_gpu_tensor *input,
                         const h3_gpu_tensor *weight, uint32_t rows,
                         uint32_t width, float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_BF16(input, count, "RMS norm input") ||
        !HK_REQ_BF16(weight, width, "RMS norm weight") ||
        !HK_REQ_BF16(output, count, "RMS norm output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "rms_norm");
    hk_row_args a = {};
    a.input = HK_CBF16(input);
    a.weight = HK_CBF16(weight);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.epsilon = epsilon;
    hk_row_launch<HK_ROW_NORM | HK_ROW_WEIGHT>(gpu, a);
    return hk_op_end(gpu, "rms_norm", HK_KIND_DIRECT);
}

int h3_gpu_layer_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *input,
                           const h3_gpu_tensor *weight,
                           const h3_gpu_tensor *bias, uint32_t rows,
                           uint32_t width, float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_BF16(input, count, "LayerNorm input") ||
        !HK_REQ_BF16(weight, width, "LayerNorm weight") ||
        !HK_REQ_BF16(bias, width, "LayerNorm bias") ||
        !HK_REQ_BF16(output, count, "LayerNorm output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "layer_norm");
    hk_row_args a = {};
    a.input = HK_CBF16(input);
    a.weight = HK_CBF16(weight);
    a.bias = HK_CBF16(bias);
    a.output = HK_BF16(output);
    a.rows = rows; a.width = width; a.epsilon = epsilon;
    hk_row_launch<HK_ROW_NORM | HK_ROW_LAYER | HK_ROW_WEIGHT | HK_ROW_BIAS>(gpu,
                                                                          a);
    return hk_op_end(gpu, "layer_norm", HK_KIND_DIRECT);
}

static int hk_row32(h3_gpu *gpu, const char *name, hk_row32_args a) {
    hk_op_begin(gpu, name);
    if (a.rows && a.width)
        hipLaunchKernelGGL(hk_row_f32, dim3(a.rows), dim3(HK_ROW_THREADS), 0,
                           gpu->stream, a);
    return hk_op_end(gpu, name, HK_KIND_DIRECT);
}

int h3_gpu_rms_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                        const h3_gpu_tensor *input,
                        const h3_gpu_tensor *weight, uint32_t rows,
                        uint32_t width, float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(input, count, "RMS norm input") ||
        !HK_REQ_F32(weight, width, "RMS norm weight") ||
        !HK_REQ_F32(output, count, "RMS norm output") ||
        !hk_require_active(gpu))
        return 0;
    hk_row32_args a = {};
    a.input = HK_CF32(input); a.weight = HK_CF32(weight);
    a.output = HK_F32(output); a.rows = rows; a.width = width;
    a.epsilon = epsilon; a.mode = 0;
    return hk_row32(gpu, "rms_norm_f32", a);
}

int h3_gpu_layer_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *input,
                          const h3_gpu_tensor *weight,
                          const h3_gpu_tensor *bias, uint32_t rows,
                          uint32_t width, float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(input, count, "LayerNorm input") ||
        !HK_REQ_F32(weight, width, "LayerNorm weight") ||
        !HK_REQ_F32(bias, width, "LayerNorm bias") ||
        !HK_REQ_F32(output, count, "LayerNorm output") ||
        !hk_require_active(gpu))
        return 0;
    hk_row32_args a = {};
    a.input = HK_CF32(input); a.weight = HK_CF32(weight);
    a.bias = HK_CF32(bias); a.output = HK_F32(output); a.rows = rows;
    a.width = width; a.epsilon = epsilon; a.mode = 2;
    return hk_row32(gpu, "layer_norm_f32", a);
}

int h3_gpu_adaln_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input,
                     const h3_gpu_tensor *norm_weight,
                     const h3_gpu_tensor *modulation,
                     const h3_gpu_tensor *row_map, uint32_t rows,
                     uint32_t width, uint32_t slots, uint32_t shift_slot,
                     uint32_t scale_slot, float epsilon) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(input, count, "AdaLN input") ||
        !HK_REQ_F32(norm_weight, width, "AdaLN norm") ||
        !HK_REQ_F32(modulation, 1, "AdaLN modulation") ||
        !HK_REQ_U32(row_map, rows, "AdaLN row map") ||
        !HK_REQ_F32(output, count, "AdaLN output") ||
        !hk_require_active(gpu))
        return 0;
    if (shift_slot >= slots || scale_slot >= slots)
        return hk_fail(gpu, "AdaLN modulation slot is out of range");
    hk_row32_args a = {};
    a.input = HK_CF32(input); a.weight = HK_CF32(norm_weight);
    a.modulation = HK_CF32(modulation); a.row_map = HK_CU32(row_map);
    a.output = HK_F32(output); a.rows = rows; a.width = width;
    a.slots = slots; a.shift_slot = shift_slot; a.scale_slot = scale_slot;
    a.epsilon = epsilon; a.mode = 1;
    return hk_row32(gpu, "adaln_f32", a);
}

int h3_gpu_gate_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *residual,
                    const h3_gpu_tensor *branch,
                    const h3_gpu_tensor *modulation,
                    const h3_gpu_tensor *row_map, uint32_t rows,
                    uint32_t width, uint32_t slots, uint32_t gate_slot) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(residual, count, "gate residual") ||
        !HK_REQ_F32(branch, count, "gate branch") ||
        !HK_REQ_F32(modulation, 1, "gate modulation") ||
        !HK_REQ_U32(row_map, rows, "gate row map") ||
        !HK_REQ_F32(output, count, "gate output") ||
        !hk_require_active(gpu))
        return 0;
    if (gate_slot >= slots)
        return hk_fail(gpu, "gate modulation slot is out of range");
    hk_op_begin(gpu, "gate_f32");
    if (count)
        hipLaunchKernelGGL(hk_gate_f32_kernel, dim3((unsigned)((count + 255) / 256)),
                           dim3(256), 0, gpu->stream, HK_CF32(residual),
                           HK_CF32(branch), HK_CF32(modulation),
                           HK_CU32(row_map), HK_F32(output), rows, width,
                           slots, gate_slot);
    return hk_op_end(gpu, "gate_f32", HK_KIND_DIRECT);
}

/* ---- elementwise ---- */

int h3_gpu_silu_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *input, uint32_t elements) {
    if (!HK_REQ_F32(input, elements, "SiLU input") ||
        !HK_REQ_F32(output, elements, "SiLU output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "silu_f32");
    hk_ew_launch<HK_EW_SILU_F32>(gpu, input->data, NULL, output->data, elements);
    return hk_op_end(gpu, "silu_f32", HK_KIND_DIRECT);
}

int h3_gpu_silu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input, uint32_t elements) {
    if (!HK_REQ_BF16(input, elements, "SiLU input") ||
        !HK_REQ_BF16(output, elements, "SiLU output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "silu_bf16");
    hk_ew_launch<HK_EW_SILU_BF16>(gpu, input->data, NULL, output->data,
                                  elements);
    return hk_op_end(gpu, "silu_bf16", HK_KIND_DIRECT);
}

int h3_gpu_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *input, uint32_t elements,
                     int approximate) {
    if (!HK_REQ_BF16(input, elements, "GELU input") ||
        !HK_REQ_BF16(output, elements, "GELU output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "gelu");
    if (approximate)
        hk_ew_launch<HK_EW_GELU_TANH>(gpu, input->data, NULL, output->data,
                                      elements);
    else
        hk_ew_launch<HK_EW_GELU_ERF>(gpu, input->data, NULL, output->data,
                                     elements);
    return hk_op_end(gpu, "gelu", HK_KIND_DIRECT);
}

int h3_gpu_cast_f32_to_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input, uint32_t elements) {
    if (!HK_REQ_F32(input, elements, "cast input") ||
        !HK_REQ_BF16(output, elements, "cast output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "cast_f32_bf16");
    hk_ew_launch<HK_EW_CAST_F2B>(gpu, input->data, NULL, output->data, elements);
    return hk_op_end(gpu, "cast_f32_bf16", HK_KIND_DIRECT);
}

int h3_gpu_cast_bf16_to_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input, uint32_t elements) {
    if (!HK_REQ_BF16(input, elements, "cast input") ||
        !HK_REQ_F32(output, elements, "cast output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "cast_bf16_f32");
    hk_ew_launch<HK_EW_CAST_B2F>(gpu, input->data, NULL, output->data, elements);
    return hk_op_end(gpu, "cast_bf16_f32", HK_KIND_DIRECT);
}

static int hk_binary_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *left,
                          const h3_gpu_tensor *right, uint32_t elements,
                          const char *name, int op) {
    if (!HK_REQ_BF16(left, elements, name) ||
        !HK_REQ_BF16(right, elements, name) ||
        !HK_REQ_BF16(output, elements, name) || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, name);
    if (op == HK_EW_ADD_BF16)
        hk_ew_launch<HK_EW_ADD_BF16>(gpu, left->data, right->data,
                                     output->data, elements);
    else if (op == HK_EW_SUB_BF16)
        hk_ew_launch<HK_EW_SUB_BF16>(gpu, left->data, right->data,
                                     output->data, elements);
    else
        hk_ew_launch<HK_EW_SILU_MUL_BF16>(gpu, left->data, right->data,
                                          output->data, elements);
    return hk_op_end(gpu, name, HK_KIND_DIRECT);
}

int h3_gpu_add_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *left, const h3_gpu_tensor *right,
                    uint32_t elements) {
    return hk_binary_bf16(gpu, output, left, right, elements, "add",
                          HK_EW_ADD_BF16);
}

int h3_gpu_sub_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *left, const h3_gpu_tensor *right,
                    uint32_t elements) {
    return hk_binary_bf16(gpu, output, left, right, elements, "sub",
                          HK_EW_SUB_BF16);
}

int h3_gpu_silu_mul_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         const h3_gpu_tensor *gate, const h3_gpu_tensor *up,
                         uint32_t elements) {
    return hk_binary_bf16(gpu, output, gate, up, elements, "silu_mul",
                          HK_EW_SILU_MUL_BF16);
}

int h3_gpu_swiglu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                       const h3_gpu_tensor *fused, uint32_t rows,
                       uint32_t width) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_BF16(fused, count * 2, "SwiGLU input") ||
        !HK_REQ_BF16(output, count, "SwiGLU output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "swiglu");
    if (count)
        hipLaunchKernelGGL(hk_swiglu_kernel<uint16_t>,
                           dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                           gpu->stream, HK_CBF16(fused), HK_BF16(output), rows,
                           width);
    return hk_op_end(gpu, "swiglu", HK_KIND_DIRECT);
}

int h3_gpu_swiglu_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                      const h3_gpu_tensor *fused, uint32_t rows,
                      uint32_t width) {
    size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(fused, count * 2, "SwiGLU input") ||
        !HK_REQ_F32(output, count, "SwiGLU output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "swiglu_f32");
    if (count)
        hipLaunchKernelGGL(hk_swiglu_kernel<float>,
                           dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                           gpu->stream, HK_CF32(fused), HK_F32(output), rows,
                           width);
    return hk_op_end(gpu, "swiglu_f32", HK_KIND_DIRECT);
}

int h3_gpu_euler_bf16(h3_gpu *gpu, h3_gpu_tensor *sample,
                      size_t sample_offset, const h3_gpu_tensor *last,
                      const h3_gpu_tensor *previous, uint32_t elements,
                      float delta, float ratio) {
    if (sample_offset > SIZE_MAX - elements)
        return hk_fail(gpu, "Euler sample offset is out of range");
    if (!HK_REQ_F32(sample, sample_offset + elements, "Euler sample") ||
        !HK_REQ_BF16(last, elements, "Euler velocity") ||
        !HK_REQ_BF16(previous, elements, "Euler previous velocity") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "euler");
    if (elements)
        hipLaunchKernelGGL(hk_euler_kernel, dim3((elements + 255) / 256),
                           dim3(256), 0, gpu->stream,
                           HK_F32(sample) + sample_offset, HK_CBF16(last),
                           HK_CBF16(previous), elements, delta, ratio);
    return hk_op_end(gpu, "euler", HK_KIND_DIRECT);
}

static int hk_copy(h3_gpu *gpu, h3_gpu_tensor *destination, size_t d_off,
                   const h3_gpu_tensor *source, size_t s_off, size_t n,
                   h3_gpu_dtype dtype, const char *name) {
    if (d_off > SIZE_MAX - n || s_off > SIZE_MAX - n)
        return hk_fail(gpu, "%s offset is out of range", name);
    if (!hk_require(gpu, destination, d_off + n, dtype, name) ||
        !hk_require(gpu, source, s_off + n, dtype, name) ||
        !hk_require_active(gpu))
        return 0;
    size_t item = hk_item_size(dtype);
    if (!n) return 1;
    hipError_t status = hipMemcpyAsync(
        (char *)destination->data + d_off * item,
        (const char *)source->data + s_off * item, n * item,
        hipMemcpyDeviceToDevice, gpu->stream);
    if (status != hipSuccess) return hk_fail_hip(gpu, name, status);
    gpu->stats.blit_copies++;
    return 1;
}

int h3_gpu_copy_bf16(h3_gpu *gpu, h3_gpu_tensor *destination,
                     size_t destination_offset, const h3_gpu_tensor *source,
                     size_t source_offset, size_t elements) {
    return hk_copy(gpu, destination, destination_offset, source,
                   source_offset, elements, H3_GPU_BF16, "bf16 copy");
}

int h3_gpu_copy_f32(h3_gpu *gpu, h3_gpu_tensor *destination,
                    size_t destination_offset, const h3_gpu_tensor *source,
                    size_t source_offset, size_t elements) {
    return hk_copy(gpu, destination, destination_offset, source,
                   source_offset, elements, H3_GPU_F32, "f32 copy");
}

/* ---- Q/K norm + RoPE ---- */

static int hk_qkv_rope(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                       h3_gpu_tensor *value, const h3_gpu_tensor *qkv,
                       const h3_gpu_tensor *q_norm,
                       const h3_gpu_tensor *k_norm,
                       const h3_gpu_tensor *rope_cos,
                       const h3_gpu_tensor *rope_sin, uint32_t sequence,
                       uint32_t heads, uint32_t head_dim, uint32_t rope_half,
                       float epsilon, uint32_t grouped) {
    size_t count = (size_t)sequence * heads * head_dim;
    if (rope_half * 2 > head_dim)
        return hk_fail(gpu, "RoPE half width exceeds the head dimension");
    if (!HK_REQ_BF16(qkv, count * 3, "QKV input") ||
        !HK_REQ_BF16(q_norm, head_dim, "Q norm") ||
        !HK_REQ_BF16(k_norm, head_dim, "K norm") ||
        !HK_REQ_BF16(rope_cos, (size_t)sequence * rope_half, "RoPE cosine") ||
        !HK_REQ_BF16(rope_sin, (size_t)sequence * rope_half, "RoPE sine") ||
        !HK_REQ_BF16(query, count, "query output") ||
        !HK_REQ_BF16(key, count, "key output") ||
        !HK_REQ_BF16(value, count, "value output") || !hk_require_active(gpu))
        return 0;
    const char *name = grouped ? "qk_norm_rope_grouped" : "qk_norm_rope";
    hk_op_begin(gpu, name);
    if (count) {
        const uintptr_t bases =
            (uintptr_t)qkv->data | (uintptr_t)q_norm->data |
            (uintptr_t)k_norm->data | (uintptr_t)rope_cos->data |
            (uintptr_t)rope_sin->data | (uintptr_t)query->data |
            (uintptr_t)key->data | (uintptr_t)value->data;
        const size_t vectors = (size_t)sequence * heads;
        if (head_dim == 128 && rope_half % 8 == 0 && (bases & 15u) == 0) {
            hipLaunchKernelGGL(hk_qk_norm_rope128v<8>,
                               dim3((unsigned)((vectors + 15) / 16)),
                               dim3(256), 0, gpu->stream, HK_CBF16(qkv),
                               HK_CBF16(q_norm), HK_CBF16(k_norm),
                               HK_CBF16(rope_cos), HK_CBF16(rope_sin),
                               HK_BF16(query), HK_BF16(key), HK_BF16(value),
                               sequence, heads, rope_half, grouped, epsilon);
        } else if (head_dim == 128 && rope_half % 4 == 0 &&
                   (bases & 7u) == 0) {
            hipLaunchKernelGGL(hk_qk_norm_rope128v<4>,
                               dim3((unsigned)((vectors + 7) / 8)), dim3(256),
                               0, gpu->stream, HK_CBF16(qkv), HK_CBF16(q_norm),
                               HK_CBF16(k_norm), HK_CBF16(rope_cos),
                               HK_CBF16(rope_sin), HK_BF16(query),
                               HK_BF16(key), HK_BF16(value), sequence, heads,
                               rope_half, grouped, epsilon);
        } else if (head_dim == 128 && rope_half % 2 == 0) {
            size_t waves = (size_t)sequence * heads;
            hipLaunchKernelGGL(hk_qk_norm_rope128,
                               dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                               gpu->stream, HK_CBF16(qkv), HK_CBF16(q_norm),
                               HK_CBF16(k_norm), HK_CBF16(rope_cos),
                               HK_CBF16(rope_sin), HK_BF16(query),
                               HK_BF16(key), HK_BF16(value), sequence, heads,
                               rope_half, grouped, epsilon);
        } else {
            hipLaunchKernelGGL(hk_qk_norm_rope_any<uint16_t>,
                               dim3((unsigned)((count + 255) / 256)),
                               dim3(256), 0, gpu->stream, HK_CBF16(qkv),
                               HK_CBF16(q_norm), HK_CBF16(k_norm),
                               HK_CBF16(rope_cos), HK_CBF16(rope_sin),
                               HK_BF16(query), HK_BF16(key), HK_BF16(value),
                               sequence, heads, head_dim, rope_half, grouped,
                               epsilon, 1u);
        }
    }
    return hk_op_end(gpu, name, HK_KIND_DIRECT);
}

int h3_gpu_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                         h3_gpu_tensor *value, const h3_gpu_tensor *qkv,
                         const h3_gpu_tensor *q_norm,
                         const h3_gpu_tensor *k_norm,
                         const h3_gpu_tensor *rope_cos,
                         const h3_gpu_tensor *rope_sin, uint32_t sequence,
                         uint32_t heads, uint32_t head_dim,
                         uint32_t rope_half, float epsilon) {
    return hk_qkv_rope(gpu, query, key, value, qkv, q_norm, k_norm, rope_cos,
                       rope_sin, sequence, heads, head_dim, rope_half,
                       epsilon, 0u);
}

int h3_gpu_grouped_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query,
                                 h3_gpu_tensor *key, h3_gpu_tensor *value,
                                 const h3_gpu_tensor *qkv,
                                 const h3_gpu_tensor *q_norm,
                                 const h3_gpu_tensor *k_norm,
                                 const h3_gpu_tensor *rope_cos,
                                 const h3_gpu_tensor *rope_sin,
                                 uint32_t sequence, uint32_t heads,
                                 uint32_t head_dim, uint32_t rope_half,
                                 float epsilon) {
    return hk_qkv_rope(gpu, query, key, value, qkv, q_norm, k_norm, rope_cos,
                       rope_sin, sequence, heads, head_dim, rope_half,
                       epsilon, 1u);
}

int h3_hip_qk_norm_rope_inplace_bf16(h3_gpu *gpu, h3_gpu_tensor *qkv,
                                     const h3_gpu_tensor *q_norm,
                                     const h3_gpu_tensor *k_norm,
                                     const h3_gpu_tensor *rope_cos,
                                     const h3_gpu_tensor *rope_sin,
                                     uint32_t sequence, uint32_t heads,
                                     uint32_t head_dim, uint32_t rope_half,
                                     float epsilon, int keys_only) {
    const size_t count = (size_t)sequence * heads * head_dim;
    if (!HK_REQ_BF16(qkv, count * 3, "QKV") ||
        !HK_REQ_BF16(q_norm, head_dim, "Q norm") ||
        !HK_REQ_BF16(k_norm, head_dim, "K norm") ||
        !HK_REQ_BF16(rope_cos, (size_t)sequence * rope_half, "RoPE cosine") ||
        !HK_REQ_BF16(rope_sin, (size_t)sequence * rope_half, "RoPE sine") ||
        !hk_require_active(gpu))
        return 0;
    const uintptr_t bases = (uintptr_t)qkv->data | (uintptr_t)q_norm->data |
                            (uintptr_t)k_norm->data |
                            (uintptr_t)rope_cos->data |
                            (uintptr_t)rope_sin->data;
    if (head_dim != 128 || rope_half % 8 != 0 || rope_half * 2 > head_dim ||
        (bases & 15u) != 0)
        return hk_fail(gpu, "in-place Q/K norm + RoPE needs head_dim 128, "
                            "rope_half a multiple of 8 and 16-byte aligned "
                            "tensors (got %u / %u)", head_dim, rope_half);
    hk_op_begin(gpu, "qk_norm_rope_inplace");
    const size_t vectors = (size_t)sequence * heads;
    if (vectors && keys_only)
        hipLaunchKernelGGL(hk_k_norm_rope128_inplace<HK_K_ITEMS>,
                           dim3((unsigned)((vectors + 16 * HK_K_ITEMS - 1) /
                                           (16 * HK_K_ITEMS))),
                           dim3(256), 0, gpu->stream, HK_BF16(qkv),
                           HK_CBF16(k_norm), HK_CBF16(rope_cos),
                           HK_CBF16(rope_sin), sequence, heads, rope_half,
                           epsilon);
    else if (vectors)
        hipLaunchKernelGGL((hk_qk_norm_rope128v<8, true>),
                           dim3((unsigned)((vectors + 15) / 16)), dim3(256), 0,
                           gpu->stream, HK_CBF16(qkv), HK_CBF16(q_norm),
                           HK_CBF16(k_norm), HK_CBF16(rope_cos),
                           HK_CBF16(rope_sin), HK_BF16(qkv), (uint16_t *)NULL,
                           (uint16_t *)NULL, sequence, heads, rope_half, 0u,
                           epsilon);
    return hk_op_end(gpu, "qk_norm_rope_inplace", HK_KIND_DIRECT);
}

int h3_gpu_qkv_rope_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                        h3_gpu_tensor *value, const h3_gpu_tensor *qkv,
                        const h3_gpu_tensor *q_norm,
                        const h3_gpu_tensor *k_norm,
                        const h3_gpu_tensor *rope_cos,
                        const h3_gpu_tensor *rope_sin, uint32_t sequence,
                        uint32_t heads, uint32_t head_dim, uint32_t rope_half,
                        float epsilon) {
    size_t count = (size_t)sequence * heads * head_dim;
    if (rope_half * 2 > head_dim)
        return hk_fail(gpu, "RoPE half width exceeds the head dimension");
    if (!HK_REQ_F32(qkv, count * 3, "QKV input") ||
        !HK_REQ_F32(q_norm, head_dim, "Q norm") ||
        !HK_REQ_F32(k_norm, head_dim, "K norm") ||
        !HK_REQ_F32(rope_cos, (size_t)sequence * rope_half, "RoPE cosine") ||
        !HK_REQ_F32(rope_sin, (size_t)sequence * rope_half, "RoPE sine") ||
        !HK_REQ_F32(query, count, "query output") ||
        !HK_REQ_F32(key, count, "key output") ||
        !HK_REQ_F32(value, count, "value output") || !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "qk_norm_rope_f32");
    if (count)
        hipLaunchKernelGGL(hk_qk_norm_rope_any<float>,
                           dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                           gpu->stream, HK_CF32(qkv), HK_CF32(q_norm),
                           HK_CF32(k_norm), HK_CF32(rope_cos),
                           HK_CF32(rope_sin), HK_F32(query), HK_F32(key),
                           HK_F32(value), sequence, heads, head_dim,
                           rope_half, 0u, epsilon, 1u);
    return hk_op_end(gpu, "qk_norm_rope_f32", HK_KIND_DIRECT);
}

int h3_gpu_head_rms_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor,
                              const h3_gpu_tensor *weight, uint32_t sequence,
                              uint32_t heads, uint32_t head_dim,
                              float epsilon) {
    size_t count = (size_t)sequence * heads * head_dim;
    if (!HK_REQ_BF16(tensor, count, "head norm tensor") ||
        !HK_REQ_BF16(weight, head_dim, "head norm weight") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "head_rms_norm");
    size_t waves = (size_t)sequence * heads;
    const bool wide = head_dim == 128 &&
                      (((uintptr_t)tensor->data | (uintptr_t)weight->data) &
                       15u) == 0;
    if (count && wide)
        hipLaunchKernelGGL(hk_head_rms128, dim3((unsigned)((waves + 15) / 16)),
                           dim3(256), 0, gpu->stream, HK_BF16(tensor),
                           HK_CBF16(weight), (uint32_t)waves, epsilon);
    else if (count)
        hipLaunchKernelGGL(hk_head_rms_kernel,
                           dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                           gpu->stream, HK_BF16(tensor), HK_CBF16(weight),
                           sequence, heads, head_dim, epsilon);
    return hk_op_end(gpu, "head_rms_norm", HK_KIND_DIRECT);
}

h3_gpu_tensor *h3_hip_head_norm_group_table(
    h3_gpu *gpu, h3_gpu_tensor *const *tensors,
    const h3_gpu_tensor *const *weights, uint32_t count, uint32_t rows,
    uint32_t heads, uint32_t head_dim) {
    if (!gpu) return NULL;
    if (!count || !tensors || !weights) {
        hk_fail(gpu, "grouped head norm table needs at least one problem");
        return NULL;
    }
    if (head_dim != 128) {
        hk_fail(gpu, "grouped head norm takes head_dim 128, not %u",
                head_dim);
        return NULL;
    }
    uint64_t *entries = (uint64_t *)calloc((size_t)count * 2, sizeof(uint64_t));
    if (!entries) {
        hk_fail(gpu, "out of host memory");
        return NULL;
    }
    for (uint32_t p = 0; p < count; p++) {
        if (!HK_REQ_BF16(tensors[p], (size_t)rows * heads * head_dim,
                         "grouped head norm tensor") ||
            !HK_REQ_BF16(weights[p], head_dim, "grouped head norm weight")) {
            free(entries);
            return NULL;
        }
        if ((((uintptr_t)tensors[p]->data | (uintptr_t)weights[p]->data) &
             15u) != 0) {
            free(entries);
            hk_fail(gpu, "grouped head norm problem %u: tensors not 16-byte "
                         "aligned", p);
            return NULL;
        }
        entries[2 * p] = (uint64_t)(uintptr_t)tensors[p]->data;
        entries[2 * p + 1] = (uint64_t)(uintptr_t)weights[p]->data;
    }
    h3_gpu_tensor *table = h3_gpu_tensor_from_u32(
        gpu, (const uint32_t *)entries, (size_t)count * 4);
    free(entries);
    if (table) {
        table->group_shape[0] = rows;
        table->group_shape[1] = heads;
        table->group_shape[2] = head_dim;
        table->group_shape[3] = count;
    }
    return table;
}

int h3_hip_head_rms_norm_group_bf16(h3_gpu *gpu, const h3_gpu_tensor *table,
                                    uint32_t first, uint32_t count,
                                    uint32_t rows, uint32_t heads,
                                    uint32_t head_dim, float epsilon) {
    if (table && table->group_shape[3] == 0)
        return hk_fail(gpu, "grouped head norm: the table was not built by "
                            "h3_hip_head_norm_group_table");
    if (table && (rows != table->group_shape[0] ||
                  heads != table->group_shape[1] ||
                  head_dim != table->group_shape[2]))
        return hk_fail(gpu, "grouped head norm: shape %ux%ux%u differs from "
                            "the table's %ux%ux%u", rows, heads, head_dim,
                       table->group_shape[0], table->group_shape[1],
                       table->group_shape[2]);
    if (table && (uint64_t)first + count > table->group_shape[3])
        return hk_fail(gpu, "grouped head norm: problems [%u, %u) past the "
                            "table's %u", first, first + count,
                       table->group_shape[3]);
    if (!hk_require(gpu, table, ((size_t)first + count) * 4, H3_GPU_U32,
                    "grouped head norm table") ||
        !hk_require_active(gpu))
        return 0;
    const uint64_t per = (uint64_t)rows * heads;
    const uint64_t vectors = per * count;
    if (!vectors) return 1;
    if (vectors > 0xffffffffull / 16u)
        return hk_fail(gpu, "grouped head norm: %llu vectors is too many",
                       (unsigned long long)vectors);
    hk_op_begin(gpu, "head_rms_norm_group");
    hipLaunchKernelGGL(hk_head_rms128_group,
                       dim3((unsigned)((vectors + 15) / 16)), dim3(256), 0,
                       gpu->stream,
                       (const uint64_t *)table->data + (size_t)first * 2,
                       (uint32_t)per, (uint32_t)vectors, epsilon);
    return hk_op_end(gpu, "head_rms_norm_group", HK_KIND_DIRECT);
}

/* ---- projections ---- */

static int hk_patch_common(h3_gpu *gpu, uint16_t *out,
                           const h3_gpu_tensor *input, size_t input_offset,
                           const h3_gpu_tensor *weight,
                           const h3_gpu_tensor *bias,
                           const uint32_t *row_map, uint32_t rows,
                           uint32_t input_dim, uint32_t output_dim,
                           const char *name) {
    hk_op_begin(gpu, name);
    if (rows && output_dim)
        hipLaunchKernelGGL(hk_patch_linear_kernel,
                           dim3((output_dim + 255) / 256, rows), dim3(256),
                           input_dim * sizeof(float), gpu->stream,
                           HK_CF32(input) + input_offset, HK_CF32(weight),
                           bias ? HK_CF32(bias) : (const float *)NULL, out,
                           row_map, rows, input_dim, output_dim);
    return hk_op_end(gpu, name, HK_KIND_DIRECT);
}

/* The reference's entry points take only its checkpoint's shapes (5376
 * outputs from 32 or 96 inputs: h3_cuda_core.cu:929-930, 1002-1003) and
 * reject the rest; the kernel itself is shape-generic, bounded by the F32
 * input row it stages in LDS, and the h3_hip_ variants below (small test
 * models) skip the fixed-shape check. */
static bool hk_patch_shape_ok(bool reference_shape, uint32_t input_dim,
                              uint32_t output_dim) {
    if (reference_shape)
        return output_dim == 5376 && (input_dim == 32 || input_dim == 96);
    return output_dim && input_dim && input_dim <= 4096;
}

static int hk_patch_offset(h3_gpu *gpu, bool reference_shape,
                           h3_gpu_tensor *output, size_t output_offset,
                           const h3_gpu_tensor *input, size_t input_offset,
                           const h3_gpu_tensor *weight,
                           const h3_gpu_tensor *bias, uint32_t rows,
                           uint32_t input_dim, uint32_t output_dim) {
    size_t input_count = (size_t)rows * input_dim;
    size_t output_count = (size_t)rows * output_dim;
    if (!hk_patch_shape_ok(reference_shape, input_dim, output_dim))
        return hk_fail(gpu, "unsupported fused patch projection shape");
    if (input_offset > SIZE_MAX - input_count ||
        output_offset > SIZE_MAX - output_count)
        return hk_fail(gpu, "fused patch projection offset is out of range");
    if (!HK_REQ_F32(input, input_offset + input_count, "patch projection input") ||
        !HK_REQ_F32(weight, (size_t)output_dim * input_dim,
                    "patch projection weight") ||
        !HK_REQ_BF16(output, output_offset + output_count,
                     "patch projection output") ||
        (bias && !HK_REQ_F32(bias, output_dim, "patch projection bias")) ||
        !hk_require_active(gpu))
        return 0;
    return hk_patch_common(gpu, HK_BF16(output) + output_offset, input,
                           input_offset, weight, bias, NULL, rows, input_dim,
                           output_dim, "patch_linear");
}

static int hk_patch_map(h3_gpu *gpu, bool reference_shape,
                        h3_gpu_tensor *output, const h3_gpu_tensor *input,
                        const h3_gpu_tensor *weight, const h3_gpu_tensor *bias,
                        const h3_gpu_tensor *row_map, uint32_t output_rows,
                        uint32_t rows, uint32_t input_dim,
                        uint32_t output_dim) {
    if (!hk_patch_shape_ok(reference_shape, input_dim, output_dim))
        return hk_fail(gpu, "unsupported mapped patch projection shape");
    if (!HK_REQ_F32(input, (size_t)rows * input_dim, "mapped patch input") ||
        !HK_REQ_F32(weight, (size_t)output_dim * input_dim,
                    "mapped patch weight") ||
        !HK_REQ_BF16(output, (size_t)output_rows * output_dim,
                     "mapped patch output") ||
        !HK_REQ_U32(row_map, rows, "mapped patch row map") ||
        (bias && !HK_REQ_F32(bias, output_dim, "mapped patch bias")) ||
        !hk_require_active(gpu))
        return 0;
    /* the kernel scatters to row_map[r]: validate targets on the host so a
     * bad map cannot write outside the output tensor */
    if (rows) {
        uint32_t *map = (uint32_t *)malloc((size_t)rows * 4);
        if (!map) return hk_fail(gpu, "out of memory");
        hipError_t status = hipStreamSynchronize(gpu->stream);
        if (status == hipSuccess)
            status = hipMemcpy(map, row_map->data, (size_t)rows * 4,
                               hipMemcpyDeviceToHost);
        if (status != hipSuccess) {
            free(map);
            return hk_fail_hip(gpu, "row map check", status);
        }
        for (uint32_t r = 0; r < rows; r++)
            if (map[r] >= output_rows) {
                free(map);
                return hk_fail(gpu, "mapped patch row %u targets row %u of %u",
                               r, map[r], output_rows);
            }
        free(map);
    }
    return hk_patch_common(gpu, HK_BF16(output), input, 0, weight, bias,
                           HK_CU32(row_map), rows, input_dim, output_dim,
                           "patch_linear_map");
}

int h3_gpu_patch_linear_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output,
                                    size_t output_offset,
                                    const h3_gpu_tensor *input,
                                    size_t input_offset,
                                    const h3_gpu_tensor *weight,
                                    const h3_gpu_tensor *bias, uint32_t rows,
                                    uint32_t input_dim, uint32_t output_dim) {
    return hk_patch_offset(gpu, true, output, output_offset, input,
                           input_offset, weight, bias, rows, input_dim,
                           output_dim);
}

int h3_gpu_patch_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                             const h3_gpu_tensor *input,
                             const h3_gpu_tensor *weight,
                             const h3_gpu_tensor *bias, uint32_t rows,
                             uint32_t input_dim, uint32_t output_dim) {
    return hk_patch_offset(gpu, true, output, 0, input, 0, weight, bias, rows,
                           input_dim, output_dim);
}

int h3_gpu_patch_linear_bf16_map(h3_gpu *gpu, h3_gpu_tensor *output,
                                 const h3_gpu_tensor *input,
                                 const h3_gpu_tensor *weight,
                                 const h3_gpu_tensor *bias,
                                 const h3_gpu_tensor *row_map,
                                 uint32_t output_rows, uint32_t rows,
                                 uint32_t input_dim, uint32_t output_dim) {
    return hk_patch_map(gpu, true, output, input, weight, bias, row_map,
                        output_rows, rows, input_dim, output_dim);
}

int h3_hip_patch_linear_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output,
                                    size_t output_offset,
                                    const h3_gpu_tensor *input,
                                    size_t input_offset,
                                    const h3_gpu_tensor *weight,
                                    const h3_gpu_tensor *bias, uint32_t rows,
                                    uint32_t input_dim, uint32_t output_dim) {
    return hk_patch_offset(gpu, false, output, output_offset, input,
                           input_offset, weight, bias, rows, input_dim,
                           output_dim);
}

int h3_hip_patch_linear_bf16_map(h3_gpu *gpu, h3_gpu_tensor *output,
                                 const h3_gpu_tensor *input,
                                 const h3_gpu_tensor *weight,
                                 const h3_gpu_tensor *bias,
                                 const h3_gpu_tensor *row_map,
                                 uint32_t output_rows, uint32_t rows,
                                 uint32_t input_dim, uint32_t output_dim) {
    return hk_patch_map(gpu, false, output, input, weight, bias, row_map,
                        output_rows, rows, input_dim, output_dim);
}

int h3_gpu_linear_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                      const h3_gpu_tensor *input, const h3_gpu_tensor *weight,
                      const h3_gpu_tensor *bias, uint32_t rows,
                      uint32_t input_dim, uint32_t output_dim) {
    if (!HK_REQ_F32(input, (size_t)rows * input_dim, "linear input") ||
        !HK_REQ_F32(weight, (size_t)output_dim * input_dim, "linear weight") ||
        !HK_REQ_F32(output, (size_t)rows * output_dim, "linear output") ||
        (bias && !HK_REQ_F32(bias, output_dim, "linear bias")) ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "linear_f32");
    if (rows && output_dim)
        hipLaunchKernelGGL(hk_linear_f32_kernel,
                           dim3((output_dim + 255) / 256, rows), dim3(256), 0,
                           gpu->stream, HK_CF32(input), HK_CF32(weight),
                           bias ? HK_CF32(bias) : (const float *)NULL,
                           HK_F32(output), rows, input_dim, output_dim);
    int kind = rows >= 32 && input_dim >= 256 && output_dim >= 256
                   ? HK_KIND_LINEAR : HK_KIND_DIRECT;
    return hk_op_end(gpu, "linear_f32", kind);
}

int h3_gpu_adaln_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                             h3_gpu_tensor *inverse,
                             const h3_gpu_tensor *input, size_t input_offset,
                             const h3_gpu_tensor *norm_weight,
                             const h3_gpu_tensor *modulation,
                             const h3_gpu_tensor *row_map,
                             const h3_gpu_tensor *weight,
                             const h3_gpu_tensor *bias, uint32_t rows,
                             uint32_t width, uint32_t output_dim,
                             uint32_t slots, uint32_t shift_slot,
                             uint32_t scale_slot, float epsilon) {
    size_t input_count = (size_t)rows * width;
    if (input_offset > SIZE_MAX - input_count)
        return hk_fail(gpu, "fused final head input offset is out of range");
    if (!HK_REQ_BF16(input, input_offset + input_count,
                     "fused final head input") ||
        !HK_REQ_F32(inverse, rows, "fused final head inverse RMS") ||
        !HK_REQ_BF16(norm_weight, width, "fused final head norm") ||
        !HK_REQ_BF16(modulation, 1, "fused final head modulation") ||
        !HK_REQ_U32(row_map, rows, "fused final head row map") ||
        !HK_REQ_BF16(weight, (size_t)output_dim * width,
                     "fused final head weight") ||
        !HK_REQ_BF16(output, (size_t)rows * output_dim,
                     "fused final head output") ||
        (bias && !HK_REQ_BF16(bias, output_dim, "fused final head bias")) ||
        !hk_require_active(gpu))
        return 0;
    if (shift_slot >= slots || scale_slot >= slots)
        return hk_fail(gpu, "fused final head modulation slot out of range");
    if ((size_t)width * sizeof(float) > 64 * 1024)
        return hk_fail(gpu, "fused final head width is too large");
    hk_op_begin(gpu, "adaln_head");
    if (rows && width)
        hipLaunchKernelGGL(hk_adaln_head_kernel, dim3(rows), dim3(256),
                           width * sizeof(float), gpu->stream,
                           HK_CBF16(input) + input_offset, HK_F32(inverse),
                           HK_CBF16(norm_weight), HK_CBF16(modulation),
                           HK_CU32(row_map), HK_CBF16(weight),
                           bias ? HK_CBF16(bias) : (const uint16_t *)NULL,
                           HK_BF16(output), width, output_dim, slots,
                           shift_slot, scale_slot, epsilon);
    return hk_op_end(gpu, "adaln_head", HK_KIND_DIRECT);
}

/* ---- seeded fill ---- */

int h3_gpu_fill_normal_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor, size_t offset,
                            size_t elements, uint64_t seed, float mean,
                            float stddev) {
    if (offset > SIZE_MAX - elements ||
        !HK_REQ_BF16(tensor, offset + elements, "normal fill"))
        return 0;
    hk_op_begin(gpu, "fill_normal");
    if (elements)
        hipLaunchKernelGGL(hk_fill_normal_kernel<uint16_t>,
                           dim3((unsigned)(gpu->num_cus * 8)), dim3(256), 0,
                           gpu->stream, HK_BF16(tensor) + offset, elements,
                           seed, mean, stddev);
    return hk_op_end(gpu, "fill_normal", HK_KIND_DIRECT);
}

int h3_gpu_fill_normal_f32(h3_gpu *gpu, h3_gpu_tensor *tensor, size_t offset,
                           size_t elements, uint64_t seed, float mean,
                           float stddev) {
    if (offset > SIZE_MAX - elements ||
        !HK_REQ_F32(tensor, offset + elements, "normal fill"))
        return 0;
    hk_op_begin(gpu, "fill_normal");
    if (elements)
        hipLaunchKernelGGL(hk_fill_normal_kernel<float>,
                           dim3((unsigned)(gpu->num_cus * 8)), dim3(256), 0,
                           gpu->stream, HK_F32(tensor) + offset, elements,
                           seed, mean, stddev);
    return hk_op_end(gpu, "fill_normal", HK_KIND_DIRECT);
}

} /* extern "C" */

/* ------------------------------------------------------ token reduction */

static int hk_token_fits(const h3_gpu_tensor *t, size_t offset, size_t count,
                         h3_gpu_dtype dtype) {
    return t && t->dtype == dtype && offset <= t->elements &&
           count <= t->elements - offset && t->bytes < 0xfffff000ull;
}

static int hk_token_launch(h3_gpu *gpu, bool expand, bool adaln,
                           hk_token_args &a, const char *name) {
    hk_op_begin(gpu, name);
    if (a.rows) {
        if (!expand && !adaln)
            hipLaunchKernelGGL((hk_token_kernel<false, false>), dim3(a.rows),
                               dim3(256), 0, gpu->stream, a);
        else if (!expand)
            hipLaunchKernelGGL((hk_token_kernel<false, true>), dim3(a.rows),
                               dim3(256), 0, gpu->stream, a);
        else if (!adaln)
            hipLaunchKernelGGL((hk_token_kernel<true, false>), dim3(a.rows),
                               dim3(256), 0, gpu->stream, a);
        else
            hipLaunchKernelGGL((hk_token_kernel<true, true>), dim3(a.rows),
                               dim3(256), 0, gpu->stream, a);
    }
    return hk_op_end(gpu, name, HK_KIND_DIRECT);
}

/* Shared validation of the pool ops (reference h3_cuda_dit.cu:797-921). */
static int hk_pool_setup(h3_gpu *gpu, hk_token_args &a, h3_gpu_tensor *output,
                         const h3_gpu_tensor *input, size_t input_offset,
                         h3_gpu_tensor *original, size_t original_offset,
                         h3_gpu_tensor *baseline, size_t baseline_offset,
                         const h3_gpu_tensor *baseline_indices,
                         const h3_gpu_tensor *pairs, uint32_t input_rows,
                         uint32_t rows, uint32_t baseline_rows,
                         uint32_t width, const char *what) {
    const size_t elements = (size_t)rows * width;
    const size_t input_elements = (size_t)input_rows * width;
    const size_t baseline_elements = (size_t)baseline_rows * width;
    if (!input_rows || !rows || rows > input_rows || baseline_rows > rows ||
        !width || elements > UINT32_MAX || input_offset > UINT32_MAX ||
        input_elements > UINT32_MAX - input_offset ||
        original_offset > UINT32_MAX ||
        input_elements > UINT32_MAX - original_offset ||
        baseline_offset > UINT32_MAX ||
        baseline_elements > UINT32_MAX - baseline_offset)
        return hk_fail(gpu, "%s shape is out of range", what);
    if (width % 8 || width > 256 * 8 * HK_TOKEN_CHUNKS)
        return hk_fail(gpu, "%s width must be a multiple of 8 up to %d", what,
                       256 * 8 * HK_TOKEN_CHUNKS);
    if (!hk_token_fits(input, input_offset, input_elements, H3_GPU_BF16))
        return hk_fail(gpu, "%s input tensor is too small", what);
    if (!hk_token_fits(original, original_offset, input_elements,
                       H3_GPU_BF16))
        return hk_fail(gpu, "%s original tensor is too small", what);
    if (!hk_token_fits(baseline, baseline_offset, baseline_elements,
                       H3_GPU_BF16))
        return hk_fail(gpu, "%s baseline tensor is too small", what);
    if (!HK_REQ_BF16(output, elements, "token pool output") ||
        !HK_REQ_U32(baseline_indices, rows, "token pool baseline indices") ||
        !HK_REQ_U32(pairs, (size_t)rows * 2, "token pool pairs") ||
        !hk_require_active(gpu))
        return 0;
    memset(&a, 0, sizeof(a));
    a.input = HK_CBF16(input);
    a.original = HK_BF16(original);
    a.baseline = HK_BF16(baseline);
    a.baseline_indices = HK_CU32(baseline_indices);
    a.index = HK_CU32(pairs);
    a.residual = HK_BF16(output);
    a.input_bytes = (uint32_t)input->bytes;
    a.original_bytes = (uint32_t)original->bytes;
    a.baseline_bytes = (uint32_t)baseline->bytes;
    a.index_bytes = (uint32_t)pairs->bytes;
    a.baseline_index_bytes = (uint32_t)baseline_indices->bytes;
    a.input_offset = (uint32_t)input_offset;
    a.original_offset = (uint32_t)original_offset;
    a.baseline_offset = (uint32_t)baseline_offset;
    a.rows = rows;
    a.width = width;
    return 1;
}

static int hk_adaln_setup(h3_gpu *gpu, hk_token_args &a, h3_gpu_tensor *out,
                          const h3_gpu_tensor *norm_weight,
                          const h3_gpu_tensor *modulation,
                          const h3_gpu_tensor *row_map, uint32_t rows,
                          uint32_t width, uint32_t slots, uint32_t shift_slot,
                          uint32_t scale_slot, float epsilon,
                          const char *what) {
    if (width > 5376)
        return hk_fail(gpu, "%s width is out of range", what);
    if (shift_slot >= slots || scale_slot >= slots)
        return hk_fail(gpu, "%s modulation slot out of range", what);
    if (!HK_REQ_BF16(norm_weight, width, "fused token adaLN norm") ||
        !HK_REQ_BF16(modulation, 1, "fused token adaLN modulation") ||
        !HK_REQ_U32(row_map, rows, "fused token adaLN row map") ||
        !HK_REQ_BF16(out, (size_t)rows * width, "fused token adaLN output"))
        return 0;
    a.adaln = HK_BF16(out);
    a.norm_weight = HK_CBF16(norm_weight);
    a.modulation = HK_CBF16(modulation);
    a.row_map = HK_CU32(row_map);
    a.slots = slots;
    a.shift_slot = shift_slot;
    a.scale_slot = scale_slot;
    a.epsilon = epsilon;
    return 1;
}

extern "C" int h3_gpu_token_pool_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                      const h3_gpu_tensor *input,
                                      size_t input_offset,
                                      h3_gpu_tensor *original,
                                      size_t original_offset,
                                      h3_gpu_tensor *baseline,
                                      size_t baseline_offset,
                                      const h3_gpu_tensor *baseline_indices,
                                      const h3_gpu_tensor *pairs,
                                      uint32_t input_rows, uint32_t rows,
                                      uint32_t baseline_rows, uint32_t width) {
    hk_token_args a;
    if (!hk_pool_setup(gpu, a, output, input, input_offset, original,
                       original_offset, baseline, baseline_offset,
                       baseline_indices, pairs, input_rows, rows,
                       baseline_rows, width, "token pool"))
        return 0;
    return hk_token_launch(gpu, false, false, a, "token_pool");
}

extern "C" int h3_gpu_token_pool_adaln_bf16(
    h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output,
    const h3_gpu_tensor *input, size_t input_offset, h3_gpu_tensor *original,
    size_t original_offset, h3_gpu_tensor *baseline, size_t baseline_offset,
    const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *pairs,
    const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation,
    const h3_gpu_tensor *row_map, uint32_t input_rows, uint32_t rows,
    uint32_t baseline_rows, uint32_t width, uint32_t slots,
    uint32_t shift_slot, uint32_t scale_slot, float epsilon) {
    hk_token_args a;
    if (!hk_pool_setup(gpu, a, residual, input, input_offset, original,
                       original_offset, baseline, baseline_offset,
                       baseline_indices, pairs, input_rows, rows,
                       baseline_rows, width, "fused token pool") ||
        !hk_adaln_setup(gpu, a, output, norm_weight, modulation, row_map,
                        rows, width, slots, shift_slot, scale_slot, epsilon,
                        "fused token pool"))
        return 0;
    return hk_token_launch(gpu, false, true, a, "token_pool_adaln");
}

/* Shared validation of the expand ops (reference h3_cuda_dit.cu:923-1074). */
static int hk_expand_setup(h3_gpu *gpu, hk_token_args &a,
                           h3_gpu_tensor *output,
                           const h3_gpu_tensor *original,
                           size_t original_offset,
                           const h3_gpu_tensor *reduced,
                           const h3_gpu_tensor *baseline,
                           size_t baseline_offset,
                           const h3_gpu_tensor *baseline_indices,
                           const h3_gpu_tensor *parents, uint32_t rows,
                           uint32_t reduced_rows, uint32_t baseline_rows,
                           uint32_t width, uint32_t exact_prefix_rows,
                           float update_scale, const char *what) {
    const size_t elements = (size_t)rows * width;
    const size_t reduced_elements = (size_t)reduced_rows * width;
    const size_t baseline_elements = (size_t)baseline_rows * width;
    if (!rows || !reduced_rows || reduced_rows > rows ||
        baseline_rows > reduced_rows || !width ||
        exact_prefix_rows > reduced_rows || elements > UINT32_MAX ||
        reduced_elements > UINT32_MAX || original_offset > UINT32_MAX ||
        elements > UINT32_MAX - original_offset ||
        baseline_offset > UINT32_MAX ||
        baseline_elements > UINT32_MAX - baseline_offset)
        return hk_fail(gpu, "%s shape is out of range", what);
    if (width % 8 || width > 256 * 8 * HK_TOKEN_CHUNKS)
        return hk_fail(gpu, "%s width must be a multiple of 8 up to %d", what,
                       256 * 8 * HK_TOKEN_CHUNKS);
    if (!hk_token_fits(original, original_offset, elements, H3_GPU_BF16))
        return hk_fail(gpu, "%s original tensor is too small", what);
    if (!hk_token_fits(baseline, baseline_offset, baseline_elements,
                       H3_GPU_BF16))
        return hk_fail(gpu, "%s baseline tensor is too small", what);
    if (!hk_token_fits(reduced, 0, reduced_elements, H3_GPU_BF16))
        return hk_fail(gpu, "%s reduced tensor is too small", what);
    if (!HK_REQ_BF16(output, elements, "token expand output") ||
        !HK_REQ_U32(baseline_indices, reduced_rows,
                    "token expand baseline indices") ||
        !HK_REQ_U32(parents, rows, "token expand parents") ||
        !hk_require_active(gpu))
        return 0;
    memset(&a, 0, sizeof(a));
    a.input = HK_CBF16(reduced);
    a.original = (uint16_t *)HK_CBF16(original);
    a.baseline = (uint16_t *)HK_CBF16(baseline);
    a.baseline_indices = HK_CU32(baseline_indices);
    a.index = HK_CU32(parents);
    a.residual = HK_BF16(output);
    a.input_bytes = (uint32_t)reduced->bytes;
    a.original_bytes = (uint32_t)original->bytes;
    a.baseline_bytes = (uint32_t)baseline->bytes;
    a.index_bytes = (uint32_t)parents->bytes;
    a.baseline_index_bytes = (uint32_t)baseline_indices->bytes;
    a.original_offset = (uint32_t)original_offset;
    a.baseline_offset = (uint32_t)baseline_offset;
    a.rows = rows;
    a.width = width;
    a.exact_prefix_rows = exact_prefix_rows;
    a.update_scale = update_scale;
    return 1;
}

extern "C" int h3_gpu_token_expand_delta_bf16(
    h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *original,
    size_t original_offset, const h3_gpu_tensor *reduced,
    const h3_gpu_tensor *baseline, size_t baseline_offset,
    const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *parents,
    uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows,
    uint32_t width, uint32_t exact_prefix_rows, float update_scale) {
    hk_token_args a;
    if (!hk_expand_setup(gpu, a, output, original, original_offset, reduced,
                         baseline, baseline_offset, baseline_indices, parents,
                         rows, reduced_rows, baseline_rows, width,
                         exact_prefix_rows, update_scale, "token expand"))
        return 0;
    return hk_token_launch(gpu, true, false, a, "token_expand");
}

extern "C" int h3_gpu_token_expand_adaln_bf16(
    h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output,
    const h3_gpu_tensor *original, size_t original_offset,
    const h3_gpu_tensor *reduced, const h3_gpu_tensor *baseline,
    size_t baseline_offset, const h3_gpu_tensor *baseline_indices,
    const h3_gpu_tensor *parents, const h3_gpu_tensor *norm_weight,
    const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map,
    uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows,
    uint32_t width, uint32_t exact_prefix_rows, float update_scale,
    uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon) {
    hk_token_args a;
    if (!hk_expand_setup(gpu, a, residual, original, original_offset, reduced,
                         baseline, baseline_offset, baseline_indices, parents,
                         rows, reduced_rows, baseline_rows, width,
                         exact_prefix_rows, update_scale,
                         "fused token adaLN") ||
        !hk_adaln_setup(gpu, a, output, norm_weight, modulation, row_map,
                        rows, width, slots, shift_slot, scale_slot, epsilon,
                        "fused token adaLN"))
        return 0;
    return hk_token_launch(gpu, true, true, a, "token_expand_adaln");
}

/* ===================== F32 utility ops outside the DiT path =====================
 * The text-encoder / VAE helpers of h3_gpu.h that the reference's own core
 * test program exercises (tests/test_cuda_core.c): GeGLU (tanh GELU of the
 * gate times the linear half), clip, a*l + b*r, residual + branch * scale
 * per column, token embedding gather and weight normalisation.  Same
 * arithmetic as the reference kernels (h3_cuda_core.cu:31-66, 116-126,
 * 296-318); the transcendental is the device library's tanhf. */
enum { HK_F32_GEGLU, HK_F32_CLIP, HK_F32_ADD_SCALED, HK_F32_SCALE_ADD };

template <int OP>
__global__ void hk_f32_util(const float *__restrict__ a,
                            const float *__restrict__ b,
                            const float *__restrict__ c, float *out,
                            size_t count, uint32_t width, float p0,
                            float p1) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const float x = a[i];
        float y;
        if (OP == HK_F32_GEGLU) {
            const float inner = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
            y = 0.5f * x * (1.0f + tanhf(inner)) * b[i];
        } else if (OP == HK_F32_CLIP) {
            y = fminf(fmaxf(x, p0), p1);
        } else if (OP == HK_F32_ADD_SCALED) {
            y = x * p0 + b[i] * p1;
        } else {
            y = x + b[i] * c[i % width];
        }
        out[i] = y;
    }
}

template <int OP>
static void hk_f32_util_launch(struct h3_gpu *gpu, const float *a,
                               const float *b, const float *c, float *out,
                               size_t count, uint32_t width, float p0,
                               float p1) {
    if (!count) return;
    size_t blocks = (count + 255) / 256;
    const size_t cap = (size_t)gpu->num_cus * 16;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(hk_f32_util<OP>, dim3((unsigned)blocks), dim3(256), 0,
                       gpu->stream, a, b, c, out, count, width, p0, p1);
}

/* row t of the output = weight row ids[t], zeros for ids past the
 * vocabulary; 16-byte copies when the width allows */
__global__ void hk_embedding_kernel(const uint16_t *__restrict__ weight,
                                    const uint32_t *__restrict__ ids,
                                    uint16_t *__restrict__ out,
                                    uint32_t vocab, uint32_t width) {
    const uint32_t token = blockIdx.x;
    const uint32_t id = ids[token];
    uint16_t *dst = out + (size_t)token * width;
    const uint16_t *src = weight + (size_t)id * width;
    const bool valid = id < vocab;
    if (width % 8 == 0) {
        for (uint32_t c = threadIdx.x * 8; c < width; c += blockDim.x * 8)
            *(uint4 *)(dst + c) =
                valid ? *(const uint4 *)(src + c) : make_uint4(0, 0, 0, 0);
    } else {
        for (uint32_t c = threadIdx.x; c < width; c += blockDim.x)
            dst[c] = valid ? src[c] : (uint16_t)0;
    }
}

/* out row = v row * (g[row] / ||v row||), no epsilon */
__global__ void __launch_bounds__(HK_ROW_THREADS)
hk_weight_norm_kernel(const float *__restrict__ v,
                      const float *__restrict__ g, float *__restrict__ out,
                      uint32_t inner) {
    __shared__ float scratch[16];
    const size_t base = (size_t)blockIdx.x * inner;
    float local = 0.0f;
    for (uint32_t i = threadIdx.x; i < inner; i += HK_ROW_THREADS)
        local = fmaf(v[base + i], v[base + i], local);
    const float scale = g[blockIdx.x] / sqrtf(hk_block_sum(local, scratch));
    for (uint32_t i = threadIdx.x; i < inner; i += HK_ROW_THREADS)
        out[base + i] = v[base + i] * scale;
}

extern "C" {

int h3_gpu_geglu_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *gate, const h3_gpu_tensor *linear,
                     uint32_t elements) {
    if (!HK_REQ_F32(gate, elements, "GeGLU gate") ||
        !HK_REQ_F32(linear, elements, "GeGLU linear") ||
        !HK_REQ_F32(output, elements, "GeGLU output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "geglu_f32");
    hk_f32_util_launch<HK_F32_GEGLU>(gpu, HK_CF32(gate), HK_CF32(linear), NULL,
                                     HK_F32(output), elements, 1, 0, 0);
    return hk_op_end(gpu, "geglu_f32", HK_KIND_DIRECT);
}

int h3_gpu_clip_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *input, uint32_t elements,
                    float minimum, float maximum) {
    if (!(minimum <= maximum))
        return hk_fail(gpu, "clip minimum exceeds maximum");
    if (!HK_REQ_F32(input, elements, "clip input") ||
        !HK_REQ_F32(output, elements, "clip output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "clip_f32");
    hk_f32_util_launch<HK_F32_CLIP>(gpu, HK_CF32(input), NULL, NULL,
                                    HK_F32(output), elements, 1, minimum,
                                    maximum);
    return hk_op_end(gpu, "clip_f32", HK_KIND_DIRECT);
}

int h3_gpu_add_scaled_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *left,
                          const h3_gpu_tensor *right, float left_scale,
                          float right_scale, uint32_t elements) {
    if (!HK_REQ_F32(left, elements, "scaled-add left") ||
        !HK_REQ_F32(right, elements, "scaled-add right") ||
        !HK_REQ_F32(output, elements, "scaled-add output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "add_scaled_f32");
    hk_f32_util_launch<HK_F32_ADD_SCALED>(gpu, HK_CF32(left), HK_CF32(right),
                                          NULL, HK_F32(output), elements, 1,
                                          left_scale, right_scale);
    return hk_op_end(gpu, "add_scaled_f32", HK_KIND_DIRECT);
}

int h3_gpu_scale_add_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                         const h3_gpu_tensor *residual,
                         const h3_gpu_tensor *branch,
                         const h3_gpu_tensor *scale, uint32_t rows,
                         uint32_t width) {
    const size_t count = (size_t)rows * width;
    if (!HK_REQ_F32(residual, count, "scale-add residual") ||
        !HK_REQ_F32(branch, count, "scale-add branch") ||
        !HK_REQ_F32(scale, width, "scale-add scale") ||
        !HK_REQ_F32(output, count, "scale-add output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "scale_add_f32");
    hk_f32_util_launch<HK_F32_SCALE_ADD>(gpu, HK_CF32(residual),
                                         HK_CF32(branch), HK_CF32(scale),
                                         HK_F32(output), count, width, 0, 0);
    return hk_op_end(gpu, "scale_add_f32", HK_KIND_DIRECT);
}

int h3_gpu_embedding_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *weight,
                          const h3_gpu_tensor *token_ids, uint32_t tokens,
                          uint32_t vocab_size, uint32_t width) {
    if (!HK_REQ_BF16(weight, (size_t)vocab_size * width, "embedding weight") ||
        !HK_REQ_U32(token_ids, tokens, "token IDs") ||
        !HK_REQ_BF16(output, (size_t)tokens * width, "embedding output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "embedding_bf16");
    if (tokens && width)
        hipLaunchKernelGGL(hk_embedding_kernel, dim3(tokens), dim3(256), 0,
                           gpu->stream, HK_CBF16(weight),
                           (const uint32_t *)token_ids->data, HK_BF16(output),
                           vocab_size, width);
    return hk_op_end(gpu, "embedding_bf16", HK_KIND_DIRECT);
}

int h3_gpu_weight_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *vector,
                           const h3_gpu_tensor *magnitude, uint32_t outer,
                           uint32_t inner) {
    const size_t count = (size_t)outer * inner;
    if (!outer || !inner)
        return hk_fail(gpu, "weight-norm dimensions must be nonzero");
    if (!HK_REQ_F32(vector, count, "weight-norm vector") ||
        !HK_REQ_F32(magnitude, outer, "weight-norm magnitude") ||
        !HK_REQ_F32(output, count, "weight-norm output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "weight_norm_f32");
    hipLaunchKernelGGL(hk_weight_norm_kernel, dim3(outer),
                       dim3(HK_ROW_THREADS), 0, gpu->stream, HK_CF32(vector),
                       HK_CF32(magnitude), HK_F32(output), inner);
    return hk_op_end(gpu, "weight_norm_f32", HK_KIND_DIRECT);
}

} /* extern "C" */

