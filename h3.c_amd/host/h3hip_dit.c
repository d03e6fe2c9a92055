/* DiT denoiser driver over the h3_gpu.h device API; see h3hip_dit.h. */
#include "h3hip_dit.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { SLOTS = 6 };

typedef struct {
    h3_gpu_tensor *norm1, *norm2, *norm3, *norm3_bias;
    h3_gpu_tensor *qkv, *qkv_bias, *q_norm, *k_norm, *out, *out_bias;
    h3_gpu_tensor *fc1, *fc1_bias, *fc2, *fc2_bias;
    h3_gpu_tensor *cq, *cq_bias, *ck, *ck_bias, *cv, *cv_bias;
    h3_gpu_tensor *cq_norm, *ck_norm, *co, *co_bias;
    h3_gpu_tensor *modulation;
    /* Wan: this block's cross-attention K and V of the text, projected for
     * all blocks at the start of a forward (they depend on the text only) */
    h3_gpu_tensor *ctx_k, *ctx_v;
} h3hip_block;

struct h3hip_dit {
    h3_gpu *gpu;
    h3hip_dit_config config;
    uint32_t modalities; /* H3: 3 tags per time row; Wan: 1 */
    h3hip_block *blocks;
    /* shared state and activations */
    h3_gpu_tensor *hidden, *row_map, *rope_cos, *rope_sin, *context;
    h3_gpu_tensor *mod_a, *mod_b, *qkv, *query, *key, *value, *attn, *proj;
    h3_gpu_tensor *cross_q, *cross_out, *ffn_act;
    /* Wan: the grouped projection's table, problems (block b's K, V) at
     * 2 b and 2 b + 1 */
    h3_gpu_tensor *ctx_table;
    /* Wan: every block's text-key head norm, problem b = block b */
    h3_gpu_tensor *knorm_table;
    int attention_adaln_ready;
    unsigned op_mask;
    /* H3 sampler */
    int sampler;
    int steps, reuse_interval;
    uint32_t video_patch, audio_channels;
    float *video_sigmas, *audio_sigmas;
    h3hip_segment *segments;
    size_t segment_count;
    uint32_t video_total, audio_total;       /* latent rows per modality */
    uint32_t video_conditions, audio_conditions;
    uint32_t video_targets, audio_targets;
    uint32_t video_target_start, audio_target_start; /* rows in hidden */
    h3_gpu_tensor *video_input, *audio_input; /* F32 latent rows */
    h3_gpu_tensor *video_patch_w, *video_patch_b; /* F32 */
    h3_gpu_tensor *audio_patch_w, *audio_patch_b;
    h3_gpu_tensor *refined_text, *final_norm, *final_mod;
    h3_gpu_tensor *final_video_w, *final_video_b;
    h3_gpu_tensor *final_audio_w, *final_audio_b;
    h3_gpu_tensor *video_velocity, *audio_velocity;
    h3_gpu_tensor *video_previous, *audio_previous;
    h3_gpu_tensor *video_inverse, *audio_inverse;
    h3_gpu_tensor **step_maps, **final_video_maps, **final_audio_maps;
    h3_gpu_tensor *default_row_map;
    h3_gpu_tensor *time_in_w, *time_in_b, *time_out_w, *time_out_b;
    char error[512];
};

static int dit_fail(h3hip_dit *dit, const char *format, ...) {
    va_list arguments;
    va_start(arguments, format);
    vsnprintf(dit->error, sizeof(dit->error), format, arguments);
    va_end(arguments);
    return 0;
}

static int dit_op(h3hip_dit *dit, int ok, const char *what) {
    if (ok) return 1;
    return dit_fail(dit, "%s: %s", what, h3_gpu_error(dit->gpu));
}

/* Issue `call` only when its op class is enabled (see run_blocks_ops). */
#define DIT_OP(klass, call, what)                                           \
    ((dit->op_mask & (klass)) ? dit_op(dit, (call), (what)) : 1)
#define K_GEMM H3HIP_OPS_GEMM
#define K_ACT H3HIP_OPS_GEMM_ACT
#define K_ATTN H3HIP_OPS_ATTENTION
#define K_ROWS H3HIP_OPS_ROWS
#define K_CTX H3HIP_OPS_CONTEXT

const char *h3hip_dit_error(const h3hip_dit *dit) {
    return dit ? dit->error : "no DiT";
}

static int is_wan(const h3hip_dit *dit) {
    return dit->config.family == H3HIP_FAMILY_WAN;
}

/* ------------------------------------------------------------ FLOPs */

double h3hip_dit_block_gemm_flops(const h3hip_dit_config *c) {
    double d = c->hidden, inner = (double)c->heads * c->head_dim;
    double n = c->rows, f = c->ffn;
    if (c->family == H3HIP_FAMILY_WAN) {
        double t = c->text_rows;
        /* qkv, out, cross q, cross out, ffn up + down; cross k,v on text */
        return 2.0 * n * (3 * d * inner + inner * d + d * inner + inner * d +
                          2 * d * f) +
               2.0 * t * (2 * d * inner);
    }
    /* qkv (3 inner), out, fc1 (2 ffn), fc2 */
    return 2.0 * n * (3 * d * inner + inner * d + 2 * d * f + f * d);
}

double h3hip_dit_block_attention_flops(const h3hip_dit_config *c) {
    double inner = (double)c->heads * c->head_dim, n = c->rows;
    double flops = 4.0 * n * n * inner;
    if (c->family == H3HIP_FAMILY_WAN) flops += 4.0 * n * c->text_rows * inner;
    return flops;
}

double h3hip_dit_block_flops(const h3hip_dit_config *c) {
    return h3hip_dit_block_gemm_flops(c) + h3hip_dit_block_attention_flops(c);
}

/* --------------------------------------------------------- lifetime */

static h3_gpu_tensor *bf16(h3hip_dit *dit, size_t n, int *ok) {
    h3_gpu_tensor *t = h3_gpu_tensor_new_bf16(dit->gpu, n);
    if (!t) *ok = 0;
    return t;
}

h3hip_dit *h3hip_dit_create(h3_gpu *gpu, const h3hip_dit_config *config,
                            char *error, size_t error_size) {
    if (!gpu || !config || !config->hidden || !config->heads ||
        !config->head_dim || !config->ffn || !config->blocks ||
        !config->rows || !config->time_rows ||
        config->rope_half * 2 > config->head_dim ||
        (config->family == H3HIP_FAMILY_WAN && !config->text_rows)) {
        if (error && error_size)
            snprintf(error, error_size, "invalid DiT configuration");
        return NULL;
    }
    h3hip_dit *dit = (h3hip_dit *)calloc(1, sizeof(*dit));
    if (!dit) return NULL;
    dit->gpu = gpu;
    dit->config = *config;
    dit->modalities = config->family == H3HIP_FAMILY_WAN ? 1u : 3u;
    dit->blocks = (h3hip_block *)calloc(config->blocks, sizeof(h3hip_block));
    if (!dit->blocks) {
        free(dit);
        return NULL;
    }
    const size_t d = config->hidden;
    const size_t inner = (size_t)config->heads * config->head_dim;
    const size_t n = config->rows, f = config->ffn, hd = config->head_dim;
    const size_t t = config->text_rows;
    int ok = 1;
    for (uint32_t b = 0; b < config->blocks && ok; b++) {
        h3hip_block *w = &dit->blocks[b];
        w->norm1 = bf16(dit, d, &ok);
        w->norm2 = bf16(dit, d, &ok);
        w->q_norm = bf16(dit, hd, &ok);
        w->k_norm = bf16(dit, hd, &ok);
        w->qkv = bf16(dit, 3 * inner * d, &ok);
        w->out = bf16(dit, d * inner, &ok);
        w->modulation = bf16(dit, (size_t)config->time_rows *
                                      dit->modalities * SLOTS * d, &ok);
        if (is_wan(dit)) {
            w->qkv_bias = bf16(dit, 3 * inner, &ok);
            w->out_bias = bf16(dit, d, &ok);
            w->norm3 = bf16(dit, d, &ok);
            w->norm3_bias = bf16(dit, d, &ok);
            w->cq = bf16(dit, inner * d, &ok);
            w->cq_bias = bf16(dit, inner, &ok);
            w->ck = bf16(dit, inner * d, &ok);
            w->ck_bias = bf16(dit, inner, &ok);
            w->cv = bf16(dit, inner * d, &ok);
            w->cv_bias = bf16(dit, inner, &ok);
            w->cq_norm = bf16(dit, hd, &ok);
            w->ck_norm = bf16(dit, hd, &ok);
            w->co = bf16(dit, d * inner, &ok);
            w->co_bias = bf16(dit, d, &ok);
            w->ctx_k = bf16(dit, t * inner, &ok);
            w->ctx_v = bf16(dit, t * inner, &ok);
            w->fc1 = bf16(dit, f * d, &ok);
            w->fc1_bias = bf16(dit, f, &ok);
            w->fc2 = bf16(dit, d * f, &ok);
            w->fc2_bias = bf16(dit, d, &ok);
        } else {
            w->fc1 = bf16(dit, 2 * f * d, &ok);
            w->fc2 = bf16(dit, d * f, &ok);
        }
    }
    dit->hidden = bf16(dit, n * d, &ok);
    dit->row_map = ok ? h3_gpu_tensor_from_u32(gpu, NULL, n) : NULL;
    if (!dit->row_map) ok = 0;
    dit->rope_cos = bf16(dit, n * config->rope_half + 1, &ok);
    dit->rope_sin = bf16(dit, n * config->rope_half + 1, &ok);
    dit->mod_a = bf16(dit, n * d, &ok);
    dit->mod_b = bf16(dit, n * d, &ok);
    dit->qkv = bf16(dit, n * 3 * inner, &ok);
    if (!is_wan(dit)) {
        /* the Wan block attends straight from the fused QKV rows */
        dit->query = bf16(dit, n * inner, &ok);
        dit->key = bf16(dit, n * inner, &ok);
        dit->value = bf16(dit, n * inner, &ok);
    }
    dit->attn = bf16(dit, n * inner, &ok);
    dit->proj = bf16(dit, n * d, &ok);
    if (is_wan(dit)) {
        dit->context = bf16(dit, t * d, &ok);
        dit->cross_q = bf16(dit, n * inner, &ok);
        dit->cross_out = bf16(dit, n * inner, &ok);
        dit->ffn_act = bf16(dit, n * f, &ok);
    }
    if (ok && is_wan(dit) && t > 0) {
        const uint32_t problems = 2 * config->blocks;
        h3_gpu_tensor **outputs =
            (h3_gpu_tensor **)calloc(problems, sizeof(*outputs));
        const h3_gpu_tensor **weights =
            (const h3_gpu_tensor **)calloc(problems, sizeof(*weights));
        const h3_gpu_tensor **biases =
            (const h3_gpu_tensor **)calloc(problems, sizeof(*biases));
        if (outputs && weights && biases) {
            for (uint32_t b = 0; b < config->blocks; b++) {
                h3hip_block *w = &dit->blocks[b];
                outputs[2 * b] = w->ctx_k;
                outputs[2 * b + 1] = w->ctx_v;
                weights[2 * b] = w->ck;
                weights[2 * b + 1] = w->cv;
                biases[2 * b] = w->ck_bias;
                biases[2 * b + 1] = w->cv_bias;
            }
            dit->ctx_table = h3_hip_linear_group_table(
                gpu, outputs, weights, biases, problems, (uint32_t)t,
                (uint32_t)d, (uint32_t)inner);
        }
        if (dit->ctx_table && outputs && weights &&
            config->head_dim == 128) {
            for (uint32_t b = 0; b < config->blocks; b++) {
                outputs[b] = dit->blocks[b].ctx_k;
                weights[b] = dit->blocks[b].ck_norm;
            }
            dit->knorm_table = h3_hip_head_norm_group_table(
                gpu, outputs, weights, config->blocks, (uint32_t)t,
                config->heads, config->head_dim);
        }
        free(outputs);
        free(weights);
        free(biases);
        if (!dit->ctx_table ||
            (config->head_dim == 128 && !dit->knorm_table))
            ok = 0;
    }
    if (!ok) {
        if (error && error_size)
            snprintf(error, error_size, "cannot allocate DiT tensors: %s",
                     h3_gpu_error(gpu));
        h3hip_dit_free(dit);
        return NULL;
    }
    return dit;
}

static void sampler_free(h3hip_dit *dit);

void h3hip_dit_free(h3hip_dit *dit) {
    if (!dit) return;
    if (dit->blocks) {
        for (uint32_t b = 0; b < dit->config.blocks; b++) {
            h3_gpu_tensor **fields = (h3_gpu_tensor **)&dit->blocks[b];
            size_t count = sizeof(h3hip_block) / sizeof(h3_gpu_tensor *);
            for (size_t i = 0; i < count; i++) h3_gpu_tensor_free(fields[i]);
        }
        free(dit->blocks);
    }
    /* a forward that failed mid-way may have left a step map installed */
    if (dit->default_row_map) dit->row_map = dit->default_row_map;
    h3_gpu_tensor *shared[] = {
        dit->hidden, dit->row_map, dit->rope_cos, dit->rope_sin,
        dit->context, dit->mod_a, dit->mod_b, dit->qkv, dit->query,
        dit->key, dit->value, dit->attn, dit->proj, dit->cross_q,
        dit->cross_out, dit->ffn_act,
        dit->ctx_table, dit->knorm_table};
    for (size_t i = 0; i < sizeof(shared) / sizeof(*shared); i++)
        h3_gpu_tensor_free(shared[i]);
    sampler_free(dit);
    free(dit);
}

h3_gpu_tensor *h3hip_dit_tensor(h3hip_dit *dit, const char *name,
                                uint32_t block) {
    if (!dit || !name) return NULL;
    if (!strcmp(name, "hidden")) return dit->hidden;
    if (!strcmp(name, "row_map")) return dit->row_map;
    if (!strcmp(name, "rope_cos")) return dit->rope_cos;
    if (!strcmp(name, "rope_sin")) return dit->rope_sin;
    if (!strcmp(name, "context")) return dit->context;
    if (dit->sampler) {
        struct { const char *name; h3_gpu_tensor *tensor; } shared[] = {
            {"video_input", dit->video_input},
            {"audio_input", dit->audio_input},
            {"video_patch_w", dit->video_patch_w},
            {"video_patch_b", dit->video_patch_b},
            {"audio_patch_w", dit->audio_patch_w},
            {"audio_patch_b", dit->audio_patch_b},
            {"refined_text", dit->refined_text},
            {"final_norm", dit->final_norm},
            {"final_modulation", dit->final_mod},
            {"final_video_w", dit->final_video_w},
            {"final_video_b", dit->final_video_b},
            {"final_audio_w", dit->final_audio_w},
            {"final_audio_b", dit->final_audio_b},
            {"video_velocity", dit->video_velocity},
            {"audio_velocity", dit->audio_velocity},
            {"time_in_w", dit->time_in_w}, {"time_in_b", dit->time_in_b},
            {"time_out_w", dit->time_out_w},
            {"time_out_b", dit->time_out_b}};
        for (size_t i = 0; i < sizeof(shared) / sizeof(*shared); i++)
            if (!strcmp(name, shared[i].name)) return shared[i].tensor;
        if ((int)block < dit->steps) {
            if (!strcmp(name, "step_row_map")) return dit->step_maps[block];
            if (!strcmp(name, "final_video_map"))
                return dit->final_video_maps[block];
            if (!strcmp(name, "final_audio_map"))
                return dit->final_audio_maps[block];
        }
    }
    if (block >= dit->config.blocks) return NULL;
    h3hip_block *w = &dit->blocks[block];
    struct { const char *name; h3_gpu_tensor *tensor; } table[] = {
        {"norm1", w->norm1}, {"norm2", w->norm2}, {"norm3", w->norm3},
        {"norm3_bias", w->norm3_bias}, {"qkv", w->qkv},
        {"qkv_bias", w->qkv_bias}, {"q_norm", w->q_norm},
        {"k_norm", w->k_norm}, {"out", w->out}, {"out_bias", w->out_bias},
        {"fc1", w->fc1}, {"fc1_bias", w->fc1_bias}, {"fc2", w->fc2},
        {"fc2_bias", w->fc2_bias}, {"cq", w->cq}, {"cq_bias", w->cq_bias},
        {"ck", w->ck}, {"ck_bias", w->ck_bias}, {"cv", w->cv},
        {"cv_bias", w->cv_bias}, {"cq_norm", w->cq_norm},
        {"ck_norm", w->ck_norm}, {"co", w->co}, {"co_bias", w->co_bias},
        {"modulation", w->modulation}, {"ctx_k", w->ctx_k},
        {"ctx_v", w->ctx_v}};
    for (size_t i = 0; i < sizeof(table) / sizeof(*table); i++)
        if (!strcmp(name, table[i].name)) return table[i].tensor;
    return NULL;
}

/* ------------------------------------------------------------- init */

static int fill(h3hip_dit *dit, h3_gpu_tensor *t, uint64_t *seed, float mean,
                float std) {
    if (!t) return 1;
    return h3_gpu_fill_normal_bf16(dit->gpu, t, 0, h3_gpu_tensor_elements(t),
                                   (*seed)++, mean, std);
}

int h3hip_dit_init_random(h3hip_dit *dit, uint64_t seed, float weight_std,
                          float mod_std) {
    if (!dit) return 0;
    h3_gpu *gpu = dit->gpu;
    if (!dit_op(dit, h3_gpu_begin(gpu), "begin DiT init")) return 0;
    uint64_t s = seed * 1000003ull + 17;
    int ok = 1;
    for (uint32_t b = 0; b < dit->config.blocks && ok; b++) {
        h3hip_block *w = &dit->blocks[b];
        ok = fill(dit, w->norm1, &s, 1.0f, 0.02f) &&
             fill(dit, w->norm2, &s, 1.0f, 0.02f) &&
             fill(dit, w->norm3, &s, 1.0f, 0.02f) &&
             fill(dit, w->norm3_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->q_norm, &s, 1.0f, 0.02f) &&
             fill(dit, w->k_norm, &s, 1.0f, 0.02f) &&
             fill(dit, w->cq_norm, &s, 1.0f, 0.02f) &&
             fill(dit, w->ck_norm, &s, 1.0f, 0.02f) &&
             fill(dit, w->qkv, &s, 0.0f, weight_std) &&
             fill(dit, w->qkv_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->out, &s, 0.0f, weight_std) &&
             fill(dit, w->out_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->cq, &s, 0.0f, weight_std) &&
             fill(dit, w->cq_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->ck, &s, 0.0f, weight_std) &&
             fill(dit, w->ck_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->cv, &s, 0.0f, weight_std) &&
             fill(dit, w->cv_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->co, &s, 0.0f, weight_std) &&
             fill(dit, w->co_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->fc1, &s, 0.0f, weight_std) &&
             fill(dit, w->fc1_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->fc2, &s, 0.0f, weight_std) &&
             fill(dit, w->fc2_bias, &s, 0.0f, 0.02f) &&
             fill(dit, w->modulation, &s, 0.0f, mod_std);
    }
    ok = ok && fill(dit, dit->hidden, &s, 0.0f, 1.0f) &&
         fill(dit, dit->context, &s, 0.0f, 1.0f);
    if (!ok) {
        dit_fail(dit, "random init: %s", h3_gpu_error(gpu));
        (void)h3_gpu_submit(gpu);
        return 0;
    }
    if (!dit_op(dit, h3_gpu_submit(gpu), "submit DiT init")) return 0;
    /* default row map: every row on time row 0 with tag 0; default RoPE:
     * identity (cos 1, sin 0) */
    size_t n = dit->config.rows, half = dit->config.rope_half;
    uint32_t *map = (uint32_t *)calloc(n, sizeof(uint32_t));
    float *c = (float *)malloc((n * half + 1) * sizeof(float));
    float *z = (float *)calloc(n * half + 1, sizeof(float));
    if (!map || !c || !z) {
        free(map); free(c); free(z);
        return dit_fail(dit, "out of memory");
    }
    for (size_t i = 0; i < n * half; i++) c[i] = 1.0f;
    ok = h3hip_dit_set_row_map(dit, map) && h3hip_dit_set_rope(dit, c, z);
    free(map); free(c); free(z);
    return ok;
}

int h3hip_dit_set_row_map(h3hip_dit *dit, const uint32_t *row_map) {
    if (!dit || !row_map) return 0;
    uint32_t limit = dit->config.time_rows * dit->modalities;
    for (uint32_t r = 0; r < dit->config.rows; r++)
        if (row_map[r] >= limit)
            return dit_fail(dit, "row map entry %u = %u exceeds %u modulation "
                                 "rows", r, row_map[r], limit);
    /* the kernels index mod[row_map[r]] directly: range checked above */
    h3_gpu_tensor *fresh =
        h3_gpu_tensor_from_u32(dit->gpu, row_map, dit->config.rows);
    if (!fresh)
        return dit_fail(dit, "row map upload: %s", h3_gpu_error(dit->gpu));
    if (dit->default_row_map == dit->row_map) dit->default_row_map = fresh;
    h3_gpu_tensor_free(dit->row_map);
    dit->row_map = fresh;
    return 1;
}

int h3hip_dit_set_rope(h3hip_dit *dit, const float *cosines,
                       const float *sines) {
    if (!dit || !cosines || !sines) return 0;
    size_t count = (size_t)dit->config.rows * dit->config.rope_half;
    if (!count) return 1;
    h3_gpu *gpu = dit->gpu;
    h3_gpu_tensor *c32 = h3_gpu_tensor_from_f32(gpu, cosines, count);
    h3_gpu_tensor *s32 = h3_gpu_tensor_from_f32(gpu, sines, count);
    int ok = c32 && s32 && h3_gpu_begin(gpu) &&
             h3_gpu_cast_f32_to_bf16(gpu, dit->rope_cos, c32,
                                     (uint32_t)count) &&
             h3_gpu_cast_f32_to_bf16(gpu, dit->rope_sin, s32,
                                     (uint32_t)count) &&
             h3_gpu_submit(gpu);
    h3_gpu_tensor_free(c32);
    h3_gpu_tensor_free(s32);
    return ok ? 1 : dit_fail(dit, "RoPE upload: %s", h3_gpu_error(gpu));
}

/* ------------------------------------------------------------ blocks */

/* One H3 block, in the reference's order (h3_dit.c:2008-2180, BF16 path
 * with fused gate+adaLN and the fused cross-block adaLN). */
static int run_h3_block(h3hip_dit *dit, uint32_t index, int fuse_next) {
    const h3hip_dit_config *c = &dit->config;
    h3_gpu *gpu = dit->gpu;
    h3hip_block *w = &dit->blocks[index];
    const uint32_t rows = c->rows, hidden = c->hidden;
    const uint32_t inner = c->heads * c->head_dim;
    const float eps = c->epsilon;
    const uint32_t slots = SLOTS;
    if (!dit->attention_adaln_ready &&
        !DIT_OP(K_ROWS, h3_gpu_adaln_bf16(gpu, dit->mod_a, dit->hidden,
                                       w->norm1, w->modulation, dit->row_map,
                                       rows, hidden, slots, 0, 1, eps),
                "attention adaLN"))
        return 0;
    dit->attention_adaln_ready = 0;
    /* h3_gpu_grouped_qkv_linear_rope_bf16 (the reference engine's call,
     * h3_dit.c:2046-2050) is exactly these two calls on this backend;
     * issuing them separately keeps the op classes apart */
    if (!DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->qkv, dit->mod_a, w->qkv,
                                        NULL, rows, hidden, 3 * inner),
                "QKV projection") ||
        !DIT_OP(K_ROWS, h3_gpu_grouped_qkv_rope_bf16(
                         gpu, dit->query, dit->key, dit->value, dit->qkv,
                         w->q_norm, w->k_norm, dit->rope_cos, dit->rope_sin,
                         rows, c->heads, c->head_dim, c->rope_half, eps),
                "Q/K norm + RoPE") ||
        !DIT_OP(K_ATTN, h3_gpu_sdpa_bf16(gpu, dit->attn, dit->query, dit->key,
                                      dit->value, rows, c->heads, c->head_dim,
                                      1.0f / sqrtf((float)c->head_dim)),
                "joint attention") ||
        !DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->proj, dit->attn, w->out,
                                        NULL, rows, inner, hidden),
                "attention output") ||
        !DIT_OP(K_ROWS, h3_gpu_gate_adaln_bf16(
                         gpu, dit->hidden, dit->mod_b, dit->hidden, dit->proj,
                         w->norm2, w->modulation, w->modulation, dit->row_map,
                         rows, hidden, slots, 2, 3, 4, eps),
                "attention gate + MLP adaLN") ||
        !DIT_OP(K_ACT, h3_gpu_mlp_bf16(gpu, dit->proj, dit->mod_b, w->fc1,
                                     w->fc2, rows, hidden, c->ffn, hidden),
                "SwiGLU MLP"))
        return 0;
    if (fuse_next) {
        h3hip_block *next = &dit->blocks[index + 1];
        if (!DIT_OP(K_ROWS, h3_gpu_gate_adaln_bf16(
                             gpu, dit->hidden, dit->mod_a, dit->hidden,
                             dit->proj, next->norm1, w->modulation,
                             next->modulation, dit->row_map, rows, hidden,
                             slots, 5, 0, 1, eps),
                    "MLP gate + next attention adaLN"))
            return 0;
        dit->attention_adaln_ready = 1;
        return 1;
    }
    return DIT_OP(K_ROWS, h3_gpu_gate_bf16(gpu, dit->hidden, dit->hidden,
                                        dit->proj, w->modulation, dit->row_map,
                                        rows, hidden, slots, 5),
                  "MLP gate");
}

/* One Wan-style block: self-attention, cross-attention, GELU FFN. */
/* One Wan-shaped block.  Each residual update is fused with the norm that
 * reads it (h3_gpu_gate_layer_adaln_bf16); with fuse_next the FFN gate also
 * produces the next block's self-attention adaLN, which that block then
 * skips. */
static int run_wan_block(h3hip_dit *dit, uint32_t index, int fuse_next) {
    const h3hip_dit_config *c = &dit->config;
    h3_gpu *gpu = dit->gpu;
    h3hip_block *w = &dit->blocks[index];
    const uint32_t rows = c->rows, d = c->hidden, t = c->text_rows;
    const uint32_t inner = c->heads * c->head_dim;
    const float eps = c->epsilon;
    const float scale = 1.0f / sqrtf((float)c->head_dim);
    const int adaln_ready = dit->attention_adaln_ready;
    dit->attention_adaln_ready = 0;
    if (!adaln_ready &&
        !DIT_OP(K_ROWS, h3_gpu_layer_adaln_bf16(
                            gpu, dit->mod_a, dit->hidden, NULL, NULL,
                            w->modulation, dit->row_map, rows, d, SLOTS, 0, 1,
                            eps),
                "self-attention adaLN"))
        return 0;
    int ok =
           DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->qkv, dit->mod_a, w->qkv,
                                          w->qkv_bias, rows, d, 3 * inner),
                  "QKV projection") &&
           DIT_OP(K_ROWS, h3_hip_qk_norm_rope_inplace_bf16(
                           gpu, dit->qkv, w->q_norm, w->k_norm, dit->rope_cos,
                           dit->rope_sin, rows, c->heads, c->head_dim,
                           c->rope_half, eps, 1),
                  "K norm + RoPE (in place)") &&
           DIT_OP(K_ATTN, h3_hip_sdpa_qkv_norm_rope_bf16(
                           gpu, dit->attn, dit->qkv, w->q_norm,
                           dit->rope_cos, dit->rope_sin, rows, c->heads,
                           c->head_dim, c->rope_half, eps, scale),
                  "self-attention (Q norm + RoPE in the kernel)") &&
           DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->proj, dit->attn, w->out,
                                          w->out_bias, rows, inner, d),
                  "self-attention output") &&
           DIT_OP(K_ROWS, h3_gpu_gate_layer_adaln_bf16(
                           gpu, dit->hidden, dit->mod_b, dit->hidden,
                           dit->proj, w->modulation, w->norm3, w->norm3_bias,
                           NULL, dit->row_map, rows, d, SLOTS, 2, 0, 0, eps),
                  "self-attention gate + cross-attention norm") &&
           DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->cross_q, dit->mod_b,
                                          w->cq, w->cq_bias, rows, d, inner),
                  "cross Q projection") &&
           DIT_OP(K_ATTN, h3_hip_sdpa_cross_norm_bf16(
                           gpu, dit->cross_out, dit->cross_q, w->ctx_k,
                           w->ctx_v, w->cq_norm, rows, t, c->heads,
                           c->head_dim, eps, scale),
                  "cross-attention (Q norm in the kernel)") &&
           DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->proj, dit->cross_out,
                                          w->co, w->co_bias, rows, inner, d),
                  "cross-attention output") &&
           DIT_OP(K_ROWS, h3_gpu_gate_layer_adaln_bf16(
                           gpu, dit->hidden, dit->mod_a, dit->hidden,
                           dit->proj, NULL, NULL, NULL, w->modulation,
                           dit->row_map, rows, d, SLOTS, 0, 3, 4, eps),
                  "cross-attention residual + FFN adaLN") &&
           DIT_OP(K_ACT, h3_gpu_linear_gelu_bf16(gpu, dit->ffn_act,
                                               dit->mod_a, w->fc1,
                                               w->fc1_bias, rows, d, c->ffn),
                  "FFN up + GELU") &&
           DIT_OP(K_GEMM, h3_gpu_linear_bf16(gpu, dit->proj, dit->ffn_act,
                                          w->fc2, w->fc2_bias, rows, c->ffn,
                                          d),
                  "FFN down");
    if (!ok) return 0;
    if (!fuse_next)
        return DIT_OP(K_ROWS, h3_gpu_gate_bf16(gpu, dit->hidden, dit->hidden,
                                               dit->proj, w->modulation,
                                               dit->row_map, rows, d, SLOTS,
                                               5),
                      "FFN gate");
    if (!DIT_OP(K_ROWS, h3_gpu_gate_layer_adaln_bf16(
                            gpu, dit->hidden, dit->mod_a, dit->hidden,
                            dit->proj, w->modulation, NULL, NULL,
                            dit->blocks[index + 1].modulation, dit->row_map,
                            rows, d, SLOTS, 5, 0, 1, eps),
                "FFN gate + next self-attention adaLN"))
        return 0;
    dit->attention_adaln_ready = 1;
    return 1;
}

int h3hip_dit_run_blocks(h3hip_dit *dit, uint32_t first, uint32_t count) {
    return h3hip_dit_run_blocks_ops(dit, first, count, H3HIP_OPS_ALL);
}

double h3hip_dit_block_class_flops(const h3hip_dit_config *c,
                                   unsigned op_class) {
    double d = c->hidden, inner = (double)c->heads * c->head_dim;
    double n = c->rows, f = c->ffn, t = c->text_rows;
    const int wan = c->family == H3HIP_FAMILY_WAN;
    switch (op_class) {
    case H3HIP_OPS_GEMM:
        /* QKV, out (+ Wan: cross q, cross out, FFN down) */
        return wan ? 2.0 * n * (3 * d * inner + 3 * d * inner + f * d)
                   : 2.0 * n * (3 * d * inner + inner * d);
    case H3HIP_OPS_CONTEXT: return wan ? 2.0 * t * 2 * d * inner : 0.0;
    case H3HIP_OPS_GEMM_ACT:
        return wan ? 2.0 * n * d * f : 2.0 * n * (2 * f * d + f * d);
    case H3HIP_OPS_ATTENTION: return h3hip_dit_block_attention_flops(c);
    default: return 0.0;
    }
}

double h3hip_dit_block_plain_gemm_flops(const h3hip_dit_config *c) {
    return h3hip_dit_block_class_flops(c, H3HIP_OPS_GEMM);
}

uint32_t h3hip_dit_block_plain_gemm_launches(const h3hip_dit_config *c) {
    return c->family == H3HIP_FAMILY_WAN ? 5u : 2u;
}

int h3hip_dit_run_blocks_ops(h3hip_dit *dit, uint32_t first, uint32_t count,
                             unsigned op_mask) {
    if (!dit) return 0;
    dit->op_mask = op_mask;
    if (first > dit->config.blocks || count > dit->config.blocks - first)
        return dit_fail(dit, "block range [%u, %u) outside %u blocks", first,
                        first + count, dit->config.blocks);
    dit->attention_adaln_ready = 0;
    if (is_wan(dit) && count && dit->config.text_rows) {
        /* every block's cross-attention K and V of the text in one launch,
         * then every block's K norm in another */
        const h3hip_dit_config *c = &dit->config;
        const uint32_t t = c->text_rows, inner = c->heads * c->head_dim;
        if (!DIT_OP(K_CTX, h3_hip_linear_group_bf16(
                               dit->gpu, dit->ctx_table, 2 * first, 2 * count,
                               dit->context, t, c->hidden, inner),
                    "cross K/V projections"))
            return 0;
        if (dit->knorm_table) {
            if (!DIT_OP(K_ROWS, h3_hip_head_rms_norm_group_bf16(
                                    dit->gpu, dit->knorm_table, first, count,
                                    t, c->heads, c->head_dim, c->epsilon),
                        "cross K norms"))
                return 0;
        } else {
            for (uint32_t b = first; b < first + count; b++)
                if (!DIT_OP(K_ROWS, h3_gpu_head_rms_norm_bf16(
                                        dit->gpu, dit->blocks[b].ctx_k,
                                        dit->blocks[b].ck_norm, t, c->heads,
                                        c->head_dim, c->epsilon),
                            "cross K norm"))
                    return 0;
        }
    }
    for (uint32_t b = first; b < first + count; b++) {
        const int fuse_next = b + 1 < first + count;
        int ok = is_wan(dit) ? run_wan_block(dit, b, fuse_next)
                             : run_h3_block(dit, b, fuse_next);
        if (!ok) return 0;
    }
    return 1;
}

/* ----------------------------------------------------------- sampler */

static void free_maps(h3_gpu_tensor **maps, int count) {
    if (!maps) return;
    for (int i = 0; i < count; i++) h3_gpu_tensor_free(maps[i]);
    free(maps);
}

static void sampler_free(h3hip_dit *dit) {
    h3_gpu_tensor *owned[] = {
        dit->video_input, dit->audio_input, dit->video_patch_w,
        dit->video_patch_b, dit->audio_patch_w, dit->audio_patch_b,
        dit->refined_text, dit->final_norm, dit->final_mod,
        dit->final_video_w, dit->final_video_b, dit->final_audio_w,
        dit->final_audio_b, dit->video_velocity, dit->audio_velocity,
        dit->video_previous, dit->audio_previous, dit->video_inverse,
        dit->audio_inverse, dit->time_in_w, dit->time_in_b, dit->time_out_w,
        dit->time_out_b};
    for (size_t i = 0; i < sizeof(owned) / sizeof(*owned); i++)
        h3_gpu_tensor_free(owned[i]);
    free_maps(dit->step_maps, dit->steps);
    free_maps(dit->final_video_maps, dit->steps);
    free_maps(dit->final_audio_maps, dit->steps);
    free(dit->video_sigmas);
    free(dit->audio_sigmas);
    free(dit->segments);
}

/* The engine's own patch projection takes only the checkpoint shapes
 * (5376 outputs from 96 / 32 inputs); reduced-width test models use the
 * shape-generic variant of the same op. */
static int patch_offset(h3_gpu *gpu, h3_gpu_tensor *output,
                        size_t output_offset, const h3_gpu_tensor *input,
                        size_t input_offset, const h3_gpu_tensor *weight,
                        const h3_gpu_tensor *bias, uint32_t rows,
                        uint32_t input_dim, uint32_t output_dim) {
    if (output_dim == 5376 && (input_dim == 32 || input_dim == 96))
        return h3_gpu_patch_linear_bf16_offset(gpu, output, output_offset,
                                               input, input_offset, weight,
                                               bias, rows, input_dim,
                                               output_dim);
    return h3_hip_patch_linear_bf16_offset(gpu, output, output_offset, input,
                                           input_offset, weight, bias, rows,
                                           input_dim, output_dim);
}

static int is_video_kind(int kind) {
    return kind == H3HIP_SEG_COND || kind == H3HIP_SEG_REF_IMAGE ||
           kind == H3HIP_SEG_VIDEO;
}

static int is_audio_kind(int kind) {
    return kind == H3HIP_SEG_REF_AUDIO || kind == H3HIP_SEG_AUDIO;
}

void h3hip_dit_sampler_rows(const h3hip_dit *dit, uint32_t *video_rows,
                            uint32_t *audio_rows, uint32_t *video_targets,
                            uint32_t *audio_targets) {
    if (video_rows) *video_rows = dit ? dit->video_total : 0;
    if (audio_rows) *audio_rows = dit ? dit->audio_total : 0;
    if (video_targets) *video_targets = dit ? dit->video_targets : 0;
    if (audio_targets) *audio_targets = dit ? dit->audio_targets : 0;
}

int h3hip_dit_sampler_create(h3hip_dit *dit,
                             const h3hip_sampler_config *cfg) {
    if (!dit) return 0;
    if (dit->sampler) return dit_fail(dit, "sampler already created");
    const h3hip_dit_config *c = &dit->config;
    if (is_wan(dit))
        return dit_fail(dit, "the sampler drives the H3 block family");
    if (!cfg || !cfg->layout || cfg->steps < 1 || !cfg->video_sigmas ||
        !cfg->audio_sigmas || cfg->reuse_interval < 1 ||
        cfg->reuse_interval > 32 || !cfg->video_patch ||
        !cfg->audio_channels)
        return dit_fail(dit, "invalid sampler configuration");
    const h3hip_layout *layout = cfg->layout;
    if (layout->seq_len != c->rows)
        return dit_fail(dit, "layout has %zu rows, the DiT %u",
                        layout->seq_len, c->rows);
    /* time rows of this schedule (reference h3_dit_schedule.c:78-161) */
    const int steps = cfg->steps;
    uint32_t *video_time = (uint32_t *)calloc(steps, sizeof(uint32_t));
    uint32_t *audio_time = (uint32_t *)calloc(steps, sizeof(uint32_t));
    uint32_t *visual_time = (uint32_t *)calloc(steps, sizeof(uint32_t));
    uint32_t *audio_cond_time = (uint32_t *)calloc(steps, sizeof(uint32_t));
    if (!video_time || !audio_time || !visual_time || !audio_cond_time) {
        free(video_time); free(audio_time); free(visual_time);
        free(audio_cond_time);
        return dit_fail(dit, "out of memory");
    }
    int visual_condition = 0, audio_condition = 0;
    uint32_t video_total = 0, audio_total = 0;
    uint32_t video_targets = 0, audio_targets = 0;
    uint32_t video_conditions = 0, audio_conditions = 0;
    uint32_t video_start = 0, audio_start = 0, text_rows = 0;
    int video_segments = 0, audio_segments = 0, ok = 1;
    for (size_t i = 0; i < layout->segment_count && ok; i++) {
        const h3hip_segment *seg = &layout->segments[i];
        uint32_t n = (uint32_t)(seg->stop - seg->start);
        if (seg->kind == H3HIP_SEG_TEXT) {
            text_rows += n;
        } else if (is_video_kind(seg->kind)) {
            if (seg->kind == H3HIP_SEG_VIDEO) {
                video_segments++;
                video_targets = n;
                video_start = (uint32_t)seg->start;
                video_conditions = video_total;
            } else {
                visual_condition = 1;
                if (video_segments) ok = 0; /* conditions precede targets */
            }
            video_total += n;
        } else if (is_audio_kind(seg->kind)) {
            if (seg->kind == H3HIP_SEG_AUDIO) {
                audio_segments++;
                audio_targets = n;
                audio_start = (uint32_t)seg->start;
                audio_conditions = audio_total;
            } else {
                audio_condition = 1;
                if (audio_segments) ok = 0;
            }
            audio_total += n;
        } else {
            ok = 0;
        }
    }
    uint32_t time_rows = ok ? h3hip_time_rows(
        steps, cfg->video_sigmas, cfg->audio_sigmas, visual_condition,
        audio_condition, video_time, audio_time, visual_time,
        audio_cond_time, NULL) : 0;
    if (!ok || video_segments != 1 || audio_segments != 1 || !time_rows ||
        time_rows != c->time_rows) {
        free(video_time); free(audio_time); free(visual_time);
        free(audio_cond_time);
        if (!ok || video_segments != 1 || audio_segments != 1)
            return dit_fail(dit, "the layout needs one video and one audio "
                                 "target segment after their conditions");
        return dit_fail(dit, "the schedule has %u time rows, the DiT "
                             "modulation %u", time_rows, c->time_rows);
    }
    dit->steps = steps;
    dit->reuse_interval = cfg->reuse_interval;
    dit->video_patch = cfg->video_patch;
    dit->audio_channels = cfg->audio_channels;
    dit->video_total = video_total;
    dit->audio_total = audio_total;
    dit->video_conditions = video_conditions;
    dit->audio_conditions = audio_conditions;
    dit->video_targets = video_targets;
    dit->audio_targets = audio_targets;
    dit->video_target_start = video_start;
    dit->audio_target_start = audio_start;
    dit->sampler = 1;
    dit->video_sigmas = (float *)malloc((steps + 1) * sizeof(float));
    dit->audio_sigmas = (float *)malloc((steps + 1) * sizeof(float));
    dit->segments = (h3hip_segment *)malloc(
        (layout->segment_count ? layout->segment_count : 1) *
        sizeof(h3hip_segment));
    dit->step_maps = (h3_gpu_tensor **)calloc(steps, sizeof(void *));
    dit->final_video_maps = (h3_gpu_tensor **)calloc(steps, sizeof(void *));
    dit->final_audio_maps = (h3_gpu_tensor **)calloc(steps, sizeof(void *));
    uint32_t *rows = (uint32_t *)malloc((size_t)c->rows * sizeof(uint32_t));
    uint32_t *video = (uint32_t *)malloc(
        (video_targets ? video_targets : 1) * sizeof(uint32_t));
    uint32_t *audio = (uint32_t *)malloc(
        (audio_targets ? audio_targets : 1) * sizeof(uint32_t));
    ok = dit->video_sigmas && dit->audio_sigmas && dit->segments &&
         dit->step_maps && dit->final_video_maps && dit->final_audio_maps &&
         rows && video && audio;
    if (ok) {
        memcpy(dit->video_sigmas, cfg->video_sigmas,
               (steps + 1) * sizeof(float));
        memcpy(dit->audio_sigmas, cfg->audio_sigmas,
               (steps + 1) * sizeof(float));
        memcpy(dit->segments, layout->segments,
               layout->segment_count * sizeof(h3hip_segment));
        dit->segment_count = layout->segment_count;
    }
    /* per-step maps (reference prepare_maps, h3_dit.c:1134-1200) */
    for (int step = 0; step < steps && ok; step++) {
        ok = h3hip_row_map(layout, video_time[step], audio_time[step],
                           visual_time[step], audio_cond_time[step], NULL,
                           text_rows, rows, c->rows);
        if (!ok) {
            dit_fail(dit, "cannot build the row map of step %d", step);
            break;
        }
        for (uint32_t r = 0; r < video_targets; r++) video[r] = video_time[step];
        for (uint32_t r = 0; r < audio_targets; r++) audio[r] = audio_time[step];
        dit->step_maps[step] = h3_gpu_tensor_from_u32(dit->gpu, rows, c->rows);
        dit->final_video_maps[step] =
            h3_gpu_tensor_from_u32(dit->gpu, video, video_targets);
        dit->final_audio_maps[step] =
            h3_gpu_tensor_from_u32(dit->gpu, audio, audio_targets);
        ok = dit->step_maps[step] && dit->final_video_maps[step] &&
             dit->final_audio_maps[step];
        if (!ok) dit_fail(dit, "row map upload: %s", h3_gpu_error(dit->gpu));
    }
    free(rows); free(video); free(audio);
    free(video_time); free(audio_time); free(visual_time);
    free(audio_cond_time);
    if (!ok) {
        if (!dit->error[0]) dit_fail(dit, "out of memory");
        sampler_free(dit);
        dit->sampler = 0;
        return 0;
    }
    const size_t d = c->hidden, vp = cfg->video_patch;
    const size_t ac = cfg->audio_channels;
    h3_gpu *gpu = dit->gpu;
    int alloc = 1;
#define F32T(n) (h3_gpu_tensor_new_f32(gpu, (n)))
    dit->video_input = F32T((size_t)video_total * vp + 1);
    dit->audio_input = F32T((size_t)audio_total * ac + 1);
    dit->video_patch_w = F32T(d * vp);
    dit->video_patch_b = F32T(d);
    dit->audio_patch_w = F32T(d * ac);
    dit->audio_patch_b = F32T(d);
    dit->video_inverse = F32T((size_t)video_targets + 1);
    dit->audio_inverse = F32T((size_t)audio_targets + 1);
#undef F32T
    dit->refined_text = bf16(dit, (size_t)text_rows * d + 1, &alloc);
    dit->final_norm = bf16(dit, d, &alloc);
    dit->final_mod = bf16(dit, (size_t)time_rows * 2 * d, &alloc);
    dit->final_video_w = bf16(dit, vp * d, &alloc);
    dit->final_video_b = bf16(dit, vp, &alloc);
    dit->final_audio_w = bf16(dit, ac * d, &alloc);
    dit->final_audio_b = bf16(dit, ac, &alloc);
    dit->video_velocity = bf16(dit, (size_t)video_targets * vp + 1, &alloc);
    dit->audio_velocity = bf16(dit, (size_t)audio_targets * ac + 1, &alloc);
    dit->video_previous = bf16(dit, (size_t)video_targets * vp + 1, &alloc);
    dit->audio_previous = bf16(dit, (size_t)audio_targets * ac + 1, &alloc);
    alloc = alloc && dit->video_input && dit->audio_input &&
            dit->video_patch_w && dit->video_patch_b && dit->audio_patch_w &&
            dit->audio_patch_b && dit->video_inverse && dit->audio_inverse;
    if (!alloc) {
        dit_fail(dit, "cannot allocate sampler tensors: %s",
                 h3_gpu_error(gpu));
        sampler_free(dit);
        dit->sampler = 0;
        return 0;
    }
    dit->default_row_map = dit->row_map;
    return 1;
}

static int fill_f32(h3hip_dit *dit, h3_gpu_tensor *t, uint64_t *seed,
                    float mean, float std) {
    return h3_gpu_fill_normal_f32(dit->gpu, t, 0, h3_gpu_tensor_elements(t),
                                  (*seed)++, mean, std);
}

int h3hip_dit_sampler_init_random(h3hip_dit *dit, uint64_t seed,
                                  float weight_std, float mod_std) {
    if (!dit || !dit->sampler) return dit ? dit_fail(dit, "no sampler") : 0;
    h3_gpu *gpu = dit->gpu;
    uint64_t s = seed * 7919ull + 101;
    if (!dit_op(dit, h3_gpu_begin(gpu), "begin sampler init")) return 0;
    int ok = fill_f32(dit, dit->video_patch_w, &s, 0.0f, weight_std) &&
             fill_f32(dit, dit->video_patch_b, &s, 0.0f, 0.02f) &&
             fill_f32(dit, dit->audio_patch_w, &s, 0.0f, weight_std) &&
             fill_f32(dit, dit->audio_patch_b, &s, 0.0f, 0.02f) &&
             fill(dit, dit->refined_text, &s, 0.0f, 1.0f) &&
             fill(dit, dit->final_norm, &s, 1.0f, 0.02f) &&
             fill(dit, dit->final_mod, &s, 0.0f, mod_std) &&
             fill(dit, dit->final_video_w, &s, 0.0f, weight_std) &&
             fill(dit, dit->final_video_b, &s, 0.0f, 0.02f) &&
             fill(dit, dit->final_audio_w, &s, 0.0f, weight_std) &&
             fill(dit, dit->final_audio_b, &s, 0.0f, 0.02f) &&
             fill_f32(dit, dit->video_input, &s, 0.0f, 1.0f) &&
             fill_f32(dit, dit->audio_input, &s, 0.0f, 1.0f);
    if (!ok) {
        dit_fail(dit, "sampler init: %s", h3_gpu_error(gpu));
        (void)h3_gpu_submit(gpu);
        return 0;
    }
    return dit_op(dit, h3_gpu_submit(gpu), "submit sampler init");
}

int h3hip_dit_sampler_write_latents(h3hip_dit *dit, const float *video,
                                    const float *audio) {
    if (!dit || !dit->sampler) return dit ? dit_fail(dit, "no sampler") : 0;
    int ok = (!video || h3_gpu_tensor_write_f32_range(
                            dit->video_input, 0, video,
                            (size_t)dit->video_total * dit->video_patch)) &&
             (!audio || h3_gpu_tensor_write_f32_range(
                            dit->audio_input, 0, audio,
                            (size_t)dit->audio_total * dit->audio_channels));
    return ok ? 1 : dit_fail(dit, "latent upload: %s", h3_gpu_error(dit->gpu));
}

int h3hip_dit_sampler_read_latents(h3hip_dit *dit, float *video,
                                   float *audio) {
    if (!dit || !dit->sampler) return dit ? dit_fail(dit, "no sampler") : 0;
    int ok = (!video || h3_gpu_tensor_read_f32_range(
                            dit->video_input, 0, video,
                            (size_t)dit->video_total * dit->video_patch)) &&
             (!audio || h3_gpu_tensor_read_f32_range(
                            dit->audio_input, 0, audio,
                            (size_t)dit->audio_total * dit->audio_channels));
    return ok ? 1 : dit_fail(dit, "latent readback: %s",
                             h3_gpu_error(dit->gpu));
}

/* Pack, blocks, final heads (reference encode_forward, h3_dit.c:2182-2528,
 * fused patch/pack and fused final head path). */
int h3hip_dit_forward_step(h3hip_dit *dit, int step) {
    if (!dit || !dit->sampler) return dit ? dit_fail(dit, "no sampler") : 0;
    if (step < 0 || step >= dit->steps)
        return dit_fail(dit, "step %d outside %d steps", step, dit->steps);
    const h3hip_dit_config *c = &dit->config;
    h3_gpu *gpu = dit->gpu;
    const size_t d = c->hidden;
    size_t video_offset = 0, audio_offset = 0, text_offset = 0;
    dit->op_mask = H3HIP_OPS_ALL;
    for (size_t i = 0; i < dit->segment_count; i++) {
        const h3hip_segment *seg = &dit->segments[i];
        const uint32_t n = (uint32_t)(seg->stop - seg->start);
        const size_t destination = seg->start * d;
        int ok;
        if (seg->kind == H3HIP_SEG_TEXT) {
            ok = dit_op(dit, h3_gpu_copy_bf16(gpu, dit->hidden, destination,
                                              dit->refined_text,
                                              text_offset * d, (size_t)n * d),
                        "pack refined text");
            text_offset += n;
        } else if (is_video_kind(seg->kind)) {
            ok = dit_op(dit, patch_offset(
                                 gpu, dit->hidden, destination,
                                 dit->video_input,
                                 video_offset * dit->video_patch,
                                 dit->video_patch_w, dit->video_patch_b, n,
                                 dit->video_patch, c->hidden),
                        "project packed video source");
            video_offset += n;
        } else {
            ok = dit_op(dit, patch_offset(
                                 gpu, dit->hidden, destination,
                                 dit->audio_input,
                                 audio_offset * dit->audio_channels,
                                 dit->audio_patch_w, dit->audio_patch_b, n,
                                 dit->audio_channels, c->hidden),
                        "project packed audio source");
            audio_offset += n;
        }
        if (!ok) return 0;
    }
    dit->row_map = dit->step_maps[step];
    int ok = h3hip_dit_run_blocks(dit, 0, c->blocks);
    dit->row_map = dit->default_row_map;
    if (!ok) return 0;
    return dit_op(dit, h3_gpu_adaln_linear_bf16(
                           gpu, dit->audio_velocity, dit->audio_inverse,
                           dit->hidden, (size_t)dit->audio_target_start * d,
                           dit->final_norm, dit->final_mod,
                           dit->final_audio_maps[step], dit->final_audio_w,
                           dit->final_audio_b, dit->audio_targets, c->hidden,
                           dit->audio_channels, 2, 0, 1, c->epsilon),
                  "final audio adaLN + head") &&
           dit_op(dit, h3_gpu_adaln_linear_bf16(
                           gpu, dit->video_velocity, dit->video_inverse,
                           dit->hidden, (size_t)dit->video_target_start * d,
                           dit->final_norm, dit->final_mod,
                           dit->final_video_maps[step], dit->final_video_w,
                           dit->final_video_b, dit->video_targets, c->hidden,
                           dit->video_patch, 2, 0, 1, c->epsilon),
                  "final video adaLN + head");
}

/* Euler loop with velocity reuse (reference denoise_euler_gpu,
 * h3_dit.c:2745-2917, the bounded one-evaluation command window). */
int h3hip_dit_denoise(h3hip_dit *dit) {
    if (!dit || !dit->sampler) return dit ? dit_fail(dit, "no sampler") : 0;
    h3_gpu *gpu = dit->gpu;
    const int steps = dit->steps;
    uint8_t *selected = (uint8_t *)calloc(steps, 1);
    if (!selected) return dit_fail(dit, "out of memory");
    if (h3hip_reuse_schedule(steps, dit->reuse_interval, selected, steps) < 0) {
        free(selected);
        return dit_fail(dit, "invalid reuse schedule");
    }
    const uint32_t video_count = dit->video_targets * dit->video_patch;
    const uint32_t audio_count = dit->audio_targets * dit->audio_channels;
    const size_t video_offset = (size_t)dit->video_conditions * dit->video_patch;
    const size_t audio_offset =
        (size_t)dit->audio_conditions * dit->audio_channels;
    int last = -1, previous = -1, evaluations = 0, ok = 1, open = 0;
    for (int step = 0; step < steps && ok; step++) {
        if (!open) {
            ok = dit_op(dit, h3_gpu_begin(gpu), "begin Euler chain");
            open = ok;
            if (!ok) break;
        }
        const int evaluate = selected[step];
        if (evaluate) {
            if (last >= 0 && dit->reuse_interval > 1) {
                ok = dit_op(dit, h3_gpu_copy_bf16(gpu, dit->video_previous, 0,
                                                  dit->video_velocity, 0,
                                                  video_count),
                            "cache previous video velocity") &&
                     dit_op(dit, h3_gpu_copy_bf16(gpu, dit->audio_previous, 0,
                                                  dit->audio_velocity, 0,
                                                  audio_count),
                            "cache previous audio velocity");
                if (ok) previous = last;
            }
            if (ok) ok = h3hip_dit_forward_step(dit, step);
            if (ok) {
                last = step;
                evaluations++;
            }
        }
        if (!ok) break;
        const int have = previous >= 0;
        const float video_ratio = evaluate ? 0.0f : h3hip_extrapolation_ratio(
            dit->video_sigmas[step], dit->video_sigmas[last],
            have ? dit->video_sigmas[previous] : 0.0f, have);
        const float audio_ratio = evaluate ? 0.0f : h3hip_extrapolation_ratio(
            dit->audio_sigmas[step], dit->audio_sigmas[last],
            have ? dit->audio_sigmas[previous] : 0.0f, have);
        ok = dit_op(dit, h3_gpu_euler_bf16(
                         gpu, dit->video_input, video_offset,
                         dit->video_velocity,
                         have ? dit->video_previous : dit->video_velocity,
                         video_count,
                         dit->video_sigmas[step] - dit->video_sigmas[step + 1],
                         video_ratio),
                    "video Euler step") &&
             dit_op(dit, h3_gpu_euler_bf16(
                         gpu, dit->audio_input, audio_offset,
                         dit->audio_velocity,
                         have ? dit->audio_previous : dit->audio_velocity,
                         audio_count,
                         dit->audio_sigmas[step] - dit->audio_sigmas[step + 1],
                         audio_ratio),
                    "audio Euler step");
        if (ok && evaluate) {
            ok = dit_op(dit, h3_gpu_submit(gpu), "submit Euler window");
            open = 0;
        }
    }
    if (open) {
        if (ok) ok = dit_op(dit, h3_gpu_submit(gpu), "submit Euler denoise");
        else (void)h3_gpu_submit(gpu);
    }
    free(selected);
    return ok ? evaluations : 0;
}

/* ------------------------------------------------- modulation schedule */

enum { TIME_INPUT = 256 };

int h3hip_dit_schedule_precompute(h3hip_dit *dit, uint64_t seed,
                                  float weight_std) {
    if (!dit || !dit->sampler)
        return dit ? dit_fail(dit, "the schedule needs the sampler") : 0;
    const h3hip_dit_config *c = &dit->config;
    const uint32_t d = c->hidden, th = d, td = d / 2;
    if (d % 2 || td % 64)
        return dit_fail(dit, "hidden %u has no 64-aligned half", d);
    /* time rows and their t = 1 - sigma (h3_dit_schedule.c:78-161) */
    const int steps = dit->steps;
    int visual = 0, audio_cond = 0;
    for (size_t i = 0; i < dit->segment_count; i++) {
        const int kind = dit->segments[i].kind;
        if (kind == H3HIP_SEG_COND || kind == H3HIP_SEG_REF_IMAGE) visual = 1;
        if (kind == H3HIP_SEG_REF_AUDIO) audio_cond = 1;
    }
    uint32_t *rows4 = (uint32_t *)calloc(4 * (size_t)steps, sizeof(uint32_t));
    float *times = (float *)calloc(c->time_rows, sizeof(float));
    float *features =
        (float *)malloc((size_t)c->time_rows * TIME_INPUT * sizeof(float));
    if (!rows4 || !times || !features) {
        free(rows4); free(times); free(features);
        return dit_fail(dit, "out of memory");
    }
    uint32_t n = h3hip_time_rows(steps, dit->video_sigmas, dit->audio_sigmas,
                                 visual, audio_cond, rows4, rows4 + steps,
                                 rows4 + 2 * steps, rows4 + 3 * steps, times);
    if (n != c->time_rows) {
        free(rows4); free(times); free(features);
        return dit_fail(dit, "schedule has %u time rows, the DiT %u", n,
                        c->time_rows);
    }
    h3hip_timestep_features(times, n, features);
    free(rows4);
    free(times);

    h3_gpu *gpu = dit->gpu;
    if (!dit->time_in_w) {
        dit->time_in_w = h3_gpu_tensor_new_f32(gpu, (size_t)th * TIME_INPUT);
        dit->time_in_b = h3_gpu_tensor_new_f32(gpu, th);
        dit->time_out_w = h3_gpu_tensor_new_f32(gpu, (size_t)td * th);
        dit->time_out_b = h3_gpu_tensor_new_f32(gpu, td);
    }
    const size_t block_out = (size_t)dit->modalities * SLOTS * d;
    h3_gpu_tensor *feat =
        h3_gpu_tensor_from_f32(gpu, features, (size_t)n * TIME_INPUT);
    free(features);
    h3_gpu_tensor *h1 = h3_gpu_tensor_new_f32(gpu, (size_t)n * th);
    h3_gpu_tensor *a1 = h3_gpu_tensor_new_f32(gpu, (size_t)n * th);
    h3_gpu_tensor *o = h3_gpu_tensor_new_f32(gpu, (size_t)n * td);
    h3_gpu_tensor *ob = h3_gpu_tensor_new_bf16(gpu, (size_t)n * td);
    h3_gpu_tensor *time = h3_gpu_tensor_new_bf16(gpu, (size_t)n * td);
    h3_gpu_tensor *pw = h3_gpu_tensor_new_bf16(gpu, block_out * td);
    h3_gpu_tensor *pb = h3_gpu_tensor_new_bf16(gpu, block_out);
    h3_gpu_tensor *temps[] = {feat, h1, a1, o, ob, time, pw, pb};
    int ok = dit->time_in_w && dit->time_in_b && dit->time_out_w &&
             dit->time_out_b;
    for (size_t i = 0; i < sizeof(temps) / sizeof(*temps); i++)
        ok = ok && temps[i];
    if (!ok) {
        for (size_t i = 0; i < sizeof(temps) / sizeof(*temps); i++)
            h3_gpu_tensor_free(temps[i]);
        return dit_fail(dit, "cannot allocate schedule tensors: %s",
                        h3_gpu_error(gpu));
    }
#define SOP(call, what) (ok = ok && dit_op(dit, (call), (what)))
    ok = dit_op(dit, h3_gpu_begin(gpu), "begin schedule precompute");
    SOP(h3_gpu_fill_normal_f32(gpu, dit->time_in_w, 0, (size_t)th * TIME_INPUT,
                               seed, 0.0f, weight_std), "time MLP init");
    SOP(h3_gpu_fill_normal_f32(gpu, dit->time_in_b, 0, th, seed + 1, 0.0f,
                               0.02f), "time MLP init");
    SOP(h3_gpu_fill_normal_f32(gpu, dit->time_out_w, 0, (size_t)td * th,
                               seed + 2, 0.0f, weight_std), "time MLP init");
    SOP(h3_gpu_fill_normal_f32(gpu, dit->time_out_b, 0, td, seed + 3, 0.0f,
                               0.02f), "time MLP init");
    /* timestep embedding (h3_dit_schedule.c:163-234) */
    SOP(h3_gpu_linear_f32(gpu, h1, feat, dit->time_in_w, dit->time_in_b, n,
                          TIME_INPUT, th), "timestep input projection");
    SOP(h3_gpu_silu_f32(gpu, a1, h1, n * th), "timestep SiLU");
    SOP(h3_gpu_linear_f32(gpu, o, a1, dit->time_out_w, dit->time_out_b, n, th,
                          td), "timestep output projection");
    SOP(h3_gpu_cast_f32_to_bf16(gpu, ob, o, n * td), "timestep BF16 cast");
    SOP(h3_gpu_silu_bf16(gpu, time, ob, n * td), "timestep adaLN SiLU");
    /* per-block adaLN projections (h3_dit_schedule.c:260-301) */
    for (uint32_t b = 0; b < c->blocks && ok; b++) {
        SOP(h3_gpu_fill_normal_bf16(gpu, pw, 0, block_out * td,
                                    seed + 16 + 2ull * b, 0.0f, weight_std),
            "adaLN projection init");
        SOP(h3_gpu_fill_normal_bf16(gpu, pb, 0, block_out,
                                    seed + 17 + 2ull * b, 0.0f, 0.02f),
            "adaLN projection init");
        SOP(h3_gpu_linear_bf16(gpu, dit->blocks[b].modulation, time, pw, pb,
                               n, td, (uint32_t)block_out),
            "adaLN block projection");
    }
    /* final adaLN projection (h3_dit_schedule.c:303-330) */
    SOP(h3_gpu_fill_normal_bf16(gpu, pw, 0, (size_t)2 * d * td, seed + 8, 0.0f,
                                weight_std), "final adaLN init");
    SOP(h3_gpu_fill_normal_bf16(gpu, pb, 0, (size_t)2 * d, seed + 9, 0.0f,
                                0.02f), "final adaLN init");
    SOP(h3_gpu_linear_bf16(gpu, dit->final_mod, time, pw, pb, n, td, 2 * d),
        "final adaLN projection");
#undef SOP
    if (ok) ok = dit_op(dit, h3_gpu_submit(gpu), "submit schedule precompute");
    else (void)h3_gpu_submit(gpu);
    for (size_t i = 0; i < sizeof(temps) / sizeof(*temps); i++)
        h3_gpu_tensor_free(temps[i]);
    return ok;
}

/* ------------------------------------------------- sparse attention */

long h3hip_dit_set_sparse_window(h3hip_dit *dit, const h3hip_layout *layout,
                                 unsigned radius_t, unsigned radius_h,
                                 unsigned radius_w, unsigned global_stride,
                                 int clear) {
    if (!dit) return -1;
    if (clear)
        return h3_gpu_sdpa_set_sparse(dit->gpu, NULL, 0, NULL, 0, 0)
                   ? 0 : (dit_fail(dit, "clear mask: %s",
                                   h3_gpu_error(dit->gpu)), -1);
    if (!layout || layout->seq_len != dit->config.rows) {
        dit_fail(dit, "the mask's layout must match the DiT rows");
        return -1;
    }
    const size_t qblocks = (layout->seq_len + 127) / 128;
    uint32_t *ptr = (uint32_t *)malloc((qblocks + 1) * sizeof(uint32_t));
    if (!ptr) return (dit_fail(dit, "out of memory"), -1);
    long total = h3hip_sparse_mask(layout, radius_t, radius_h, radius_w,
                                   global_stride, ptr, NULL, 0);
    if (total < 0) {
        free(ptr);
        return 0; /* no single target video segment: stays dense */
    }
    uint32_t *idx = (uint32_t *)malloc((total ? total : 1) * sizeof(uint32_t));
    if (!idx) {
        free(ptr);
        return (dit_fail(dit, "out of memory"), -1);
    }
    (void)h3hip_sparse_mask(layout, radius_t, radius_h, radius_w,
                            global_stride, ptr, idx, (size_t)total);
    int ok = total > 0 &&
             h3_gpu_sdpa_set_sparse(dit->gpu, ptr, qblocks + 1, idx,
                                    (size_t)total, dit->config.rows);
    free(ptr);
    free(idx);
    if (!ok) {
        dit_fail(dit, "sparse mask: %s", h3_gpu_error(dit->gpu));
        return -1;
    }
    return total;
}

/* ----------------------------------------------------- text refiner */

struct h3hip_refiner {
    h3_gpu *gpu;
    uint32_t hidden, heads, head_dim, ffn, text_dim;
    h3_gpu_tensor *condition_w, *condition_b, *final_norm;
    struct {
        h3_gpu_tensor *norm1, *qkv, *q_norm, *k_norm, *out, *norm2, *fc1,
            *fc2;
    } block[2];
    char error[512];
};

static int refiner_fail(h3hip_refiner *r, const char *what) {
    snprintf(r->error, sizeof(r->error), "%s: %s", what,
             h3_gpu_error(r->gpu));
    return 0;
}

h3hip_refiner *h3hip_refiner_create(h3_gpu *gpu, uint32_t hidden,
                                    uint32_t heads, uint32_t head_dim,
                                    uint32_t ffn, uint32_t text_dim,
                                    char *error, size_t error_size) {
    if (!gpu || !hidden || !heads || !head_dim || !ffn || !text_dim) {
        if (error && error_size)
            snprintf(error, error_size, "invalid refiner configuration");
        return NULL;
    }
    h3hip_refiner *r = (h3hip_refiner *)calloc(1, sizeof(*r));
    if (!r) return NULL;
    r->gpu = gpu;
    r->hidden = hidden;
    r->heads = heads;
    r->head_dim = head_dim;
    r->ffn = ffn;
    r->text_dim = text_dim;
    const size_t d = hidden, inner = (size_t)heads * head_dim, f = ffn;
    int ok = 1;
#define NEW(n) (ok && (t = h3_gpu_tensor_new_bf16(gpu, (n))) ? t : (ok = 0, NULL))
    h3_gpu_tensor *t = NULL;
    r->condition_w = NEW(d * text_dim);
    r->condition_b = NEW(d);
    r->final_norm = NEW(d);
    for (int b = 0; b < 2; b++) {
        r->block[b].norm1 = NEW(d);
        r->block[b].qkv = NEW(3 * inner * d);
        r->block[b].q_norm = NEW(head_dim);
        r->block[b].k_norm = NEW(head_dim);
        r->block[b].out = NEW(d * inner);
        r->block[b].norm2 = NEW(d);
        r->block[b].fc1 = NEW(2 * f * d);
        r->block[b].fc2 = NEW(d * f);
    }
#undef NEW
    if (!ok) {
        if (error && error_size)
            snprintf(error, error_size, "cannot allocate refiner weights: %s",
                     h3_gpu_error(gpu));
        h3hip_refiner_free(r);
        return NULL;
    }
    return r;
}

void h3hip_refiner_free(h3hip_refiner *r) {
    if (!r) return;
    h3_gpu_tensor_free(r->condition_w);
    h3_gpu_tensor_free(r->condition_b);
    h3_gpu_tensor_free(r->final_norm);
    for (int b = 0; b < 2; b++) {
        h3_gpu_tensor **fields = (h3_gpu_tensor **)&r->block[b];
        for (size_t i = 0; i < sizeof(r->block[b]) / sizeof(*fields); i++)
            h3_gpu_tensor_free(fields[i]);
    }
    free(r);
}

const char *h3hip_refiner_error(const h3hip_refiner *r) {
    return r ? r->error : "no refiner";
}

h3_gpu_tensor *h3hip_refiner_tensor(h3hip_refiner *r, const char *name,
                                    uint32_t block) {
    if (!r || !name) return NULL;
    if (!strcmp(name, "condition_w")) return r->condition_w;
    if (!strcmp(name, "condition_b")) return r->condition_b;
    if (!strcmp(name, "final_norm")) return r->final_norm;
    if (block > 1) return NULL;
    struct { const char *name; h3_gpu_tensor *tensor; } table[] = {
        {"norm1", r->block[block].norm1}, {"qkv", r->block[block].qkv},
        {"q_norm", r->block[block].q_norm},
        {"k_norm", r->block[block].k_norm}, {"out", r->block[block].out},
        {"norm2", r->block[block].norm2}, {"fc1", r->block[block].fc1},
        {"fc2", r->block[block].fc2}};
    for (size_t i = 0; i < sizeof(table) / sizeof(*table); i++)
        if (!strcmp(name, table[i].name)) return table[i].tensor;
    return NULL;
}

static int refiner_fill(h3hip_refiner *r, h3_gpu_tensor *t, uint64_t *seed,
                        float mean, float std) {
    return h3_gpu_fill_normal_bf16(r->gpu, t, 0, h3_gpu_tensor_elements(t),
                                   (*seed)++, mean, std);
}

int h3hip_refiner_init_random(h3hip_refiner *r, uint64_t seed,
                              float weight_std) {
    if (!r) return 0;
    if (!h3_gpu_begin(r->gpu)) return refiner_fail(r, "begin refiner init");
    uint64_t s = seed * 1000003ull + 29;
    int ok = refiner_fill(r, r->condition_w, &s, 0.0f, weight_std) &&
             refiner_fill(r, r->condition_b, &s, 0.0f, 0.02f) &&
             refiner_fill(r, r->final_norm, &s, 1.0f, 0.02f);
    for (int b = 0; b < 2 && ok; b++)
        ok = refiner_fill(r, r->block[b].norm1, &s, 1.0f, 0.02f) &&
             refiner_fill(r, r->block[b].qkv, &s, 0.0f, weight_std) &&
             refiner_fill(r, r->block[b].q_norm, &s, 1.0f, 0.02f) &&
             refiner_fill(r, r->block[b].k_norm, &s, 1.0f, 0.02f) &&
             refiner_fill(r, r->block[b].out, &s, 0.0f, weight_std) &&
             refiner_fill(r, r->block[b].norm2, &s, 1.0f, 0.02f) &&
             refiner_fill(r, r->block[b].fc1, &s, 0.0f, weight_std) &&
             refiner_fill(r, r->block[b].fc2, &s, 0.0f, weight_std);
    if (!ok) {
        refiner_fail(r, "refiner init");
        (void)h3_gpu_submit(r->gpu);
        return 0;
    }
    return h3_gpu_submit(r->gpu) ? 1 : refiner_fail(r, "refiner init");
}

int h3hip_refiner_run(h3hip_refiner *r, h3_gpu_tensor *output,
                      const h3_gpu_tensor *source, uint32_t rows) {
    if (!r) return 0;
    h3_gpu *gpu = r->gpu;
    const uint32_t d = r->hidden, hd = r->head_dim, heads = r->heads;
    const uint32_t inner = heads * hd, f = r->ffn;
    if (!rows || !output || !source ||
        h3_gpu_tensor_elements(output) < (size_t)rows * d ||
        h3_gpu_tensor_elements(source) < (size_t)rows * r->text_dim) {
        snprintf(r->error, sizeof(r->error), "invalid refiner run");
        return 0;
    }
    h3_gpu_tensor *norm = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * d);
    h3_gpu_tensor *qkv = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * inner * 3);
    h3_gpu_tensor *query = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * inner);
    h3_gpu_tensor *key = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * inner);
    h3_gpu_tensor *value = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * inner);
    h3_gpu_tensor *heads_out = h3_gpu_tensor_new_bf16(gpu,
                                                      (size_t)rows * inner);
    h3_gpu_tensor *branch = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * d);
    h3_gpu_tensor *fc1 = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * f * 2);
    h3_gpu_tensor *act = h3_gpu_tensor_new_bf16(gpu, (size_t)rows * f);
    h3_gpu_tensor *scratch[] = {norm, qkv, query, key, value, heads_out,
                                branch, fc1, act};
    int ok = 1;
    for (size_t i = 0; i < sizeof(scratch) / sizeof(*scratch); i++)
        if (!scratch[i]) ok = 0;
    if (!ok) refiner_fail(r, "cannot allocate refiner scratch");
    const float scale = 1.0f / sqrtf((float)hd);
    h3_gpu_tensor *x = output;
#define STEP(call, what) (ok = ok && ((call) || refiner_fail(r, what)))
    STEP(h3_gpu_begin(gpu), "begin token refinement");
    int begun = ok;
    STEP(h3_gpu_linear_bf16(gpu, x, source, r->condition_w, r->condition_b,
                            rows, r->text_dim, d), "condition projection");
    for (int b = 0; b < 2; b++) {
        STEP(h3_gpu_rms_norm_bf16(gpu, norm, x, r->block[b].norm1, rows, d,
                                  1e-5f), "refiner attention norm");
        STEP(h3_gpu_linear_bf16(gpu, qkv, norm, r->block[b].qkv, NULL, rows,
                                d, inner * 3), "refiner QKV");
        /* rope_half 0: per-head RMS of q and k only, the tables unread */
        STEP(h3_gpu_grouped_qkv_rope_bf16(gpu, query, key, value, qkv,
                                          r->block[b].q_norm,
                                          r->block[b].k_norm,
                                          r->block[b].q_norm,
                                          r->block[b].q_norm, rows, heads,
                                          hd, 0, 1e-5f), "refiner QK norm");
        STEP(h3_gpu_sdpa_bf16(gpu, heads_out, query, key, value, rows, heads,
                              hd, scale), "refiner attention");
        STEP(h3_gpu_linear_bf16(gpu, branch, heads_out, r->block[b].out, NULL,
                                rows, inner, d), "refiner attention output");
        STEP(h3_gpu_add_bf16(gpu, x, x, branch, (size_t)rows * d),
             "refiner attention residual");
        STEP(h3_gpu_rms_norm_bf16(gpu, norm, x, r->block[b].norm2, rows, d,
                                  1e-5f), "refiner MLP norm");
        STEP(h3_gpu_linear_bf16(gpu, fc1, norm, r->block[b].fc1, NULL, rows,
                                d, f * 2), "refiner MLP input");
        STEP(h3_gpu_swiglu_bf16(gpu, act, fc1, rows, f), "refiner SwiGLU");
        STEP(h3_gpu_linear_bf16(gpu, branch, act, r->block[b].fc2, NULL, rows,
                                f, d), "refiner MLP output");
        STEP(h3_gpu_add_bf16(gpu, x, x, branch, (size_t)rows * d),
             "refiner MLP residual");
    }
    STEP(h3_gpu_rms_norm_bf16(gpu, x, x, r->final_norm, rows, d, 1e-5f),
         "refiner final norm");
#undef STEP
    if (begun && !h3_gpu_submit(gpu) && ok) ok = refiner_fail(r, "submit");
    for (size_t i = 0; i < sizeof(scratch) / sizeof(*scratch); i++)
        h3_gpu_tensor_free(scratch[i]);
    return ok;
}
