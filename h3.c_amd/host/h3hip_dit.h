/* DiT denoiser driver over the h3_gpu.h device API.
 *
 * Two block families share the same kernels:
 *   H3HIP_FAMILY_H3  - the engine's MiniMax-H3 block (reference
 *                      h3_dit.c:2008-2180): RMS adaLN, grouped QKV with
 *                      per-head Q/K RMS norm and 3D RoPE, one joint
 *                      self-attention over the packed sequence, SwiGLU MLP,
 *                      gates fused with the next adaLN.
 *   H3HIP_FAMILY_WAN - the Wan-style block the benchmark configs describe:
 *                      LayerNorm adaLN, self-attention with per-head Q/K RMS
 *                      norm and 3D RoPE, text cross-attention, GELU-tanh
 *                      FFN, biases on every projection.
 * All weights of all blocks stay resident in HBM.  The driver issues only
 * h3_gpu.h / h3_hip.h calls; it never touches device memory itself.
 */
#ifndef H3HIP_DIT_H
#define H3HIP_DIT_H

#include "../../include/h3_gpu.h"
#include "../../include/h3_hip.h"
#include "h3hip_host.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { H3HIP_FAMILY_H3 = 0, H3HIP_FAMILY_WAN = 1 };

typedef struct {
    int family;
    uint32_t hidden;     /* H3: 5376, Wan: 5120 */
    uint32_t heads;      /* H3: 56, Wan: 40 */
    uint32_t head_dim;   /* 128 */
    uint32_t ffn;        /* H3: 14336 (SwiGLU), Wan: 13824 (GELU) */
    uint32_t blocks;     /* resident blocks (50) */
    uint32_t rows;       /* H3: packed sequence; Wan: video rows */
    uint32_t text_rows;  /* Wan: cross-attention context rows */
    uint32_t time_rows;  /* modulation rows */
    uint32_t rope_half;  /* 48 */
    float epsilon;       /* 1e-5 for H3, 1e-6 for Wan */
} h3hip_dit_config;

typedef struct h3hip_dit h3hip_dit;

/* Allocates every weight, modulation and activation tensor (uninitialised).
 * Returns NULL and fills error on failure. */
h3hip_dit *h3hip_dit_create(h3_gpu *gpu, const h3hip_dit_config *config,
                            char *error, size_t error_size);
void h3hip_dit_free(h3hip_dit *dit);

/* Seeded device-side init: projection weights ~ N(0, weight_std^2), norm
 * weights ~ 1 + N(0, 0.02^2), biases ~ N(0, 0.02^2), modulation
 * ~ N(0, mod_std^2), hidden/context ~ N(0, 1).  Must be called outside a
 * batch. */
int h3hip_dit_init_random(h3hip_dit *dit, uint64_t seed, float weight_std,
                          float mod_std);

/* Upload RoPE tables ([rows][rope_half] F32 each; cast to bf16 with RNE on
 * the device, as the reference does, h3_dit.c:960-1003) and the modulation
 * row map ([rows] u32).  Outside a batch. */
int h3hip_dit_set_rope(h3hip_dit *dit, const float *cosines,
                       const float *sines);
int h3hip_dit_set_row_map(h3hip_dit *dit, const uint32_t *row_map);

/* Tensor handles, for tests and harnesses:
 *   per block: "norm1" "norm2" "norm3" "norm3_bias" "qkv" "qkv_bias"
 *              "q_norm" "k_norm" "out" "out_bias" "fc1" "fc1_bias" "fc2"
 *              "fc2_bias" "cq" "cq_bias" "ck" "ck_bias" "cv" "cv_bias"
 *              "cq_norm" "ck_norm" "co" "co_bias" "modulation"
 *   shared (block ignored): "hidden" "row_map" "rope_cos" "rope_sin"
 *              "context"
 *   sampler (block ignored): "video_input" "audio_input" "video_patch_w"
 *              "video_patch_b" "audio_patch_w" "audio_patch_b"
 *              "refined_text" "final_norm" "final_modulation"
 *              "final_video_w" "final_video_b" "final_audio_w"
 *              "final_audio_b" "video_velocity" "audio_velocity"
 *              "time_in_w" "time_in_b" "time_out_w" "time_out_b" (after
 *              h3hip_dit_schedule_precompute)
 *   per step (block = step): "step_row_map" "final_video_map"
 *              "final_audio_map"
 * Returns NULL for a name the family does not use. */
h3_gpu_tensor *h3hip_dit_tensor(h3hip_dit *dit, const char *name,
                                uint32_t block);

/* Run blocks [first, first + count) on the current hidden state inside an
 * open batch (h3_gpu_begin .. h3_gpu_submit is the caller's).  For H3, the
 * MLP gate of a block is fused with the next block's attention adaLN when
 * the next block is in the range (reference h3_dit.c:2139-2178). */
int h3hip_dit_run_blocks(h3hip_dit *dit, uint32_t first, uint32_t count);

/* Op classes of a block, for isolating one kernel family when timing:
 * run_blocks_ops() issues only the ops whose class bit is set, in the same
 * order and with the same shapes and tensors as run_blocks() (the numerics
 * of a partial run are meaningless; the launches are identical). */
enum {
    H3HIP_OPS_GEMM = 1,      /* plain-epilogue projections (+bias) over the
                                sequence rows */
    H3HIP_OPS_GEMM_ACT = 2,  /* projections with a SwiGLU / GELU epilogue */
    H3HIP_OPS_ATTENTION = 4, /* flash attention (self and cross) */
    H3HIP_OPS_ROWS = 8,      /* adaLN, gates, norms, RoPE, residual adds */
    H3HIP_OPS_CONTEXT = 16,  /* Wan: cross K / V projections of the text */
    H3HIP_OPS_ALL = 31
};
int h3hip_dit_run_blocks_ops(h3hip_dit *dit, uint32_t first, uint32_t count,
                             unsigned op_mask);
/* FLOPs one block spends in the plain-epilogue projections (class GEMM). */
double h3hip_dit_block_plain_gemm_flops(const h3hip_dit_config *config);
/* FLOPs one block spends in the ops of one class (a single H3HIP_OPS_ bit;
 * GEMM FLOPs for the projection classes, QK^T and PV for attention, 0 for
 * the row ops). */
double h3hip_dit_block_class_flops(const h3hip_dit_config *config,
                                   unsigned op_class);
/* Launches of class GEMM per block. */
uint32_t h3hip_dit_block_plain_gemm_launches(const h3hip_dit_config *config);

/* Algorithmic FLOPs of one block at the configured shape (GEMMs + attention,
 * 2 flops per multiply-add). */
double h3hip_dit_block_flops(const h3hip_dit_config *config);
/* FLOPs of the GEMMs alone and of the attention alone. */
double h3hip_dit_block_gemm_flops(const h3hip_dit_config *config);
double h3hip_dit_block_attention_flops(const h3hip_dit_config *config);

/* ------------------------------------------------------------------
 * H3 sampler: the step either side of the blocks and the Euler loop
 * (reference h3_dit.c encode_forward :2182-2528, denoise_euler_gpu
 * :2745-2917, prepare_maps :1134-1200).
 *
 * The packed sequence follows `layout` (config.rows == layout->seq_len):
 * text segments are copied from the refined text rows, video-kind segments
 * (condition, reference image, video) are projected from the F32 video
 * latent rows in layout order, audio-kind segments (reference audio, audio)
 * from the audio latent rows.  The layout holds one video and one audio
 * target segment, each after its modality's condition segments.  The
 * modulation of every block has one row per time row of the schedule
 * (config.time_rows must equal h3hip_time_rows() for these sigmas); the
 * final adaLN modulation is [time_rows][2][hidden].
 * ------------------------------------------------------------------ */
typedef struct {
    const h3hip_layout *layout;
    int steps;
    const float *video_sigmas;  /* steps + 1 */
    const float *audio_sigmas;  /* steps + 1 */
    int reuse_interval;         /* 1 = every step evaluated */
    uint32_t video_patch;       /* 96 */
    uint32_t audio_channels;    /* 32 */
} h3hip_sampler_config;

/* Allocate the sampler tensors and upload the per-step row maps. */
int h3hip_dit_sampler_create(h3hip_dit *dit, const h3hip_sampler_config *cfg);
/* Seeded init of the patch projections (F32), final norm, final heads,
 * final modulation and refined text rows, like h3hip_dit_init_random. */
int h3hip_dit_sampler_init_random(h3hip_dit *dit, uint64_t seed,
                                  float weight_std, float mod_std);
/* Write / read the F32 latent rows: video [video rows][video_patch],
 * audio [audio rows][audio_channels], condition rows first. */
int h3hip_dit_sampler_write_latents(h3hip_dit *dit, const float *video,
                                    const float *audio);
int h3hip_dit_sampler_read_latents(h3hip_dit *dit, float *video,
                                   float *audio);
/* One forward at `step` inside an open batch: pack the sequence, run all
 * blocks, final adaLN + heads into the bf16 velocity tensors. */
int h3hip_dit_forward_step(h3hip_dit *dit, int step);
/* The whole Euler denoise with velocity reuse; opens and submits its own
 * batches. Returns the number of forwards evaluated, 0 on failure. */
int h3hip_dit_denoise(h3hip_dit *dit);
/* Modulation precompute (reference h3_dit_schedule.c:78-337), after
 * h3hip_dit_sampler_create: 256-d timestep features of the schedule's
 * time rows (t = 1 - sigma) -> F32 linear 256 -> hidden, SiLU, F32 linear
 * hidden -> hidden/2, bf16 cast, bf16 SiLU -> per block the adaLN
 * projection hidden/2 -> 3 x 6 x hidden (+bias) into that block's
 * modulation, and the final projection hidden/2 -> 2 x hidden (+bias) into
 * the final modulation.  Opens and submits its own batch.
 *
 * Synthetic weights, generated on the device with h3_gpu_fill_normal_*:
 * time MLP in/out weights ~ N(0, weight_std^2) with seeds seed, seed + 2,
 * biases ~ N(0, 0.02^2) with seeds seed + 1, seed + 3 (kept, names
 * "time_in_w" "time_in_b" "time_out_w" "time_out_b"); the projection of
 * block b ~ N(0, weight_std^2) with seed seed + 16 + 2b, its bias
 * ~ N(0, 0.02^2) with seed seed + 17 + 2b; the final projection seeds
 * seed + 8 and seed + 9.  Like the reference, which loads each block's
 * projection, uses it once and frees it, the projection weights live in
 * one buffer that is regenerated per block. */
int h3hip_dit_schedule_precompute(h3hip_dit *dit, uint64_t seed,
                                  float weight_std);

/* Opt-in block-sparse joint attention, the reference's H3_SPARSE_ATTN=T:H:W:G
 * (h3_dit.c:1006-1132): builds the layout's CSR window mask
 * (h3hip_sparse_mask) and registers it with h3_gpu_sdpa_set_sparse, so
 * every joint attention over config.rows rows is masked.  Radii 0 with
 * global_stride 0 and clear = 1 removes the mask.  Outside a batch.
 * Returns the kept-tile count, 0 when the layout has no single target
 * video segment (attention stays dense), -1 on failure. */
long h3hip_dit_set_sparse_window(h3hip_dit *dit, const h3hip_layout *layout,
                                 unsigned radius_t, unsigned radius_h,
                                 unsigned radius_w, unsigned global_stride,
                                 int clear);

/* Rows of each latent array: video / audio totals and their targets. */
void h3hip_dit_sampler_rows(const h3hip_dit *dit, uint32_t *video_rows,
                            uint32_t *audio_rows, uint32_t *video_targets,
                            uint32_t *audio_targets);

const char *h3hip_dit_error(const h3hip_dit *dit);

/* Text token refiner (reference refine_text / run_refiner_block,
 * h3_dit.c:766-884): the text encoder's rows (text_dim wide) are projected
 * to the model width with a biased linear, passed through two pre-norm
 * self-attention + SwiGLU blocks with no RoPE and no modulation, and
 * RMS-normalised.  Its weights are separate from the denoiser blocks; the
 * shapes follow the DiT it refines for (hidden, heads x head_dim, ffn).
 * Tensor names, block 0 or 1: "norm1" "qkv" "q_norm" "k_norm" "out" "norm2"
 * "fc1" "fc2"; block ignored: "condition_w" [hidden x text_dim]
 * "condition_b" [hidden] "final_norm" [hidden]. */
typedef struct h3hip_refiner h3hip_refiner;

h3hip_refiner *h3hip_refiner_create(h3_gpu *gpu, uint32_t hidden,
                                    uint32_t heads, uint32_t head_dim,
                                    uint32_t ffn, uint32_t text_dim,
                                    char *error, size_t error_size);
void h3hip_refiner_free(h3hip_refiner *refiner);
const char *h3hip_refiner_error(const h3hip_refiner *refiner);
h3_gpu_tensor *h3hip_refiner_tensor(h3hip_refiner *refiner,
                                    const char *name, uint32_t block);
/* Seeded device-side init: norms ~ N(1, 0.02^2), matrices
 * ~ N(0, weight_std^2), the condition bias ~ N(0, 0.02^2). */
int h3hip_refiner_init_random(h3hip_refiner *refiner, uint64_t seed,
                              float weight_std);
/* output [rows x hidden] BF16 <- refine(source [rows x text_dim] BF16).
 * Runs in its own batch; scratch is allocated for the call and freed. */
int h3hip_refiner_run(h3hip_refiner *refiner, h3_gpu_tensor *output,
                      const h3_gpu_tensor *source, uint32_t rows);

#ifdef __cplusplus
}
#endif

#endif
