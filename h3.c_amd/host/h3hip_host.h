/* Host-side math of the DiT denoiser path: temporal shapes, sigma grids,
 * the packed-sequence layout with (t, h, w) positions, the PCG32 +
 * Box-Muller RNG, 3D RoPE tables, timestep rows and modulation row maps,
 * the reuse schedule and patchify/pack conversions.
 *
 * Every function reproduces the reference engine's arithmetic bit for bit
 * (same float/double types, same operation order); each definition cites
 * the reference lines it follows.  Pure C11, no device code.
 */
#ifndef H3HIP_HOST_H
#define H3HIP_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3HIP_MAX_STEPS 1000
#define H3HIP_VIDEO_SIGMA_SHIFT 12.0
#define H3HIP_AUDIO_SIGMA_SHIFT 3.0

typedef struct {
    double t, h, w;
} h3hip_position;

/* segment kinds in the reference's enum order (h3_host.h:32-39) */
enum {
    H3HIP_SEG_TEXT = 0,
    H3HIP_SEG_COND,
    H3HIP_SEG_REF_IMAGE,
    H3HIP_SEG_REF_AUDIO,
    H3HIP_SEG_AUDIO,
    H3HIP_SEG_VIDEO
};

typedef struct {
    size_t start, stop;
    int kind;
} h3hip_segment;

enum { H3HIP_REF_IMAGE = 0, H3HIP_REF_AUDIO, H3HIP_REF_VIDEO };

typedef struct {
    int kind;
    int latent_t, latent_h, latent_w, audio_t;
} h3hip_layout_ref;

typedef struct {
    size_t seq_len;
    h3hip_segment *segments;
    size_t segment_count;
    h3hip_position *positions;
    size_t img_cond_rows, img_target_rows;
    size_t audio_cond_rows, audio_target_rows;
} h3hip_layout;

typedef struct {
    uint64_t state, increment;
    float spare;
    int has_spare;
} h3hip_rng;

/* temporal / canvas (reference h3_host.c:14-40) */
int h3hip_align_frame_count(int requested);
int h3hip_video_latent_t(int frame_count);
void h3hip_temporal(int requested_frames, int *frame_count, int *video_t,
                    int *audio_t);

/* sigma grids: arrays of steps + 1 values (reference h3_host.c:131-167) */
int h3hip_schedule_build(int steps, float *video, float *audio);
int h3hip_serving_schedule_build(int evaluations, float *video, float *audio);

/* packed layout (reference h3_host.c:233-475) */
int h3hip_layout_build(int text_len, int latent_t, int latent_h, int latent_w,
                       int audio_t, int frame_count, const int *keyframes,
                       size_t keyframe_count,
                       const h3hip_layout_ref *references,
                       size_t reference_count, h3hip_layout *layout,
                       char *error, size_t error_size);
void h3hip_layout_free(h3hip_layout *layout);

/* RNG (reference h3_host.c:496-530) */
void h3hip_rng_seed(h3hip_rng *rng, uint64_t seed);
uint32_t h3hip_rng_u32(h3hip_rng *rng);
float h3hip_rng_normal(h3hip_rng *rng);
void h3hip_rng_fill_normal(h3hip_rng *rng, float *values, size_t count);

/* 3D RoPE tables [rows][48] in F32 (reference h3_dit.c:907-922):
 * angle = axis_position * inv_freq[f], axis in (t, h*scale, w*scale),
 * index row*48 + axis*16 + f. */
void h3hip_rope_tables(const h3hip_position *positions, size_t rows,
                       const float inv_freq[16], float spatial_scale,
                       float *cosines, float *sines);
/* inv_freq[f] = 10000^(-f/16), the synthetic stand-in for the checkpoint's
 * rope.inv_freq tensor */
void h3hip_default_inv_freq(float inv_freq[16]);

/* Timestep rows (reference h3_dit_schedule.c:78-161).  video_rows /
 * audio_rows / *_condition_rows get one entry per step; times receives one
 * value (1 - sigma) per time row.  Returns the number of time rows, 0 on
 * invalid input.  times may be NULL to query the count. */
uint32_t h3hip_time_rows(int steps, const float *video_sigmas,
                         const float *audio_sigmas, int visual_condition,
                         int audio_condition, uint32_t *video_rows,
                         uint32_t *audio_rows,
                         uint32_t *visual_condition_rows,
                         uint32_t *audio_condition_rows, float *times);
/* Sinusoidal 256-d features per time row (cos half, then sin half). */
void h3hip_timestep_features(const float *times, uint32_t count,
                             float *features);
/* Modulation row map (reference h3_dit_schedule.c:434-485):
 * rows[r] = time_row * 3 + tag. */
int h3hip_row_map(const h3hip_layout *layout, uint32_t video_row,
                  uint32_t audio_row, uint32_t visual_condition_row,
                  uint32_t audio_condition_row, const uint8_t *text_tags,
                  size_t text_tag_count, uint32_t *rows, size_t row_count);

/* Block-sparse attention mask of a packed layout (reference
 * h3_dit.c:1006-1132): a CSR over 128-row query blocks of 64-row key
 * tiles.  Target-video tiles attend within a 3D window of the given radii
 * (latent-patch units, positions rounded with lrint) plus every
 * global_stride-th tile (0 disables); a tile holding any text, audio,
 * condition or reference row is global in both directions.  ptr receives
 * qblocks + 1 offsets; idx (when idx_capacity suffices) the tile lists.
 * Returns the number of kept tiles, or -1 when the layout has no single
 * target video segment (the reference then stays dense). */
long h3hip_sparse_mask(const h3hip_layout *layout, unsigned radius_t,
                       unsigned radius_h, unsigned radius_w,
                       unsigned global_stride, uint32_t *ptr, uint32_t *idx,
                       size_t idx_capacity);

/* Evaluated steps under velocity reuse (reference h3_dit.c:2672-2687). */
int h3hip_reuse_schedule(int steps, int reuse_interval, uint8_t *selected,
                         size_t selected_count);
/* Clamped velocity extrapolation ratio (reference h3_dit.c:2644-2655). */
float h3hip_extrapolation_ratio(float current_sigma, float last_sigma,
                                float previous_sigma, int have_previous);

/* Latent <-> row conversions (reference h3_dit.c:3209-3283). */
int h3hip_patchify_video(const float *latent, int channels, int time,
                         int height, int width, float *rows, size_t count);
int h3hip_unpatchify_video(const float *rows, int channels, int time,
                           int height, int width, float *latent,
                           size_t count);
int h3hip_pack_audio(const float *latent, int channels, int time,
                     float *rows, size_t count);
int h3hip_unpack_audio(const float *rows, int channels, int time,
                       float *latent, size_t count);

/* Host Euler step (reference h3_host.c:689-697). */
int h3hip_euler_velocity_step(float *sample, const float *velocity,
                              size_t count, float sigma, float sigma_next);

/* bf16 helpers matching the device rounding (RNE) */
uint16_t h3hip_f32_to_bf16(float value);
float h3hip_bf16_to_f32(uint16_t value);

#ifdef __cplusplus
}
#endif

#endif
