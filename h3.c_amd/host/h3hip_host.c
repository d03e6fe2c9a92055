/* Host-side math of the DiT path; see h3hip_host.h.  Arithmetic follows the
 * reference engine exactly (cited per function) because the sigma grid,
 * positions, RoPE tables and row maps must match bit for bit. */
#include "h3hip_host.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ temporal */

/* frames are aligned up to 5 + 17 k (reference h3_host.c:14-21) */
int h3hip_align_frame_count(int requested) {
    int frames = requested < 5 ? 5 : requested;
    int over = (frames - 5) % 17;
    if (over < 0) over += 17;
    return over ? frames + (17 - over) : frames;
}

/* 5 + 17 k frames -> 2 + 5 k latent frames (reference h3_host.c:23-26) */
int h3hip_video_latent_t(int frame_count) {
    return frame_count <= 5 ? 2 : ((frame_count - 5) / 17) * 5 + 2;
}

/* audio latents at 40 Hz for 24 fps video (reference h3_host.c:32-40) */
void h3hip_temporal(int requested_frames, int *frame_count, int *video_t,
                    int *audio_t) {
    int frames = h3hip_align_frame_count(requested_frames);
    if (frame_count) *frame_count = frames;
    if (video_t) *video_t = h3hip_video_latent_t(frames);
    if (audio_t) *audio_t = (int)llround((double)frames * 40 / 24);
}

/* --------------------------------------------------------- sigma grids */

/* reference h3_host.c:131-150: base index (i*1000)/steps on a 1000-step
 * grid, shifted with s*b/(1+(s-1)*b) in float */
int h3hip_schedule_build(int steps, float *video, float *audio) {
    if (!video || !audio || steps < 1 || steps > H3HIP_MAX_STEPS) return 0;
    const float vs = (float)H3HIP_VIDEO_SIGMA_SHIFT;
    const float as = (float)H3HIP_AUDIO_SIGMA_SHIFT;
    for (int i = 0; i < steps; i++) {
        float base = (float)(1000 - (i * 1000) / steps) / 1000.0f;
        video[i] = vs * base / (1.0f + (vs - 1.0f) * base);
        audio[i] = as * base / (1.0f + (as - 1.0f) * base);
    }
    video[steps] = 0.0f;
    audio[steps] = 0.0f;
    return 1;
}

/* reference h3_host.c:152-167: linear base 1 - i/n, same shift, terminal 0 */
int h3hip_serving_schedule_build(int evaluations, float *video,
                                 float *audio) {
    if (!video || !audio || evaluations < 2 ||
        evaluations > H3HIP_MAX_STEPS)
        return 0;
    const float n = (float)evaluations;
    const float vs = (float)H3HIP_VIDEO_SIGMA_SHIFT;
    const float as = (float)H3HIP_AUDIO_SIGMA_SHIFT;
    for (int i = 0; i <= evaluations; i++) {
        float base = 1.0f - (float)i / n;
        video[i] = vs * base / (1.0f + (vs - 1.0f) * base);
        audio[i] = as * base / (1.0f + (as - 1.0f) * base);
    }
    video[evaluations] = 0.0f;
    audio[evaluations] = 0.0f;
    return 1;
}

/* -------------------------------------------------------------- layout */

/* token time advance per latent frame: 5/3 * {1,4,4,4,4}[i % 5]
 * (reference h3_host.c:14-15, 283-289) */
static double h3hip_frame_step(int index) {
    static const int per_token[5] = {1, 4, 4, 4, 4};
    return 5.0 / 3.0 * per_token[index % 5];
}

static double h3hip_video_span(int latent_t) {
    double sum = 0.0;
    for (int i = 0; i < latent_t; i++) sum += h3hip_frame_step(i);
    return sum;
}

typedef struct {
    h3hip_layout *layout;
    size_t position_capacity, segment_capacity;
} h3hip_builder;

static int h3hip_append(h3hip_builder *b, int kind,
                        const h3hip_position *rows, size_t count) {
    h3hip_layout *l = b->layout;
    if (l->seq_len + count > b->position_capacity) {
        size_t capacity = b->position_capacity ? b->position_capacity : 256;
        while (capacity < l->seq_len + count) capacity *= 2;
        h3hip_position *grown = (h3hip_position *)realloc(
            l->positions, capacity * sizeof(*grown));
        if (!grown) return 0;
        l->positions = grown;
        b->position_capacity = capacity;
    }
    if (l->segment_count == b->segment_capacity) {
        size_t capacity = b->segment_capacity ? b->segment_capacity * 2 : 16;
        h3hip_segment *grown = (h3hip_segment *)realloc(
            l->segments, capacity * sizeof(*grown));
        if (!grown) return 0;
        l->segments = grown;
        b->segment_capacity = capacity;
    }
    if (count)
        memcpy(l->positions + l->seq_len, rows, count * sizeof(*rows));
    l->segments[l->segment_count].start = l->seq_len;
    l->seq_len += count;
    l->segments[l->segment_count].stop = l->seq_len;
    l->segments[l->segment_count].kind = kind;
    l->segment_count++;
    return 1;
}

/* One latent frame's 2x2-patch grid centred in a 32-unit square whose
 * aspect follows the canvas (reference h3_host.c:253-281).  Also returns the
 * w coordinates of the columns. */
static h3hip_position *h3hip_frame_grid(int latent_h, int latent_w,
                                        size_t *count, double **w_axis,
                                        size_t *w_count) {
    if (latent_h < 2 || latent_w < 2 || latent_h % 2 || latent_w % 2)
        return NULL;
    size_t nh = (size_t)latent_h / 2, nw = (size_t)latent_w / 2;
    h3hip_position *grid =
        (h3hip_position *)malloc(nh * nw * sizeof(*grid));
    double *ws = (double *)malloc(nw * sizeof(*ws));
    if (!grid || !ws) {
        free(grid);
        free(ws);
        return NULL;
    }
    double area = sqrt((double)latent_h * (double)latent_w);
    double ratio_h = latent_h / area, ratio_w = latent_w / area;
    double step_h = ratio_h / (double)nh, step_w = ratio_w / (double)nw;
    double base_h = (1.0 - ratio_h) / 2.0, base_w = (1.0 - ratio_w) / 2.0;
    for (size_t c = 0; c < nw; c++)
        ws[c] = ((double)c * step_w + base_w) * 32.0;
    for (size_t r = 0; r < nh; r++) {
        double hh = ((double)r * step_h + base_h) * 32.0;
        for (size_t c = 0; c < nw; c++) {
            h3hip_position p = {0.0, hh, ws[c]};
            grid[r * nw + c] = p;
        }
    }
    *count = nh * nw;
    *w_axis = ws;
    *w_count = nw;
    return grid;
}

/* audio rows: two streams of audio_t rows at w = low and w = high
 * (reference h3_host.c:291-306) */
static h3hip_position *h3hip_audio_grid(double cursor, int audio_t,
                                        double low, double high,
                                        size_t *count) {
    if (audio_t < 0) return NULL;
    size_t rows = (size_t)audio_t * 2;
    h3hip_position *grid =
        (h3hip_position *)malloc((rows ? rows : 1) * sizeof(*grid));
    if (!grid) return NULL;
    for (int i = 0; i < audio_t; i++) {
        h3hip_position a = {cursor + i, 0.0, low};
        h3hip_position b = {cursor + i, 0.0, high};
        grid[i] = a;
        grid[(size_t)audio_t + (size_t)i] = b;
    }
    *count = rows;
    return grid;
}

/* latent_t frames of the spatial grid with advancing time
 * (reference h3_host.c:308-325) */
static h3hip_position *h3hip_video_grid(double cursor, int latent_t,
                                        const h3hip_position *frame,
                                        size_t frame_rows, size_t *count) {
    if (latent_t < 0) return NULL;
    size_t rows = (size_t)latent_t * frame_rows;
    h3hip_position *grid =
        (h3hip_position *)malloc((rows ? rows : 1) * sizeof(*grid));
    if (!grid) return NULL;
    double time = cursor;
    size_t at = 0;
    for (int i = 0; i < latent_t; i++) {
        for (size_t s = 0; s < frame_rows; s++) {
            h3hip_position p = {time, frame[s].h, frame[s].w};
            grid[at++] = p;
        }
        time += h3hip_frame_step(i);
    }
    *count = rows;
    return grid;
}

static int h3hip_layout_error(char *error, size_t error_size,
                              const char *message) {
    if (error && error_size) snprintf(error, error_size, "%s", message);
    return 0;
}

/* Segment order: text, keyframe conditions or references, audio, video
 * (reference h3_host.c:327-466). */
int h3hip_layout_build(int text_len, int latent_t, int latent_h, int latent_w,
                       int audio_t, int frame_count, const int *keyframes,
                       size_t keyframe_count,
                       const h3hip_layout_ref *references,
                       size_t reference_count, h3hip_layout *layout,
                       char *error, size_t error_size) {
    if (!layout) return 0;
    memset(layout, 0, sizeof(*layout));
    if (error && error_size) error[0] = '\0';
    if (text_len < 1 || latent_t < 1 || audio_t < 0 || frame_count < 5)
        return h3hip_layout_error(error, error_size,
                                  "invalid target layout dimensions");
    if (keyframe_count && reference_count)
        return h3hip_layout_error(error, error_size,
                                  "keyframes and references are mutually "
                                  "exclusive");
    h3hip_builder b = {layout, 0, 0};
    size_t frame_rows = 0, w_count = 0;
    double *w_axis = NULL;
    h3hip_position *frame =
        h3hip_frame_grid(latent_h, latent_w, &frame_rows, &w_axis, &w_count);
    if (!frame)
        return h3hip_layout_error(error, error_size,
                                  "invalid latent canvas or out of memory");
    const char *failure = "out of memory while building layout";
    h3hip_position *text =
        (h3hip_position *)malloc((size_t)text_len * sizeof(*text));
    if (!text) goto fail;
    for (int i = 0; i < text_len; i++) {
        h3hip_position p = {(double)i, 0.0, 0.0};
        text[i] = p;
    }
    if (!h3hip_append(&b, H3HIP_SEG_TEXT, text, (size_t)text_len)) {
        free(text);
        goto fail;
    }
    free(text);

    double cursor = (double)text_len;
    for (size_t i = 0; i < keyframe_count; i++) {
        double when;
        if (keyframes[i] == 0) {
            when = (double)text_len;
        } else if (keyframes[i] == frame_count - 1) {
            when = (double)text_len + h3hip_video_span(latent_t) - 5.0 / 3.0;
        } else {
            failure = "only first and last keyframes are valid";
            goto fail;
        }
        for (size_t r = 0; r < frame_rows; r++) frame[r].t = when;
        if (!h3hip_append(&b, H3HIP_SEG_COND, frame, frame_rows)) goto fail;
        layout->img_cond_rows += frame_rows;
    }

    for (size_t i = 0; i < reference_count; i++) {
        const h3hip_layout_ref *ref = &references[i];
        if (ref->kind == H3HIP_REF_IMAGE) {
            size_t rows = 0, wc = 0;
            double *wa = NULL;
            h3hip_position *grid = h3hip_frame_grid(
                ref->latent_h, ref->latent_w, &rows, &wa, &wc);
            if (!grid) goto fail;
            for (size_t r = 0; r < rows; r++) grid[r].t = cursor;
            int ok = h3hip_append(&b, H3HIP_SEG_REF_IMAGE, grid, rows);
            free(grid);
            free(wa);
            if (!ok) goto fail;
            layout->img_cond_rows += rows;
            cursor += 1.0;
        } else if (ref->kind == H3HIP_REF_AUDIO) {
            size_t rows = 0;
            h3hip_position *grid = h3hip_audio_grid(
                cursor, ref->audio_t, w_axis[0], w_axis[w_count - 1], &rows);
            if (!grid) goto fail;
            int ok = rows ? h3hip_append(&b, H3HIP_SEG_REF_AUDIO, grid, rows)
                          : 1;
            free(grid);
            if (!ok) goto fail;
            layout->audio_cond_rows += rows;
            cursor += ref->audio_t;
        } else if (ref->kind == H3HIP_REF_VIDEO) {
            size_t rows = 0, wc = 0;
            double *wa = NULL;
            h3hip_position *grid = h3hip_frame_grid(
                ref->latent_h, ref->latent_w, &rows, &wa, &wc);
            if (!grid) goto fail;
            if (ref->audio_t > 0) {
                size_t audio_rows = 0;
                h3hip_position *audio = h3hip_audio_grid(
                    cursor, ref->audio_t, wa[0], wa[wc - 1], &audio_rows);
                int ok = audio &&
                         h3hip_append(&b, H3HIP_SEG_REF_AUDIO, audio,
                                      audio_rows);
                free(audio);
                if (!ok) {
                    free(grid);
                    free(wa);
                    goto fail;
                }
                layout->audio_cond_rows += audio_rows;
            }
            size_t video_rows = 0;
            h3hip_position *video = h3hip_video_grid(
                cursor, ref->latent_t, grid, rows, &video_rows);
            free(grid);
            free(wa);
            if (!video) goto fail;
            int ok = h3hip_append(&b, H3HIP_SEG_REF_IMAGE, video, video_rows);
            free(video);
            if (!ok) goto fail;
            layout->img_cond_rows += video_rows;
            cursor += fmax((double)ref->audio_t,
                           h3hip_video_span(ref->latent_t));
        } else {
            failure = "unknown reference layout type";
            goto fail;
        }
    }

    {
        size_t audio_rows = 0;
        h3hip_position *audio = h3hip_audio_grid(
            cursor, audio_t, w_axis[0], w_axis[w_count - 1], &audio_rows);
        if (!audio) goto fail;
        int ok = h3hip_append(&b, H3HIP_SEG_AUDIO, audio, audio_rows);
        free(audio);
        if (!ok) goto fail;
        size_t video_rows = 0;
        h3hip_position *video =
            h3hip_video_grid(cursor, latent_t, frame, frame_rows, &video_rows);
        if (!video) goto fail;
        ok = h3hip_append(&b, H3HIP_SEG_VIDEO, video, video_rows);
        free(video);
        if (!ok) goto fail;
        layout->img_target_rows = video_rows;
        layout->audio_target_rows = audio_rows;
    }
    free(frame);
    free(w_axis);
    return 1;

fail:
    free(frame);
    free(w_axis);
    h3hip_layout_free(layout);
    return h3hip_layout_error(error, error_size, failure);
}

void h3hip_layout_free(h3hip_layout *layout) {
    if (!layout) return;
    free(layout->segments);
    free(layout->positions);
    memset(layout, 0, sizeof(*layout));
}

/* ----------------------------------------------------------------- RNG */

/* PCG32 XSH-RR step (reference h3_host.c:496-502) */
uint32_t h3hip_rng_u32(h3hip_rng *rng) {
    uint64_t old = rng->state;
    rng->state = old * UINT64_C(6364136223846793005) + rng->increment;
    uint32_t xorshifted = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    uint32_t rot = (uint32_t)(old >> 59u);
    return (xorshifted >> rot) | (xorshifted << ((-(int32_t)rot) & 31));
}

/* reference h3_host.c:504-510 */
void h3hip_rng_seed(h3hip_rng *rng, uint64_t seed) {
    memset(rng, 0, sizeof(*rng));
    rng->increment = (seed << 1u) | 1u;
    (void)h3hip_rng_u32(rng);
    rng->state += seed ^ UINT64_C(0x9e3779b97f4a7c15);
    (void)h3hip_rng_u32(rng);
}

/* Box-Muller in double, cos first then the cached sin
 * (reference h3_host.c:512-524) */
float h3hip_rng_normal(h3hip_rng *rng) {
    if (rng->has_spare) {
        rng->has_spare = 0;
        return rng->spare;
    }
    double u1 = ((double)h3hip_rng_u32(rng) + 1.0) / 4294967297.0;
    double u2 = ((double)h3hip_rng_u32(rng) + 0.5) / 4294967296.0;
    double radius = sqrt(-2.0 * log(u1));
    double angle = 2.0 * 3.14159265358979323846 * u2;
    rng->spare = (float)(radius * sin(angle));
    rng->has_spare = 1;
    return (float)(radius * cos(angle));
}

void h3hip_rng_fill_normal(h3hip_rng *rng, float *values, size_t count) {
    for (size_t i = 0; i < count; i++) values[i] = h3hip_rng_normal(rng);
}

/* ---------------------------------------------------------------- RoPE */

void h3hip_rope_tables(const h3hip_position *positions, size_t rows,
                       const float inv_freq[16], float spatial_scale,
                       float *cosines, float *sines) {
    for (size_t r = 0; r < rows; r++) {
        const float axes[3] = {(float)positions[r].t,
                               (float)positions[r].h * spatial_scale,
                               (float)positions[r].w * spatial_scale};
        for (int axis = 0; axis < 3; axis++)
            for (int f = 0; f < 16; f++) {
                size_t index = r * 48 + (size_t)axis * 16 + (size_t)f;
                float angle = axes[axis] * inv_freq[f];
                cosines[index] = cosf(angle);
                sines[index] = sinf(angle);
            }
    }
}

void h3hip_default_inv_freq(float inv_freq[16]) {
    for (int f = 0; f < 16; f++)
        inv_freq[f] = (float)pow(10000.0, -(double)f / 16.0);
}

/* ------------------------------------------------- timestep rows, maps */

uint32_t h3hip_time_rows(int steps, const float *video_sigmas,
                         const float *audio_sigmas, int visual_condition,
                         int audio_condition, uint32_t *video_rows,
                         uint32_t *audio_rows,
                         uint32_t *visual_condition_rows,
                         uint32_t *audio_condition_rows, float *times) {
    if (steps < 1 || !video_sigmas || !audio_sigmas || !video_rows ||
        !audio_rows)
        return 0;
    /* one row per distinct (video, audio) time, ordered by t = 1 - sigma
     * (reference h3_dit_schedule.c:99-111) */
    uint32_t count = 0;
    for (int s = 0; s < steps; s++) {
        float video = 1.0f - video_sigmas[s];
        float audio = 1.0f - audio_sigmas[s];
        if (video == audio) {
            video_rows[s] = count;
            audio_rows[s] = count++;
        } else if (video < audio) {
            video_rows[s] = count++;
            audio_rows[s] = count++;
        } else {
            audio_rows[s] = count++;
            video_rows[s] = count++;
        }
    }
    uint32_t visual_row = UINT32_MAX, audio_row = UINT32_MAX;
    if (visual_condition) visual_row = count++;
    if (audio_condition) audio_row = count++;
    for (int s = 0; s < steps; s++) {
        float video = 1.0f - video_sigmas[s];
        float audio = 1.0f - audio_sigmas[s];
        if (visual_condition && visual_condition_rows)
            visual_condition_rows[s] =
                video >= 0.999f ? video_rows[s] : visual_row;
        if (audio_condition && audio_condition_rows)
            audio_condition_rows[s] = audio >= 1.0f ? audio_rows[s] : audio_row;
    }
    if (times) {
        for (uint32_t i = 0; i < count; i++) times[i] = 0.0f;
        for (int s = 0; s < steps; s++) {
            times[video_rows[s]] = 1.0f - video_sigmas[s];
            times[audio_rows[s]] = 1.0f - audio_sigmas[s];
        }
        if (visual_condition) times[visual_row] = 0.999f;
        if (audio_condition) times[audio_row] = 1.0f;
    }
    return count;
}

/* reference h3_dit_schedule.c:146-157 */
void h3hip_timestep_features(const float *times, uint32_t count,
                             float *features) {
    for (uint32_t r = 0; r < count; r++)
        for (uint32_t i = 0; i < 128; i++) {
            float frequency =
                expf(-logf(10000.0f) * (float)i / (float)128);
            float angle = times[r] * frequency;
            features[(size_t)r * 256 + i] = cosf(angle);
            features[(size_t)r * 256 + 128 + i] = sinf(angle);
        }
}

int h3hip_row_map(const h3hip_layout *layout, uint32_t video_row,
                  uint32_t audio_row, uint32_t visual_condition_row,
                  uint32_t audio_condition_row, const uint8_t *text_tags,
                  size_t text_tag_count, uint32_t *rows, size_t row_count) {
    if (!layout || !rows || row_count != layout->seq_len) return 0;
    size_t text_seen = 0;
    for (size_t i = 0; i < layout->segment_count; i++) {
        const h3hip_segment *seg = &layout->segments[i];
        if (seg->start > seg->stop || seg->stop > row_count) return 0;
        uint32_t time_row, tag;
        switch (seg->kind) {
        case H3HIP_SEG_TEXT:
            for (size_t r = seg->start; r < seg->stop; r++) {
                uint32_t text_tag = 1u;
                if (text_tags) {
                    if (text_seen >= text_tag_count) return 0;
                    text_tag = text_tags[text_seen];
                }
                if (text_tag >= 3u) return 0;
                rows[r] = video_row * 3u + text_tag;
                text_seen++;
            }
            continue;
        case H3HIP_SEG_COND:
        case H3HIP_SEG_REF_IMAGE:
            if (visual_condition_row == UINT32_MAX) return 0;
            time_row = visual_condition_row;
            tag = 0;
            break;
        case H3HIP_SEG_REF_AUDIO:
            if (audio_condition_row == UINT32_MAX) return 0;
            time_row = audio_condition_row;
            tag = 2;
            break;
        case H3HIP_SEG_AUDIO:
            time_row = audio_row;
            tag = 2;
            break;
        case H3HIP_SEG_VIDEO:
            time_row = video_row;
            tag = 0;
            break;
        default:
            return 0;
        }
        for (size_t r = seg->start; r < seg->stop; r++)
            rows[r] = time_row * 3u + tag;
    }
    return !text_tags || text_seen == text_tag_count;
}

int h3hip_reuse_schedule(int steps, int reuse_interval, uint8_t *selected,
                         size_t selected_count) {
    if (steps < 1 || reuse_interval < 1 || reuse_interval > 32 ||
        !selected || selected_count < (size_t)steps)
        return -1;
    int count = 0;
    for (int s = 0; s < steps; s++) {
        int pick = reuse_interval == 1 || s == 0 || s == steps - 1 ||
                   s % reuse_interval == 0;
        selected[s] = (uint8_t)pick;
        count += pick;
    }
    return count;
}

float h3hip_extrapolation_ratio(float current_sigma, float last_sigma,
                                float previous_sigma, int have_previous) {
    if (!have_previous) return 0.0f;
    float denominator = last_sigma - previous_sigma;
    float ratio = denominator != 0.0f
                      ? (current_sigma - last_sigma) / denominator
                      : 0.0f;
    if (ratio < -2.0f) ratio = -2.0f;
    if (ratio > 2.0f) ratio = 2.0f;
    return ratio;
}

/* ----------------------------------------------------- row conversions */

/* row (t, h/2, w/2) holds [c][dh][dw] of the 2x2 patch */
static int h3hip_video_ok(int c, int t, int h, int w, size_t count) {
    return c > 0 && t > 0 && h > 0 && w > 0 && h % 2 == 0 && w % 2 == 0 &&
           count == (size_t)c * t * h * w;
}

int h3hip_patchify_video(const float *latent, int channels, int time,
                         int height, int width, float *rows, size_t count) {
    if (!latent || !rows || !h3hip_video_ok(channels, time, height, width,
                                            count))
        return 0;
    size_t out = 0;
    for (int t = 0; t < time; t++)
        for (int h = 0; h < height; h += 2)
            for (int w = 0; w < width; w += 2)
                for (int c = 0; c < channels; c++)
                    for (int dh = 0; dh < 2; dh++)
                        for (int dw = 0; dw < 2; dw++)
                            rows[out++] = latent[(((size_t)c * time + t) *
                                                      height + h + dh) *
                                                     width + w + dw];
    return 1;
}

int h3hip_unpatchify_video(const float *rows, int channels, int time,
                           int height, int width, float *latent,
                           size_t count) {
    if (!latent || !rows || !h3hip_video_ok(channels, time, height, width,
                                            count))
        return 0;
    size_t in = 0;
    for (int t = 0; t < time; t++)
        for (int h = 0; h < height; h += 2)
            for (int w = 0; w < width; w += 2)
                for (int c = 0; c < channels; c++)
                    for (int dh = 0; dh < 2; dh++)
                        for (int dw = 0; dw < 2; dw++)
                            latent[(((size_t)c * time + t) * height + h +
                                    dh) * width + w + dw] = rows[in++];
    return 1;
}

/* audio latent [channel][stream][time] -> rows [stream][time][channel] */
int h3hip_pack_audio(const float *latent, int channels, int time,
                     float *rows, size_t count) {
    if (!latent || !rows || channels < 1 || time < 1 ||
        count != (size_t)channels * 2 * time)
        return 0;
    size_t out = 0;
    for (int s = 0; s < 2; s++)
        for (int t = 0; t < time; t++)
            for (int c = 0; c < channels; c++)
                rows[out++] = latent[((size_t)c * 2 + s) * time + t];
    return 1;
}

int h3hip_unpack_audio(const float *rows, int channels, int time,
                       float *latent, size_t count) {
    if (!latent || !rows || channels < 1 || time < 1 ||
        count != (size_t)channels * 2 * time)
        return 0;
    size_t in = 0;
    for (int s = 0; s < 2; s++)
        for (int t = 0; t < time; t++)
            for (int c = 0; c < channels; c++)
                latent[((size_t)c * 2 + s) * time + t] = rows[in++];
    return 1;
}

int h3hip_euler_velocity_step(float *sample, const float *velocity,
                              size_t count, float sigma, float sigma_next) {
    if (!sample || !velocity || !isfinite(sigma) || !isfinite(sigma_next) ||
        !(sigma > sigma_next) || sigma_next < 0.0f)
        return 0;
    float delta = sigma - sigma_next;
    for (size_t i = 0; i < count; i++) sample[i] += delta * velocity[i];
    return 1;
}

uint16_t h3hip_f32_to_bf16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

float h3hip_bf16_to_f32(uint16_t value) {
    uint32_t bits = (uint32_t)value << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* ------------------------------------------------ block-sparse attention */

typedef struct {
    int global, min_t, max_t, min_h, max_h, min_w, max_w;
} hh_box;

static int hh_gap(int qmin, int qmax, int kmin, int kmax) {
    return kmin > qmax ? kmin - qmax : qmin > kmax ? qmin - kmax : 0;
}

long h3hip_sparse_mask(const h3hip_layout *layout, unsigned radius_t,
                       unsigned radius_h, unsigned radius_w,
                       unsigned global_stride, uint32_t *ptr, uint32_t *idx,
                       size_t idx_capacity) {
    if (!layout || !ptr || !layout->positions) return -1;
    size_t video_start = 0, video_stop = 0;
    unsigned video_segments = 0;
    for (size_t i = 0; i < layout->segment_count; i++)
        if (layout->segments[i].kind == H3HIP_SEG_VIDEO) {
            video_start = layout->segments[i].start;
            video_stop = layout->segments[i].stop;
            video_segments++;
        }
    if (video_segments != 1) return -1;
    const size_t rows = layout->seq_len;
    const size_t qblocks = (rows + 127) / 128, ktiles = (rows + 63) / 64;
    hh_box *boxes = (hh_box *)calloc(qblocks + ktiles, sizeof(hh_box));
    if (!boxes) return -1;
    hh_box *qbox = boxes, *kbox = boxes + qblocks;
    for (size_t b = 0; b < qblocks + ktiles; b++) {
        boxes[b].min_t = boxes[b].min_h = boxes[b].min_w = INT_MAX;
        boxes[b].max_t = boxes[b].max_h = boxes[b].max_w = INT_MIN;
    }
    for (size_t row = 0; row < rows; row++) {
        hh_box *sides[2] = {&qbox[row / 128], &kbox[row / 64]};
        for (int side = 0; side < 2; side++) {
            hh_box *box = sides[side];
            if (row < video_start || row >= video_stop) {
                box->global = 1;
                continue;
            }
            const int t = (int)lrint(layout->positions[row].t);
            const int h = (int)lrint(layout->positions[row].h);
            const int w = (int)lrint(layout->positions[row].w);
            if (t < box->min_t) box->min_t = t;
            if (t > box->max_t) box->max_t = t;
            if (h < box->min_h) box->min_h = h;
            if (h > box->max_h) box->max_h = h;
            if (w < box->min_w) box->min_w = w;
            if (w > box->max_w) box->max_w = w;
        }
    }
    size_t at = 0;
    for (size_t q = 0; q < qblocks; q++) {
        ptr[q] = (uint32_t)at;
        for (size_t k = 0; k < ktiles; k++) {
            int keep = qbox[q].global || kbox[k].global ||
                       (global_stride && k % global_stride == 0);
            if (!keep && qbox[q].min_t <= qbox[q].max_t &&
                kbox[k].min_t <= kbox[k].max_t)
                keep = hh_gap(qbox[q].min_t, qbox[q].max_t, kbox[k].min_t,
                              kbox[k].max_t) <= (int)radius_t &&
                       hh_gap(qbox[q].min_h, qbox[q].max_h, kbox[k].min_h,
                              kbox[k].max_h) <= (int)radius_h &&
                       hh_gap(qbox[q].min_w, qbox[q].max_w, kbox[k].min_w,
                              kbox[k].max_w) <= (int)radius_w;
            if (keep) {
                if (idx && at < idx_capacity) idx[at] = (uint32_t)k;
                at++;
            }
        }
    }
    ptr[qblocks] = (uint32_t)at;
    free(boxes);
    return (long)at;
}
