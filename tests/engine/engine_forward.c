/* engine_forward: one velocity evaluation through the reference engine's own
 * DiT model layer (h3_dit.c, h3_dit_schedule.c, h3_weights.c,
 * h3_safetensors.c, h3_host.c, compiled unmodified from the reference tree)
 * running on this repository's HIP backend, libh3_gpu_hip.so.
 *
 *   engine_forward <checkpoint dir> <text.bin> <text rows> <latent_t>
 *                  <latent_h> <latent_w> <audio_t> <frames> <steps> <step>
 *                  <active blocks> <seed> <out dir>
 *
 * text.bin holds text rows x 5120 bf16 values.  The program builds the packed
 * layout (h3_layout_build) and the serving sigma grid
 * (h3_serving_schedule_build), loads the model with h3_dit_load_t2va
 * (h3_dit.c:1833: text refinement, AdaLN schedule precompute, core blocks),
 * draws N(0,1) video [24,T,H,W] and audio [32,2,T] latents from the
 * reference's own PCG32 + Box-Muller stream (h3_rng), runs h3_dit_forward
 * (h3_dit.c:2574) for one step, and writes into <out dir>:
 *   video_rows.f32 / audio_rows.f32       the latents as packed rows
 *                                          (h3_dit_patchify_video,
 *                                          h3_dit_pack_audio)
 *   video_velocity.f32 / audio_velocity.f32  the velocities as packed rows
 * The layer policy is pinned to "uniform" (configure_active_blocks,
 * h3_dit.c:1312-1322) so the active blocks follow from the count alone. */
#include "h3_dit.h"
#include "h3_host.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int write_file(const char *dir, const char *name, const void *data,
                      size_t bytes) {
    char path[4096];
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) return 0;
    int ok = fwrite(data, 1, bytes, f) == bytes;
    return fclose(f) == 0 && ok;
}

int main(int argc, char **argv) {
    if (argc != 14) {
        fprintf(stderr, "usage: %s ckpt text.bin text_rows lt lh lw at "
                        "frames steps step active seed out_dir\n", argv[0]);
        return 2;
    }
    const char *ckpt = argv[1], *text_path = argv[2], *out_dir = argv[13];
    const int text_rows = atoi(argv[3]);
    h3_layout_spec spec;
    memset(&spec, 0, sizeof(spec));
    spec.text_len = text_rows;
    spec.latent_t = atoi(argv[4]);
    spec.latent_h = atoi(argv[5]);
    spec.latent_w = atoi(argv[6]);
    spec.audio_t = atoi(argv[7]);
    spec.frame_count = atoi(argv[8]);
    const int steps = atoi(argv[9]), step = atoi(argv[10]);
    const unsigned active = (unsigned)atoi(argv[11]);
    const uint64_t seed = strtoull(argv[12], NULL, 10);
    char error[1024] = {0};

    setenv("H3_DIT_LAYER_POLICY", "uniform", 1);

    h3_layout layout;
    memset(&layout, 0, sizeof(layout));
    if (!h3_layout_build(&spec, &layout, error, sizeof(error))) {
        fprintf(stderr, "layout: %s\n", error);
        return 1;
    }
    static h3_sigma_schedule sigmas;
    if (!h3_serving_schedule_build(steps, &sigmas)) {
        fprintf(stderr, "sigma schedule failed\n");
        return 1;
    }
    size_t text_elements = (size_t)text_rows * H3_TEXT_HIDDEN_SIZE;
    uint16_t *text_values = malloc(text_elements * sizeof(uint16_t));
    FILE *tf = fopen(text_path, "rb");
    if (!text_values || !tf ||
        fread(text_values, sizeof(uint16_t), text_elements, tf) !=
            text_elements) {
        fprintf(stderr, "cannot read %s\n", text_path);
        return 1;
    }
    fclose(tf);
    h3_text_embedding text;
    memset(&text, 0, sizeof(text));
    text.tokens = (size_t)text_rows;
    text.width = H3_TEXT_HIDDEN_SIZE;
    text.values = text_values;

    h3_dit *dit = h3_dit_load_t2va(
        ckpt, "", &text, &layout, &sigmas, active, 1, 0, 0, 1.0f,
        0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, NULL, NULL, error, sizeof(error));
    if (!dit) {
        fprintf(stderr, "h3_dit_load_t2va: %s\n", error);
        return 1;
    }
    const size_t ve = h3_dit_video_elements(dit);
    const size_t ae = h3_dit_audio_elements(dit);
    float *video = malloc(ve * sizeof(float));
    float *audio = malloc(ae * sizeof(float));
    float *video_v = malloc(ve * sizeof(float));
    float *audio_v = malloc(ae * sizeof(float));
    float *rows_v = malloc(ve * sizeof(float));
    float *rows_a = malloc(ae * sizeof(float));
    if (!video || !audio || !video_v || !audio_v || !rows_v || !rows_a) {
        fprintf(stderr, "out of memory\n");
        return 1;
    }
    h3_rng rng;
    h3_rng_seed(&rng, seed);
    h3_rng_fill_normal(&rng, video, ve);
    h3_rng_fill_normal(&rng, audio, ae);
    if (!h3_dit_forward(dit, step, video, audio, video_v, audio_v, error,
                        sizeof(error))) {
        fprintf(stderr, "h3_dit_forward: %s\n", error);
        return 1;
    }
    int ok =
        h3_dit_patchify_video(video, 24, spec.latent_t, spec.latent_h,
                              spec.latent_w, rows_v, ve) &&
        h3_dit_pack_audio(audio, 32, spec.audio_t, rows_a, ae) &&
        write_file(out_dir, "video_rows.f32", rows_v, ve * sizeof(float)) &&
        write_file(out_dir, "audio_rows.f32", rows_a, ae * sizeof(float)) &&
        h3_dit_patchify_video(video_v, 24, spec.latent_t, spec.latent_h,
                              spec.latent_w, rows_v, ve) &&
        h3_dit_pack_audio(audio_v, 32, spec.audio_t, rows_a, ae) &&
        write_file(out_dir, "video_velocity.f32", rows_v,
                   ve * sizeof(float)) &&
        write_file(out_dir, "audio_velocity.f32", rows_a, ae * sizeof(float));
    if (!ok) {
        fprintf(stderr, "cannot write the outputs to %s\n", out_dir);
        return 1;
    }
    h3_gpu_stats stats;
    if (h3_dit_get_gpu_stats(dit, &stats))
        printf("engine: %llu tensors, %.3f GiB allocated, %llu SDPA, "
               "%llu linear dispatches\n",
               (unsigned long long)stats.tensor_allocations,
               (double)stats.allocated_bytes / (1024.0 * 1024.0 * 1024.0),
               (unsigned long long)stats.mps_sdpa_dispatches,
               (unsigned long long)stats.mps_linear_dispatches);
    printf("engine forward ok: %zu video, %zu audio elements\n", ve, ae);
    h3_dit_free(dit);
    h3_layout_free(&layout);
    free(text_values);
    free(video); free(audio); free(video_v); free(audio_v);
    free(rows_v); free(rows_a);
    return 0;
}
