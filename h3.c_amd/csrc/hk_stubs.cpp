/* Entry points of h3_gpu.h that lie outside the DiT denoiser path (VAE,
 * audio, vision and text-encoder ops) and the Apple-only int8/NAX paths.
 * They exist so that the engine's model layer links against this backend;
 * each returns 0 with a clear message, like the reference's permanent stubs
 * (h3_cuda_dit.cu:1076-1216).  The capability probes report 0 for NAX and
 * int8, so the DiT model layer never selects the int8/NAX entries. */
#include "hk_internal.h"

#define HK_STUB(name, ...)                                                   \
    extern "C" int name(h3_gpu *gpu, __VA_ARGS__) {                          \
        return hk_fail(gpu, #name " is not implemented on the HIP backend"); \
    }

/* The Apple-only int8 / NAX paths: the reference's CUDA backend rejects
 * them with "... requires Metal 4 TensorOps and is not available in the CUDA
 * backend" (h3_cuda_dit.cu:1076-1216), which callers and the reference's
 * tests (tests/test_cuda_dit.c:771-815) match on. */
#define HK_METAL_STUB(name, ...)                                             \
    extern "C" int name(h3_gpu *gpu, __VA_ARGS__) {                          \
        return hk_fail(gpu, #name " requires Metal 4 TensorOps: not "        \
                            "available in the CUDA backend nor in this HIP " \
                            "backend");                                      \
    }

typedef h3_gpu_tensor T;
typedef const h3_gpu_tensor CT;

HK_STUB(h3_gpu_sdpa_f32, T *, CT *, CT *, CT *, uint32_t, uint32_t, uint32_t,
        float)
HK_STUB(h3_gpu_video_qkv_rope_f32, T *, T *, T *, CT *, CT *, CT *, uint32_t,
        uint32_t, uint32_t, uint32_t, float)
HK_STUB(h3_gpu_conv1d_f32, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_conv1d_stride_f32, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_conv_transpose1d_f32, T *, CT *, CT *, CT *, uint32_t,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_alias_free_snake_f32, T *, CT *, CT *, CT *, CT *, CT *,
        uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_snake1d_f32, T *, CT *, CT *, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_audio_qkv_split_f32, T *, T *, T *, CT *, CT *, CT *, CT *,
        uint32_t, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_sdpa_causal_f32, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, float)
HK_STUB(h3_gpu_audio_attention_pool_f32, T *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_vae_encoder_pad_f32, T *, CT *, uint32_t, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_conv3d_f32, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
        uint32_t, uint32_t, uint32_t)
HK_STUB(h3_gpu_vae_encoder_group_norm_silu_f32, T *, CT *, CT *, CT *,
        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, float)
HK_METAL_STUB(h3_gpu_mlp_nax_bf16, T *, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t)
HK_METAL_STUB(h3_gpu_quantize_weight_int8, T *, T *, CT *, uint32_t, uint32_t)
HK_METAL_STUB(h3_gpu_linear_int8_bf16, T *, T *, T *, CT *, CT *, CT *, uint32_t,
        uint32_t, uint32_t, int)
HK_METAL_STUB(h3_gpu_linear_int8_head_major_bf16, T *, T *, T *, CT *, CT *, CT *,
        uint32_t, uint32_t, uint32_t, uint32_t)
HK_METAL_STUB(h3_gpu_mlp_int8_bf16, T *, T *, T *, T *, CT *, CT *, CT *, CT *,
        CT *, CT *, CT *, uint32_t, uint32_t, uint32_t, uint32_t, int, int,
        int, int)
HK_STUB(h3_gpu_vision_qkv_rope_bf16, T *, T *, T *, CT *, CT *, CT *,
        uint32_t, uint32_t, uint32_t, uint32_t)
HK_METAL_STUB(h3_gpu_gate_adaln_quantize_int8, T *, T *, T *, CT *, CT *, CT *,
        CT *, CT *, CT *, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
        uint32_t, uint32_t, float)
HK_METAL_STUB(h3_gpu_grouped_qkv_linear_rope_int8, T *, T *, T *, T *, T *, CT *,
        CT *, CT *, CT *, CT *, CT *, CT *, uint32_t, uint32_t, uint32_t,
        uint32_t, uint32_t, float, int, int, int, int)
HK_STUB(h3_gpu_text_qk_rope_bf16, T *, T *, CT *, CT *, CT *, CT *, CT *,
        CT *, uint32_t, uint32_t, uint32_t, uint32_t, float)
HK_STUB(h3_gpu_rope_text_bf16, T *, T *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t)
HK_STUB(h3_gpu_gqa_causal_bf16, T *, CT *, CT *, CT *, uint32_t, uint32_t,
        uint32_t, uint32_t, float)
