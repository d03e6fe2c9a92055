/* Device helpers shared by the gfx950 kernels: bf16 <-> f32, 16-byte vector
 * access, wave64 and workgroup reductions. */
#ifndef HK_COMMON_H
#define HK_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 hk_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 hk_bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 hk_bf16x2 __attribute__((ext_vector_type(2)));
typedef float hk_f32x16 __attribute__((ext_vector_type(16)));
typedef float hk_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t hk_u32x4 __attribute__((ext_vector_type(4)));

/* Exact widening: bf16 bits are the top half of the f32 bits. */
__device__ __forceinline__ float hk_bf2f(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

/* Round-to-nearest-even narrowing (v_cvt_pk_bf16_f32 on gfx950). */
__device__ __forceinline__ uint16_t hk_f2bf(float value) {
    return __builtin_bit_cast(uint16_t, (__bf16)value);
}

__device__ __forceinline__ uint32_t hk_pack2(float lo, float hi) {
    hk_bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

/* 8 bf16 in a uint4 -> 8 floats and back. */
__device__ __forceinline__ void hk_unpack8(uint4 v, float *out) {
    out[0] = __uint_as_float(v.x << 16);
    out[1] = __uint_as_float(v.x & 0xffff0000u);
    out[2] = __uint_as_float(v.y << 16);
    out[3] = __uint_as_float(v.y & 0xffff0000u);
    out[4] = __uint_as_float(v.z << 16);
    out[5] = __uint_as_float(v.z & 0xffff0000u);
    out[6] = __uint_as_float(v.w << 16);
    out[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 hk_pack8(const float *in) {
    uint4 v;
    v.x = hk_pack2(in[0], in[1]);
    v.y = hk_pack2(in[2], in[3]);
    v.z = hk_pack2(in[4], in[5]);
    v.w = hk_pack2(in[6], in[7]);
    return v;
}

__device__ __forceinline__ float hk_wave_sum(float value) {
#pragma unroll
    for (int offset = 32; offset; offset >>= 1)
        value += __shfl_xor(value, offset, 64);
    return value;
}

__device__ __forceinline__ float hk_wave_max(float value) {
#pragma unroll
    for (int offset = 32; offset; offset >>= 1)
        value = fmaxf(value, __shfl_xor(value, offset, 64));
    return value;
}

/* Sum over the whole workgroup (blockDim.x a multiple of 64, <= 1024).
 * scratch must hold 16 floats.  Every thread receives the total. */
__device__ __forceinline__ float hk_block_sum(float value, float *scratch) {
    value = hk_wave_sum(value);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    __syncthreads(); /* scratch may still be read by a previous call */
    if (lane == 0) scratch[wave] = value;
    __syncthreads();
    float total = 0.0f;
    for (int w = 0; w < waves; w++) total += scratch[w];
    return total;
}

#endif
