/* gemm_ceiling_wide: the main loop of a wider wave tile, for comparison with
 * gemm_ceiling's 128 x 128 tile.  Each wave owns 128 (W) x 192 (X) outputs:
 * 4 x 6 v_mfma_f32_32x32x16_bf16 accumulators (384 f32 per lane; 16 in the
 * AGPRs, 8 in VGPRs, through inline-asm MFMAs that pin each to its file), so
 * a 16-wide K substep runs 24 MFMAs on 10 fragment reads instead of 16 on 8
 * (a sixth fewer LDS bytes per flop).  Operands are never refreshed from
 * memory, as in gemm_ceiling:
 *
 *   mfma  the 24 MFMAs per substep alone (768 cycles is the issue bound)
 *   lds   + the 10 swizzled ds_read_b128 fragment reads per substep, one per
 *           two MFMAs, and one workgroup barrier per 64-wide K stage
 *   dma   lds + the 20 direct-to-LDS 16-byte loads per wave and stage
 *           (a 256 x 384 workgroup tile, L2-resident) and their vmcnt wait
 *
 * Each line prints the rate against the flops issued, the shader clock
 * (s_memtime against the 100 MHz s_memrealtime) and cycles per substep. */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));
enum { MFMA, LDS, DMA };

#define MF_A(acc, a, b) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b))
#define MF_V(acc, a, b) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b))

template <int MODE>
__global__ void __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
wide(float *buf, int iters, unsigned long long *clk) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 81920 / 4; i += 256) ((uint32_t *)sm)[i] = i * 2654435761u;
    __syncthreads();
    i4v fw[2][4], fx[2][6];
    for (int b = 0; b < 2; b++) {
        for (int i = 0; i < 4; i++) fw[b][i] = i4v{lane + i, 1, 2, 3};
        for (int i = 0; i < 6; i++) fx[b][i] = i4v{lane * 3 + i, 5, 6, 7};
    }
    const uint32_t row = lane & 31;
    const uint32_t key = (row & 7) ^ ((row >> 3) & 1);
    uint32_t choff[4];
    for (int ks = 0; ks < 4; ks++) choff[ks] = ((ks * 2 + (lane >> 5)) ^ key) << 4;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)sm;
    const uint32_t wa = lds0 + (wave & 1) * 16384 + row * 128;
    const uint32_t xa = lds0 + 32768 + (wave >> 1) * 24576 + row * 128;
    f16v a00 = {}, a01 = {}, a02 = {}, a03 = {}, a10 = {}, a11 = {}, a12 = {}, a13 = {},
         a20 = {}, a21 = {}, a22 = {}, a23 = {}, a30 = {}, a31 = {}, a32 = {}, a33 = {};
    f16v v0 = {}, v1 = {}, v2 = {}, v3 = {}, v4 = {}, v5 = {}, v6 = {}, v7 = {};
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)buf, (short)0, 4 << 20, 0x00020000);
    const uint32_t gofs = ((blockIdx.x * 256 + threadIdx.x) * 16) & ((4 << 20) - 1);
    bool dma = false;
    auto issue_load = [&](int j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(sm + 81920 + (wave * 20 + j) * 1024),
                                                 16, gofs, (j * 65536) & ((4 << 20) - 1), 0, 0);
    };
    auto read_one = [&](int b, int idx, int ks) {
        if (idx < 4)
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(fw[b][idx]) : "v"(wa + choff[ks]), "i"(idx * 4096));
        else
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(fx[b][idx - 4]) : "v"(xa + choff[ks]), "i"((idx - 4) * 4096));
    };
    auto wait_frags = [&](int b) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fw[b][0]), "+v"(fw[b][1]), "+v"(fw[b][2]), "+v"(fw[b][3]),
                     "+v"(fx[b][0]), "+v"(fx[b][1]), "+v"(fx[b][2]), "+v"(fx[b][3]), "+v"(fx[b][4]), "+v"(fx[b][5]));
    };
    auto substep = [&](int b, int ks) {
        // 24 MFMAs; 10 reads (slots 1,3,...,19 -> reads 0..9); 20 DMA loads per stage spread over two substeps
        int t = 0;
#define STEP(ACCM, acc, i, j)                                               \
        ACCM(acc, fw[b][i], fx[b][j]);                                      \
        if (MODE != MFMA && (t & 1) && (t >> 1) < 10) read_one(b ^ 1, t >> 1, ks); \
        if (MODE == DMA && dma && (t & 1) && (t >> 1) < 10) issue_load(t >> 1 ); \
        t++;
        STEP(MF_A, a00, 0, 0) STEP(MF_A, a01, 0, 1) STEP(MF_A, a02, 0, 2) STEP(MF_A, a03, 0, 3)
        STEP(MF_V, v0, 0, 4) STEP(MF_V, v1, 0, 5)
        STEP(MF_A, a10, 1, 0) STEP(MF_A, a11, 1, 1) STEP(MF_A, a12, 1, 2) STEP(MF_A, a13, 1, 3)
        STEP(MF_V, v2, 1, 4) STEP(MF_V, v3, 1, 5)
        STEP(MF_A, a20, 2, 0) STEP(MF_A, a21, 2, 1) STEP(MF_A, a22, 2, 2) STEP(MF_A, a23, 2, 3)
        STEP(MF_V, v4, 2, 4) STEP(MF_V, v5, 2, 5)
        STEP(MF_A, a30, 3, 0) STEP(MF_A, a31, 3, 1) STEP(MF_A, a32, 3, 2) STEP(MF_A, a33, 3, 3)
        STEP(MF_V, v6, 3, 4) STEP(MF_V, v7, 3, 5)
        if (MODE != MFMA) wait_frags(b ^ 1);
    };
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
        dma = true; substep(0, 1);
        dma = false; substep(1, 2);
        substep(0, 3);
        if (MODE == DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (MODE != MFMA) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        dma = true; substep(1, 0);
    }
    f16v s = a00 + a01 + a02 + a03 + a10 + a11 + a12 + a13 + a20 + a21 + a22 + a23 + a30 + a31 + a32 + a33 +
             v0 + v1 + v2 + v3 + v4 + v5 + v6 + v7;
    float t = 0;
    for (int r = 0; r < 16; r++) t += s[r];
    buf[blockIdx.x * 256 + threadIdx.x] = t;
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) { clk[blockIdx.x * 2] = c1 - c0; clk[blockIdx.x * 2 + 1] = r1 - r0; }
}

template <int MODE>
static void run(const char *name, float *buf, unsigned long long *clk) {
    const int iters = 4000, reps = 10, lds = 81920 + 4 * 20 * 1024;
    (void)hipFuncSetAttribute((const void *)wide<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(wide<MODE>, dim3(256), dim3(256), lds, 0, buf, iters, clk);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(e0);
    for (int r = 0; r < reps; r++) hipLaunchKernelGGL(wide<MODE>, dim3(256), dim3(256), lds, 0, buf, iters, clk);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms = 0; (void)hipEventElapsedTime(&ms, e0, e1);
    const double flops = (double)reps * 256 * 4 * iters * 4 * 24 * 32768.0;
    unsigned long long h[512];
    (void)hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
    double cycles = 0, real = 0;
    for (int i = 0; i < 256; i++) { cycles += h[2 * i]; real += h[2 * i + 1]; }
    printf("%-8s %7.1f TFLOP/s  clock %.2f GHz  cycles/substep %.0f (bound 768)\n", name, flops / ms / 1e9,
           cycles / real * 0.1, cycles / 256 / (iters * 4.0));
    fflush(stdout);
}
int main() {
    float *buf = NULL; unsigned long long *clk = NULL;
    if (hipMalloc(&buf, 4 << 20) != hipSuccess || hipMalloc(&clk, 4096) != hipSuccess || hipMemset(buf, 0, 4 << 20) != hipSuccess) return 1;
    for (int pass = 0; pass < 3; pass++) { run<MFMA>("mfma", buf, clk); run<LDS>("lds", buf, clk); run<DMA>("dma", buf, clk); }
    return 0;
}
