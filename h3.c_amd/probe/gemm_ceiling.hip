/* gemm_ceiling: what the GEMM main loop can reach on this GPU, piece by
 * piece.  One workgroup of four waves per CU (256 workgroups), each wave
 * running the main loop of hk_gemm_mfma's 128 x 128 wave tile (4 x 4
 * v_mfma_f32_32x32x16_bf16 accumulators per 16-wide K substep, four
 * substeps per 64-wide K stage) on operands that are never refreshed from
 * memory, and adding one ingredient at a time:
 *
 *   mfma            the 16 MFMAs per substep alone
 *   lds             + the 8 ds_read_b128 fragment reads per substep into the
 *                     other register buffer, one per two MFMAs, with the
 *                     GEMM's XOR swizzle (conflict-free)
 *   lds_early       + the same reads issued over the first 8 MFMAs
 *   lds_unswizzled  + the reads without the swizzle (32 rows of one 16-byte
 *                     column: bank conflicts)
 *   barrier         lds + one workgroup barrier per stage
 *   dma             barrier + the 16 direct-to-LDS 16-byte loads per wave
 *                     and stage (from a 4 MiB buffer that stays in L2) and
 *                     their vmcnt wait
 *
 * Each line prints the rate against the flops issued, the shader clock
 * (s_memtime against the 100 MHz s_memrealtime) and cycles per substep (512
 * is the MFMA issue bound). */
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef int i4v __attribute__((ext_vector_type(4)));

enum { MFMA, LDS, LDS_EARLY, LDS_UNSWIZZLED, BARRIER, DMA };

template <int MODE>
__global__ void __launch_bounds__(256, 1)
__attribute__((amdgpu_waves_per_eu(1, 1)))
ceiling(float *buf, int iters, unsigned long long *clk) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 65536 / 4; i += 256)
        ((uint32_t *)sm)[i] = i * 2654435761u;
    __syncthreads();
    i4v fw[2][4], fx[2][4];
    for (int b = 0; b < 2; b++)
        for (int i = 0; i < 4; i++) {
            fw[b][i] = i4v{lane + i, 1, 2, 3};
            fx[b][i] = i4v{lane * 3 + i, 5, 6, 7};
        }
    const uint32_t row = lane & 31;
    const uint32_t key = (row & 7) ^ ((row >> 3) & 1);
    uint32_t choff[4];
    for (int ks = 0; ks < 4; ks++)
        choff[ks] = MODE == LDS_UNSWIZZLED
                        ? (ks * 2 + (lane >> 5)) << 4
                        : ((ks * 2 + (lane >> 5)) ^ key) << 4;
    const uint32_t lds0 =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)sm;
    const uint32_t wa = lds0 + (wave & 1) * 16384 + row * 128;
    const uint32_t xa = lds0 + 32768 + (wave >> 1) * 16384 + row * 128;
    f16v acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)buf, (short)0, 4 << 20, 0x00020000);
    const uint32_t gofs = ((blockIdx.x * 256 + threadIdx.x) * 16) & ((4 << 20) - 1);
    bool dma = false;
    auto issue_load = [&](int j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs,
            (__attribute__((address_space(3))) void *)(sm + 65536 +
                                                       (wave * 16 + j) * 1024),
            16, gofs, (j * 65536) & ((4 << 20) - 1), 0, 0);
    };
    auto read_one = [&](int b, int idx, int ks) {
        if (idx < 4)
            asm volatile("ds_read_b128 %0, %1 offset:%2"
                         : "=&v"(fw[b][idx])
                         : "v"(wa + choff[ks]), "i"(idx * 4096));
        else
            asm volatile("ds_read_b128 %0, %1 offset:%2"
                         : "=&v"(fx[b][idx - 4])
                         : "v"(xa + choff[ks]), "i"((idx - 4) * 4096));
    };
    auto wait_frags = [&](int b) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(fw[b][0]), "+v"(fw[b][1]), "+v"(fw[b][2]),
                       "+v"(fw[b][3]), "+v"(fx[b][0]), "+v"(fx[b][1]),
                       "+v"(fx[b][2]), "+v"(fx[b][3]));
    };
    auto substep = [&](int b, int ks) {
#pragma unroll
        for (int t = 0; t < 16; t++) {
            acc[t >> 2][t & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf8, fw[b][t >> 2]),
                __builtin_bit_cast(bf8, fx[b][t & 3]), acc[t >> 2][t & 3], 0,
                0, 0);
            if (MODE == LDS_EARLY) {
                if (t < 8) read_one(b ^ 1, t, ks);
            } else if (MODE != MFMA && (t & 1)) {
                read_one(b ^ 1, t >> 1, ks);
            }
            if (MODE == DMA && dma && (t & 1)) issue_load(t >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (MODE != MFMA) wait_frags(b ^ 1);
    };
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; it++) {
        dma = true;
        substep(0, 1);
        dma = false;
        substep(1, 2);
        substep(0, 3);
        if (MODE == DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (MODE >= BARRIER) __syncthreads();
        dma = true;
        substep(1, 0);
    }
    float s = 0;
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int r = 0; r < 16; r++) s += acc[i][j][r];
    buf[blockIdx.x * 256 + threadIdx.x] = s;
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        clk[blockIdx.x * 2] = c1 - c0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

template <int MODE>
static void run(const char *name, float *buf, unsigned long long *clk) {
    const int iters = 5000, reps = 10, lds = 131072;
    (void)hipFuncSetAttribute((const void *)ceiling<MODE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(ceiling<MODE>, dim3(256), dim3(256), lds, 0, buf, iters,
                       clk);
    (void)hipDeviceSynchronize();
    (void)hipEventRecord(e0);
    for (int r = 0; r < reps; r++)
        hipLaunchKernelGGL(ceiling<MODE>, dim3(256), dim3(256), lds, 0, buf,
                           iters, clk);
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    const double flops = (double)reps * 256 * 4 * iters * 4 * 16 * 32768.0;
    unsigned long long h[512];
    (void)hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
    double cycles = 0, real = 0;
    for (int i = 0; i < 256; i++) {
        cycles += h[2 * i];
        real += h[2 * i + 1];
    }
    printf("%-16s %7.1f TFLOP/s  clock %.2f GHz  cycles/substep %.0f\n", name,
           flops / ms / 1e9, cycles / real * 0.1,
           cycles / 256 / (iters * 4.0));
    fflush(stdout);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
}

int main() {
    float *buf = NULL;
    unsigned long long *clk = NULL;
    if (hipMalloc(&buf, 4 << 20) != hipSuccess ||
        hipMalloc(&clk, 512 * sizeof(unsigned long long)) != hipSuccess ||
        hipMemset(buf, 0, 4 << 20) != hipSuccess) {
        fprintf(stderr, "allocation failed\n");
        return 1;
    }
    for (int pass = 0; pass < 3; pass++) {
        run<MFMA>("mfma", buf, clk);
        run<LDS>("lds", buf, clk);
        run<LDS_EARLY>("lds_early", buf, clk);
        run<LDS_UNSWIZZLED>("lds_unswizzled", buf, clk);
        run<BARRIER>("barrier", buf, clk);
        run<DMA>("dma", buf, clk);
    }
    return 0;
}
