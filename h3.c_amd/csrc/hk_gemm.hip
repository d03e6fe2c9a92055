/* BF16 GEMM for gfx950: C[M,N] = epilogue(X[M,K] . W[N,K]^T (+ bias)).
 *
 * Both operands are K-contiguous (activations row-major, weights in the
 * checkpoint's [out, in] order), which is the natural operand order of the
 * CDNA matrix cores: every MFMA operand fragment is 8 consecutive k values
 * of one row, i.e. one 16-byte LDS read per lane.
 *
 * Tiling (per 256-thread workgroup, one workgroup per CU at a time):
 *   - 256 (W rows) x 256 (X rows) output tile, K step 64;
 *   - four wave64s in a 2x2 grid, each owning a 128x128 sub-tile held as
 *     8x8 accumulators of v_mfma_f32_16x16x32_bf16 (256 f32 per lane; the
 *     kernel body is in hk_gemm_kernel.inc);
 *   - X and W tiles staged into two LDS stages by direct-to-LDS buffer
 *     loads (16 B per lane; rows past M read as zero through the buffer
 *     bound).  Once every wave holds a stage's fragments in registers, the
 *     loads of the stage after next (K step k+2) go into it, spread over
 *     that stage's last 32-deep step, so each load has a step to a step
 *     and a half to land;
 *   - that is too short for lines that come from HBM, and in the forward
 *     both operands do (weights are read once per forward, activations
 *     were stored nontemporally), so the K loop also prefetches into L2
 *     the lines HK_GEMM_PF stages further on (4-byte loads, the lines
 *     split among the tiles that share them);
 *   - LDS rows are 128 B (64 bf16); 16-byte chunks are XOR-swizzled with the
 *     row index so that the 16 (or 32) rows a fragment read touches fall on
 *     distinct banks;
 *   - the MFMA computes D = W_tile . X_tile^T, so each lane's accumulator
 *     holds 4 consecutive output columns of one output row: the epilogue
 *     packs them into 8-byte bf16 groups in LDS and stores the tile as
 *     whole rows, 16 bytes per lane;
 *   - the workgroup -> tile order is XCD-aware: consecutive workgroups are
 *     dealt round-robin to the 8 XCDs, so workgroup ids are first regrouped
 *     per XCD and then walked in GROUP_M-tall column bands, keeping the
 *     tiles that share W (and X) rows inside one XCD's L2.
 *
 * Epilogues: plain store (+bias), SwiGLU (the tile's W rows interleave 64
 * gate and 64 up rows per wave so each lane holds matching gate/up values;
 * activation bf16(silu(bf16 g) * bf16 u), the reference's rounding,
 * h3_cuda_core.cu:104-114 fed by a bf16 fc1 output, :1067-1104), GELU-tanh,
 * and the split-K pieces' F32 partial tiles, which hk_splitk_reduce sums
 * before the bias and activation.
 *
 * A sequential-k reference kernel (one thread per output, fmaf from the
 * bias, bf16 inputs: the reference's hand kernel h3_cuda_core.cu:358-371)
 * serves shapes the MFMA path does not take and H3_HIP_REFERENCE=1.
 */
#include "hk_common.h"
#include "hk_internal.h"

#include <pthread.h>
#include <string.h>

#include <math.h>
#include <stdlib.h>

#define HK_BM 256
#define HK_BN 256
#define HK_BK 64
#define HK_STAGES 2
#define HK_GEMM_THREADS 256
#define HK_TILE_BYTES (HK_BM * HK_BK * 2)       /* 32 KiB per operand */
#define HK_STAGE_BYTES (2 * HK_TILE_BYTES)      /* X tile then W tile */
/* L2 prefetch distance of the 16x16x32 kernel's K loop, in 64-deep
 * stages past the stage loads' k step */
#define HK_GEMM_PF 2
/* + 256 bytes that the L2 prefetch loads write and nothing reads */
#define HK_GEMM_LDS (HK_STAGES * HK_STAGE_BYTES + 256) /* 128 KiB + 256 */
#define HK_GROUP_M 8

typedef int hk_v4i __attribute__((ext_vector_type(4)));
typedef int hk_v2i __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t hk_rsrc(const void *base,
                                                          uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base),
                                             (short)0, (int)bytes,
                                             0x00020000);
}

/* LDS rows are 128 B (64 bf16 = 8 chunks of 16 B); logical chunk c of row
 * r lives at physical chunk c ^ key(r).  Any 8 consecutive rows get
 * distinct keys (32-bank view, 128 B per cycle) and any 16 consecutive rows
 * distinct (r & 1, key) pairs (64-bank view, 256 B per cycle), so the
 * 32-row fragment reads are conflict-free under either bank model. */
__device__ __forceinline__ uint32_t hk_swz_key(uint32_t row) {
    return (row & 7u) ^ ((row >> 3) & 1u);
}

/* Epilogue activations from the hardware exp2/rcp (v_exp_f32, v_rcp_f32,
 * about 1 ulp each), far below half a bf16 ulp, the rounding applied right
 * after.  silu(x) = x / (1 + e^-x).  The reference's tanh-form GELU
 * (h3_cuda_core.cu:139-158), 0.5 x (1 + tanh u) with
 * u = sqrt(2/pi) (x + 0.044715 x^3), is evaluated as x - x r with
 * r = 1 / (e^(2u) + 1) and e^(2u) = 2^(x (A + B x^2)): five VALU ops and
 * two transcendentals.  Its +-10 saturation needs no branch for finite x
 * (u <= -10 gives 1 + e^(2u) == 1, so r == 1 and x - x r == 0; u >= 10
 * gives |x r| below half an ulp of x); the clamps keep +-inf exact. */
__device__ __forceinline__ float hk_exp_fast(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

__device__ __forceinline__ float hk_silu_f(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + hk_exp_fast(-x));
}

__device__ __forceinline__ float hk_gelu_tanh_f(float x) {
    /* A = 2 log2(e) sqrt(2/pi), B = 0.044715 A; v = 2 u log2(e) */
    const float A = 2.302208198144325f, B = 0.1029432395800235f;
    const float v = x * __builtin_fmaf(x * x, B, A);
    const float r =
        __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(v) + 1.0f);
    const float g = __builtin_fmaf(-x, r, x);
    /* u = +-10 */
    return v <= -28.853900817779268f ? 0.0f
         : v >= 28.853900817779268f  ? x
                                     : g;
}

struct hk_gemm_args {
    const uint16_t *x;     /* [M, K] */
    const uint16_t *w;     /* [W rows, K] */
    const uint16_t *bias;  /* [N] or null */
    uint16_t *c;           /* [M, N] */
    uint32_t m, n, k;      /* n = output columns */
    uint32_t tiles_m, tiles_n;
    uint32_t x_bytes, w_bytes;
    /* split-K (EPI == HK_EPI_PARTIAL only): workgroup pid covers tile
     * tile_base + pid % part_tiles over K steps [split * split_steps,
     * +split_steps), split = pid / part_tiles, and writes the F32 tile to
     * partial[split][pid % part_tiles][256][256] */
    float *partial;
    uint32_t split_steps, tile_base, part_tiles;
    /* tiles [0, tile_count) of the launch, dealt to the workgroups in
     * rounds of gridDim.x (one round when the grid covers them all) */
    uint32_t tile_count;
    /* split-K over two problems of one shape and one X (EPI_PARTIAL):
     * parts [pair_tiles, 2 pair_tiles) use w1 / bias1 / c1; 0 = one
     * problem */
    uint32_t pair_tiles;
    const uint16_t *w1, *bias1;
    uint16_t *c1;
    /* a group of problems of one shape and one X (the GROUP kernel): tile
     * t is tile t % group_tiles of problem t / group_tiles, whose W, bias
     * and C are group[3 p], group[3 p + 1], group[3 p + 2] */
    uint32_t group_tiles;
    const uint64_t *group;
};

/* A word of the GROUP kernel's problem table, read with a uniform index:
 * marked uniform so that the buffer resources built from it stay in
 * scalar registers (a table load otherwise counts as divergent, and every
 * buffer load would become a loop over the lanes' descriptors). */
__device__ __forceinline__ uint64_t hk_group_word(const uint64_t *table,
                                                  uint32_t index) {
    const uint64_t v = table[index];
    /* readfirstlane returns int: widen through uint32_t, not sign-extend */
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi =
        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

/* Tile index -> (tile_m, tile_n): column bands of HK_GROUP_M row tiles, so
 * consecutive tiles share W rows (and, band by band, X rows). */
__device__ __forceinline__ void hk_tile_coords(uint32_t tile, uint32_t tiles_m,
                                               uint32_t tiles_n,
                                               uint32_t &tile_m,
                                               uint32_t &tile_n) {
    const uint32_t band = HK_GROUP_M * tiles_n;
    const uint32_t first_m = (tile / band) * HK_GROUP_M;
    const uint32_t band_rows = min(tiles_m - first_m, (uint32_t)HK_GROUP_M);
    const uint32_t in_band = tile % band;
    tile_m = first_m + in_band % band_rows;
    tile_n = in_band / band_rows;
}

/* Phase trace of the MFMA GEMM (built only with -DHK_GEMM_TRACE, the
 * `make trace` library; the product build compiles none of it).  Thread 0
 * of each workgroup records the constant 100 MHz real-time counter at the
 * phase boundaries of each of its tiles, and the shader-clock counter at a
 * tile's start and end:
 *   0 tile start          1 first stage landed (prologue done)
 *   2 main loop done      3 bias loaded, LDS free (epilogue start)
 *   4 tile staged in LDS  5 global stores issued
 *   6 tile end (LDS reads done, barrier)
 *   7 the tile's index in the launch
 *   8 / 9 shader clock at 0 / 6
 *   10 shader cycles wave 0 spent in the K loop's stage waits (its DMA
 *      loads, then the barrier), summed over the tile's K steps
 *   11 shader cycles wave 0 spent waiting for fragment reads in the K loop
 *   (10 and 11 only with -DHK_GEMM_TRACE_STALLS as well: the clock reads
 *   inside the loop wait for their results and slow the 16x16x32 loop by
 *   about a third, so the default trace build leaves them out)
 * h3_hip_gemm_trace_clear / _read (trace build only) reset and fetch it. */
#ifdef HK_GEMM_TRACE
#define HK_TRACE_WG 1024u
#define HK_TRACE_ITERS 16u
#define HK_TRACE_SLOTS 12u
static __device__ uint64_t
    hk_gemm_trace[HK_TRACE_WG * HK_TRACE_ITERS * HK_TRACE_SLOTS];
/* Branch-free: every lane stores, through a buffer resource, and all but
 * thread 0 of the workgroup get an offset past the end, which the hardware
 * drops.  A divergent branch here changed the shape of the kernel's tile
 * loop enough for the register allocator to rotate the 16x16 accumulators
 * through copies inside the K loop. */
__device__ __forceinline__ void hk_trace_put(uint32_t iter, uint32_t slot,
                                             uint64_t value) {
    const __amdgpu_buffer_rsrc_t r =
        hk_rsrc(hk_gemm_trace, (uint32_t)sizeof(hk_gemm_trace));
    const bool mine = threadIdx.x == 0 && blockIdx.x < HK_TRACE_WG &&
                      iter < HK_TRACE_ITERS;
    const uint32_t off =
        mine ? ((blockIdx.x * HK_TRACE_ITERS + iter) * HK_TRACE_SLOTS + slot) *
                   8u
             : 0xfffffff0u;
    const hk_v2i v = {(int)(uint32_t)value, (int)(uint32_t)(value >> 32)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}
#define HK_TRACE(p) \
    hk_trace_put((item - slot) / nwg, (p), __builtin_amdgcn_s_memrealtime())
#define HK_TRACE_CLOCK(p) \
    hk_trace_put((item - slot) / nwg, (p), __builtin_amdgcn_s_memtime())
#define HK_TRACE_VALUE(p, v) hk_trace_put((item - slot) / nwg, (p), (v))
#define HK_CYCLES() __builtin_amdgcn_s_memtime()
#else
#define HK_TRACE(p) ((void)0)
#define HK_TRACE_CLOCK(p) ((void)0)
#define HK_TRACE_VALUE(p, v) ((void)0)
#define HK_CYCLES() 0ull
#endif

/* The MFMA shape of the main loop: v_mfma_f32_16x16x32_bf16 for every
 * launch, full tiles and split-K pieces.  At the same 1400 W it runs the
 * GEMM at a higher clock than 32x32x16 (less register-file traffic per
 * flop).  -DHK_MFMA32 builds the kernel with 32x32x16 (4x4 blocks) instead,
 * for comparison. */
#define HK_KERNEL_NAME hk_gemm_mfma
#ifdef HK_MFMA32
#define HK_KERNEL_MFMA16 0
#else
#define HK_KERNEL_MFMA16 1
#endif
#include "hk_gemm_kernel.inc"
#undef HK_KERNEL_NAME
#undef HK_KERNEL_MFMA16

#ifdef HK_GEMM_TRACE
extern "C" int h3_hip_gemm_trace_clear(void) {
    static uint64_t zeros[HK_TRACE_WG * HK_TRACE_ITERS * HK_TRACE_SLOTS];
    return hipMemcpyToSymbol(HIP_SYMBOL(hk_gemm_trace), zeros,
                             sizeof(zeros)) == hipSuccess;
}

/* copies the trace, [workgroup][tile iteration][slot] u64, to `out`
 * (HK_TRACE_WG x HK_TRACE_ITERS x HK_TRACE_SLOTS entries) */
extern "C" int h3_hip_gemm_trace_read(uint64_t *out, size_t entries) {
    if (entries < (size_t)HK_TRACE_WG * HK_TRACE_ITERS * HK_TRACE_SLOTS)
        return 0;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(hk_gemm_trace),
                               sizeof(hk_gemm_trace)) == hipSuccess;
}
#endif

/* Skinny GEMM for M <= 64 rows (the per-block modulation projections:
 * time rows x 2688 against 96768 x 2688 weights).  Bound by streaming W
 * from HBM once, and W is never re-read: each wave owns 32 W rows (output
 * columns) and loads them into registers D - 1 64-wide k steps ahead of
 * the MFMAs, as whole 128-byte lines (a load gives lane l chunk l % 8 of
 * row 8 q + l / 8: eight rows per load, where loading the MFMA fragments
 * directly touches 32 partial rows per load and runs into the cache-line
 * request rate, 27% slower).  The lines go through the wave's own 4-KiB
 * LDS buffer (row-major, the big GEMM's chunk swizzle) and come back out
 * as MFMA fragments.  X (MB x 32 rows) is shared by the workgroup's four
 * waves:
 * one DMA load per thread and step stages it into LDS (double-buffered,
 * 128-byte rows with the 16-byte-chunk swizzle of the big GEMM), so L2
 * serves it once per workgroup instead of once per wave.  The step's k
 * offset goes in the buffer's scalar offset; rows past M or N keep a lane
 * offset beyond the buffer and read zeros.
 *
 * Ordering: the prologue issues W(0), W(1), X(0), W(2); step s waits until
 * at most the 4 loads of W(s+2) are outstanding (loads retire in order, so
 * X(s) and W(s) have landed), synchronises, stages X(s+1) into the buffer
 * every wave finished reading in step s-1, issues W(s+3) and computes. */
/* One 64-wide k step of X rows into an LDS stage: thread tid's MB
 * direct-to-LDS loads fill slots 256 i + tid. */
template <int MB>
__device__ __forceinline__ void hk_skinny_stage_x(
    __amdgpu_buffer_rsrc_t xr, uint8_t *stage, const uint32_t *xo,
    uint32_t wave, uint32_t step) {
#pragma unroll
    for (int i = 0; i < MB; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr,
            (__attribute__((address_space(3))) void *)(
                stage + (256u * i + wave * 64u) * 16u),
            16, xo[i], step * 128u, 0, 0);
}

template <int MB>
__global__ void __launch_bounds__(256)
hk_gemm_skinny(const uint16_t *x, const uint16_t *w, const uint16_t *bias,
               uint16_t *c, uint32_t m, uint32_t n, uint32_t k,
               uint32_t x_bytes, uint32_t w_bytes) {
    constexpr int D = 4;
    constexpr uint32_t XSTAGE = MB * 32u * 128u; /* bytes of X per k step */
    /* two X stages (2 XSTAGE bytes), then the four waves' 4-KiB W buffers:
     * 2 XSTAGE + 16 KiB of dynamic LDS */
    extern __shared__ __attribute__((aligned(16))) uint8_t hk_xs[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t row = lane & 31u, half = lane >> 5;
    const uint32_t n0 = (blockIdx.x * 4u + wave) * 32u;
    const __amdgpu_buffer_rsrc_t xr = hk_rsrc(x, x_bytes);
    const __amdgpu_buffer_rsrc_t wr = hk_rsrc(w, w_bytes);
    uint32_t wo[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        wo[q] = (min(n0 + 8u * q + (lane >> 3), n) * k + (lane & 7u) * 8u) *
                2u;
    /* the wave's W buffer, after the two X stages */
    uint8_t *wbuf = hk_xs + 2u * XSTAGE + wave * 4096u;
    /* X staging: slot p = 256 i + tid holds row p / 8, physical chunk p % 8
     * = logical chunk (p % 8) ^ key(row) */
    uint32_t xo[MB];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        const uint32_t p = 256u * i + tid, r = p >> 3;
        const uint32_t chunk = (p & 7u) ^ hk_swz_key(r);
        xo[i] = (min(r, m) * k + chunk * 8u) * 2u;
    }
    auto stage_x = [&](int buf, uint32_t step) {
        hk_skinny_stage_x<MB>(xr, hk_xs + buf * XSTAGE, xo, wave, step);
    };
    hk_v4i wf[D][4];
    auto load_w = [&](int slot, uint32_t step) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            wf[slot][q] = __builtin_amdgcn_raw_buffer_load_b128(
                wr, wo[q], step * 128u, 0);
    };
    /* fragment of X rows mb*32 + row, logical chunk 2q + half */
    auto read_x = [&](int buf, int mb, int q) {
        const uint32_t r = mb * 32u + row;
        return *(const hk_bf16x8 *)(
            hk_xs + buf * XSTAGE + r * 128u +
            (((2u * q + half) ^ hk_swz_key(r)) << 4));
    };
    hk_f32x16 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[mb][r] = 0.0f;
    const uint32_t steps = k / 64u;
    load_w(0, 0);
    if (steps > 1) load_w(1, 1);
    stage_x(0, 0);
    if (steps > 2) load_w(2, 2);
    for (uint32_t s0 = 0; s0 < steps; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const uint32_t s = s0 + d;
            if (s >= steps) break;
            if (s + 2 < steps)
                asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            /* the barrier as inline assembly: __syncthreads() would also
             * wait for every load in flight (vmcnt(0)), the W loads of the
             * steps ahead included */
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (s + 1 < steps) stage_x((d + 1) & 1, s + 1);
            if (s + 3 < steps) load_w((d + 3) % D, s + 3);
            /* W(s)'s lines into the wave's buffer and back out as
             * fragments (a wave's LDS operations run in order: no
             * barrier) */
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t r = 8u * q + (lane >> 3);
                *(hk_v4i *)(wbuf + r * 128u +
                            (((lane & 7u) ^ hk_swz_key(r)) << 4)) = wf[d][q];
            }
            hk_v4i wfrag[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                wfrag[q] = *(const hk_v4i *)(
                    wbuf + row * 128u +
                    (((2u * q + half) ^ hk_swz_key(row)) << 4));
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
                    acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(hk_bf16x8, wfrag[q]),
                        read_x(d & 1, mb, q), acc[mb], 0, 0, 0);
        }
    }
    /* acc[mb][r] = C[mb*32 + row][n0 + (r/4)*8 + half*4 + r%4] */
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const uint32_t mm = mb * 32u + row;
        if (mm >= m) continue;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t col = n0 + q * 8u + half * 4u;
            if (col >= n) continue;
            float out[4];
#pragma unroll
            for (int e = 0; e < 4; e++) out[e] = acc[mb][q * 4 + e];
            if (bias) {
                uint2 b = *(const uint2 *)(bias + col);
                out[0] += hk_bf2f(b.x & 0xffffu);
                out[1] += hk_bf2f(b.x >> 16);
                out[2] += hk_bf2f(b.y & 0xffffu);
                out[3] += hk_bf2f(b.y >> 16);
            }
            *(uint2 *)(c + (size_t)mm * n + col) =
                uint2{hk_pack2(out[0], out[1]), hk_pack2(out[2], out[3])};
        }
    }
}

/* Sequential-k reference GEMM (any shape).  For SwiGLU it writes the fused
 * [M, 2N] bf16 projection into `c` (caller runs the activation). */
__global__ void hk_gemm_reference(const uint16_t *x, const uint16_t *w,
                                  const uint16_t *bias, uint16_t *c,
                                  uint32_t m, uint32_t n, uint32_t k,
                                  int gelu) {
    uint32_t col = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t row = blockIdx.y;
    if (row >= m || col >= n) return;
    float sum = bias ? hk_bf2f(bias[col]) : 0.0f;
    const uint16_t *xr = x + (size_t)row * k;
    const uint16_t *wr = w + (size_t)col * k;
    for (uint32_t i = 0; i < k; i++)
        sum = fmaf(hk_bf2f(xr[i]), hk_bf2f(wr[i]), sum);
    if (gelu) sum = hk_gelu_tanh_f(hk_bf2f(hk_f2bf(sum)));
    c[(size_t)row * n + col] = hk_f2bf(sum);
}

__global__ void hk_swiglu_rows(const uint16_t *fused, uint16_t *out,
                               uint32_t rows, uint32_t width) {
    size_t index = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (index >= (size_t)rows * width) return;
    size_t row = index / width, col = index % width;
    float gate = hk_bf2f(fused[row * 2 * width + col]);
    float up = hk_bf2f(fused[row * 2 * width + width + col]);
    out[index] = hk_f2bf(hk_silu_f(gate) * up);
}

/* devices (bit = ordinal) whose GEMM kernels have their LDS limit raised:
 * the attribute is set with the device current, once per device */
static uint64_t hk_gemm_lds_ready = 0;

/* Split-K reduction over the tile-local partials: 4 tile rows per
 * workgroup, 4 columns per thread; C = epilogue(bf16 rounding of
 * sum_s partial + bias), GELU after the reference's bf16 rounding. */
template <int EPI>
__global__ void __launch_bounds__(256)
hk_splitk_reduce(hk_gemm_args g, uint32_t splits) {
    if (EPI == HK_EPI_SWIGLU) {
        /* 8 tile rows per workgroup, 4 output columns per thread: output
         * column c of the tile (128 per tile) is W-tile row (c/64)*128 +
         * c%64 (gate) and that + 64 (up); out = bf16(silu(bf16 g) bf16 u) */
        const uint32_t part = blockIdx.x >> 5;
        const uint32_t row = (blockIdx.x & 31u) * 8u + (threadIdx.x >> 5);
        const uint32_t c4 = (threadIdx.x & 31u) * 4u;
        uint32_t tile_m, tile_n;
        hk_tile_coords(g.tile_base + part, g.tiles_m, g.tiles_n,
                       tile_m, tile_n);
        const uint32_t m = tile_m * HK_BM + row, n = tile_n * 128u + c4;
        if (m >= g.m || n >= g.n) return;
        const size_t stride = (size_t)g.part_tiles * (HK_BM * HK_BN);
        const float *p = g.partial + (size_t)part * (HK_BM * HK_BN) +
                         row * HK_BN + (c4 >> 6) * 128u + (c4 & 63u);
        float4 gs = *(const float4 *)p, us = *(const float4 *)(p + 64);
        for (uint32_t s = 1; s < splits; s++) {
            const float4 gv = *(const float4 *)(p + s * stride);
            const float4 uv = *(const float4 *)(p + s * stride + 64);
            gs.x += gv.x; gs.y += gv.y; gs.z += gv.z; gs.w += gv.w;
            us.x += uv.x; us.y += uv.y; us.z += uv.z; us.w += uv.w;
        }
        const float gg[4] = {gs.x, gs.y, gs.z, gs.w};
        const float uu[4] = {us.x, us.y, us.z, us.w};
        float out[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            out[e] = hk_silu_f(hk_bf2f(hk_f2bf(gg[e]))) *
                     hk_bf2f(hk_f2bf(uu[e]));
        *(uint2 *)(g.c + (size_t)m * g.n + n) =
            make_uint2(hk_pack2(out[0], out[1]), hk_pack2(out[2], out[3]));
        return;
    }
    const uint32_t part = blockIdx.x >> 6;
    const uint32_t row = (blockIdx.x & 63u) * 4u + (threadIdx.x >> 6);
    const uint32_t tcol = (threadIdx.x & 63u) * 4u;
    const bool second = g.pair_tiles && part >= g.pair_tiles;
    uint32_t tile_m, tile_n;
    hk_tile_coords(g.tile_base + (second ? part - g.pair_tiles : part),
                   g.tiles_m, g.tiles_n, tile_m, tile_n);
    const uint32_t m = tile_m * HK_BM + row, n = tile_n * HK_BN + tcol;
    if (m >= g.m || n >= g.n) return;
    const uint16_t *bias = second ? g.bias1 : g.bias;
    uint16_t *c = second ? g.c1 : g.c;
    const size_t stride = (size_t)g.part_tiles * (HK_BM * HK_BN);
    const float *p = g.partial + (size_t)part * (HK_BM * HK_BN) +
                     row * HK_BN + tcol;
    float4 sum = *(const float4 *)p;
    for (uint32_t s = 1; s < splits; s++) {
        const float4 v = *(const float4 *)(p + s * stride);
        sum.x += v.x; sum.y += v.y; sum.z += v.z; sum.w += v.w;
    }
    float out[4] = {sum.x, sum.y, sum.z, sum.w};
    if (bias) {
        const uint2 b = *(const uint2 *)(bias + n);
        out[0] += hk_bf2f(b.x & 0xffffu);
        out[1] += hk_bf2f(b.x >> 16);
        out[2] += hk_bf2f(b.y & 0xffffu);
        out[3] += hk_bf2f(b.y >> 16);
    }
    if (EPI == HK_EPI_GELU) {
#pragma unroll
        for (int e = 0; e < 4; e++)
            out[e] = hk_gelu_tanh_f(hk_bf2f(hk_f2bf(out[e])));
    }
    *(uint2 *)(c + (size_t)m * g.n + n) =
        make_uint2(hk_pack2(out[0], out[1]), hk_pack2(out[2], out[3]));
}

/* Workgroups for a launch of `tiles` tiles, one workgroup per CU: the
 * fewest that still finish in the same number of rounds, rounded up to a
 * multiple of the 8 XCDs (480 or 1440 tiles on 256 CUs: 240 workgroups). */
static uint32_t hk_gemm_grid(uint32_t tiles, uint32_t cus) {
    static int persist = -1;
    if (persist < 0) {
        const char *e = getenv("H3_HIP_GEMM_PERSIST");
        persist = e ? atoi(e) : 1;
    }
    /* a multiple of 8 workgroups, so that the kernel's XCD regroup applies
     * (each XCD a contiguous run of tiles sharing its L2); the few extra
     * workgroups of a one-round launch find no tile and exit */
    if (!persist || tiles <= cus) return (tiles + 7u) & ~7u;
    const uint32_t rounds = (tiles + cus - 1) / cus;
    const uint32_t wgs = ((tiles + rounds - 1) / rounds + 7u) & ~7u;
    return wgs < cus ? wgs : cus;
}

/* Whether the MFMA kernels take this shape and these pointers. */
static bool hk_gemm_mfma_ok(const struct h3_gpu *gpu, const void *x,
                            const void *w, const void *bias, const void *c,
                            uint32_t m, uint32_t n, uint32_t k, int epilogue) {
    const uint64_t w_rows = epilogue == HK_EPI_SWIGLU ? 2ull * n : n;
    const uint64_t x_bytes = (uint64_t)m * k * 2, w_bytes = w_rows * k * 2;
    /* operand buffers must leave room for a row offset plus a k offset
     * (2 K bytes) below 2^32: rows past the end keep such offsets, which
     * the buffer bound turns into zeros */
    const uint64_t margin = 2ull * k + 4096;
    return !gpu->reference_kernels && k % HK_BK == 0 && k > 0 &&
           n % 4 == 0 && x_bytes + margin < 0x100000000ull &&
           w_bytes + margin < 0x100000000ull &&
           (epilogue != HK_EPI_SWIGLU || n % 64 == 0) &&
           ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
           ((uintptr_t)c & 7) == 0 && ((uintptr_t)bias & 7) == 0;
}

static void hk_gemm_lds_setup(const struct h3_gpu *gpu) {
    const uint64_t bit = 1ull << (gpu->device & 63);
    if (hk_gemm_lds_ready & bit) return;
    (void)hipFuncSetAttribute((const void *)hk_gemm_mfma<HK_EPI_STORE>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              HK_GEMM_LDS);
    (void)hipFuncSetAttribute((const void *)hk_gemm_mfma<HK_EPI_SWIGLU>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              HK_GEMM_LDS);
    (void)hipFuncSetAttribute((const void *)hk_gemm_mfma<HK_EPI_GELU>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              HK_GEMM_LDS);
    (void)hipFuncSetAttribute((const void *)hk_gemm_mfma<HK_EPI_PARTIAL>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              HK_GEMM_LDS);
    (void)hipFuncSetAttribute(
        (const void *)hk_gemm_mfma<HK_EPI_PARTIAL_SWIGLU>,
        hipFuncAttributeMaxDynamicSharedMemorySize, HK_GEMM_LDS);
    (void)hipFuncSetAttribute((const void *)hk_gemm_mfma<HK_EPI_STORE, true>,
                              hipFuncAttributeMaxDynamicSharedMemorySize,
                              HK_GEMM_LDS);
    hk_gemm_lds_ready |= bit;
}

int hk_gemm_bf16(struct h3_gpu *gpu, const uint16_t *x, const uint16_t *w,
                 const uint16_t *bias, uint16_t *c, uint32_t m, uint32_t n,
                 uint32_t k, int epilogue, float *scratch,
                 size_t scratch_bytes) {
    if (!m || !n) return 1;
    const uint64_t w_rows = epilogue == HK_EPI_SWIGLU ? 2ull * n : n;
    const uint64_t x_bytes = (uint64_t)m * k * 2, w_bytes = w_rows * k * 2;
    const bool mfma = hk_gemm_mfma_ok(gpu, x, w, bias, c, m, n, k, epilogue);
    if (mfma && m <= 64 && epilogue == HK_EPI_STORE) {
        if (m <= 32)
            hipLaunchKernelGGL(hk_gemm_skinny<1>, dim3((n + 127) / 128),
                               dim3(256), 2 * 32 * 128 + 16384, gpu->stream, x, w,
                               bias, c, m, n, k, (uint32_t)x_bytes,
                               (uint32_t)w_bytes);
        else
            hipLaunchKernelGGL(hk_gemm_skinny<2>, dim3((n + 127) / 128),
                               dim3(256), 2 * 64 * 128 + 16384, gpu->stream, x, w,
                               bias, c, m, n, k, (uint32_t)x_bytes,
                               (uint32_t)w_bytes);
        return 1;
    }
    if (mfma) {
        hk_gemm_lds_setup(gpu);
        hk_gemm_args g;
        g.x = x; g.w = w; g.bias = bias; g.c = c;
        g.m = m; g.n = n; g.k = k;
        g.tiles_m = (m + HK_BM - 1) / HK_BM;
        const uint32_t cols_per_tile = epilogue == HK_EPI_SWIGLU ? 128 : HK_BN;
        g.tiles_n = (n + cols_per_tile - 1) / cols_per_tile;
        g.x_bytes = (uint32_t)x_bytes;
        g.w_bytes = (uint32_t)w_bytes;
        g.partial = NULL;
        g.split_steps = 0;
        g.tile_base = 0;
        g.part_tiles = 0;
        g.tile_count = g.tiles_m * g.tiles_n;
        g.pair_tiles = 0;
        g.group_tiles = 0;
        g.group = NULL;
        g.w1 = g.bias1 = NULL;
        g.c1 = NULL;
        const uint32_t cus = gpu->num_cus > 0 ? (uint32_t)gpu->num_cus : 256u;
        dim3 grid(hk_gemm_grid(g.tile_count, cus));
        /* Split-K for a sparse last round: when the tiles left after the
         * full rounds of one tile per CU (all of them, for small launches
         * like the 512-row cross-attention K/V projections) would leave over
         * half the CUs idle, those tiles are cut along K into up to
         * num_cus / tiles pieces of at least 4 K steps each; a reduction
         * adds the F32 partials, the bias and the activation (SwiGLU: the
         * gate and up sums, each rounded to bf16 as the fused epilogue
         * does). */
        const uint32_t tiles = g.tiles_m * g.tiles_n;
        const uint32_t k_steps = k / HK_BK;
        const uint32_t full = tiles - tiles % cus, tail = tiles % cus;
        if (tail && tail * 2 <= cus && k_steps >= 8) {
            uint32_t splits = min(cus / tail, k_steps / 4);
            const uint32_t steps = (k_steps + splits - 1) / splits;
            splits = (k_steps + steps - 1) / steps;
            const size_t partial_bytes =
                (size_t)splits * tail * HK_BM * HK_BN * 4;
            if (scratch && partial_bytes > scratch_bytes)
                return hk_fail(gpu,
                               "linear needs %zu bytes of split-K scratch, "
                               "over the %zu-byte static maximum",
                               partial_bytes, scratch_bytes);
            float *partial = scratch ? scratch
                                     : (float *)hk_splitk_space(
                                           gpu, partial_bytes);
            if (!partial) return 0;
            if (full) {
                g.tile_count = full;
                const dim3 fgrid(hk_gemm_grid(full, cus));
                if (epilogue == HK_EPI_GELU)
                    hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_GELU>, fgrid,
                                       dim3(HK_GEMM_THREADS), HK_GEMM_LDS,
                                       gpu->stream, g);
                else if (epilogue == HK_EPI_SWIGLU)
                    hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_SWIGLU>, fgrid,
                                       dim3(HK_GEMM_THREADS), HK_GEMM_LDS,
                                       gpu->stream, g);
                else
                    hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_STORE>, fgrid,
                                       dim3(HK_GEMM_THREADS), HK_GEMM_LDS,
                                       gpu->stream, g);
            }
            g.partial = partial;
            g.split_steps = steps;
            g.tile_base = full;
            g.part_tiles = tail;
            if (epilogue == HK_EPI_SWIGLU)
                hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_PARTIAL_SWIGLU>,
                                   dim3(tail * splits), dim3(HK_GEMM_THREADS),
                                   HK_GEMM_LDS, gpu->stream, g);
            else
                hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_PARTIAL>,
                                   dim3(tail * splits), dim3(HK_GEMM_THREADS),
                                   HK_GEMM_LDS, gpu->stream, g);
            if (epilogue == HK_EPI_SWIGLU)
                hipLaunchKernelGGL(hk_splitk_reduce<HK_EPI_SWIGLU>,
                                   dim3(tail * 32), dim3(256), 0, gpu->stream,
                                   g, splits);
            else if (epilogue == HK_EPI_GELU)
                hipLaunchKernelGGL(hk_splitk_reduce<HK_EPI_GELU>,
                                   dim3(tail * 64), dim3(256), 0, gpu->stream,
                                   g, splits);
            else
                hipLaunchKernelGGL(hk_splitk_reduce<HK_EPI_STORE>,
                                   dim3(tail * 64), dim3(256), 0, gpu->stream,
                                   g, splits);
            return 1;
        }
        if (epilogue == HK_EPI_SWIGLU)
            hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_SWIGLU>, grid,
                               dim3(HK_GEMM_THREADS), HK_GEMM_LDS, gpu->stream,
                               g);
        else if (epilogue == HK_EPI_GELU)
            hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_GELU>, grid,
                               dim3(HK_GEMM_THREADS), HK_GEMM_LDS, gpu->stream,
                               g);
        else
            hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_STORE>, grid,
                               dim3(HK_GEMM_THREADS), HK_GEMM_LDS, gpu->stream,
                               g);
        return 1;
    }
    if (epilogue == HK_EPI_SWIGLU) {
        uint16_t *fused = (uint16_t *)hk_workspace(gpu, (size_t)m * n * 4);
        if (!fused) return 0;
        hipLaunchKernelGGL(hk_gemm_reference, dim3((2 * n + 255) / 256, m),
                           dim3(256), 0, gpu->stream, x, w, bias, fused, m,
                           2 * n, k, 0);
        size_t count = (size_t)m * n;
        hipLaunchKernelGGL(hk_swiglu_rows, dim3((unsigned)((count + 255) / 256)),
                           dim3(256), 0, gpu->stream, fused, c, m, n);
        return 1;
    }
    hipLaunchKernelGGL(hk_gemm_reference, dim3((n + 255) / 256, m), dim3(256),
                       0, gpu->stream, x, w, bias, c, m, n, k,
                       epilogue == HK_EPI_GELU ? 1 : 0);
    return 1;
}

/* Two projections of one input with one shape, C0 = X W0^T + b0 and
 * C1 = X W1^T + b1 (the text's cross-attention K and V).  When each alone
 * would run entirely as split-K (together they fill at most half the CUs,
 * as for the 512-row cross K/V projections), both go into one split-K
 * launch and one reduction, so every CU works on both; otherwise they run
 * one after the other. */
int hk_gemm_bf16_pair(struct h3_gpu *gpu, const uint16_t *x,
                      const uint16_t *w0, const uint16_t *b0, uint16_t *c0,
                      const uint16_t *w1, const uint16_t *b1, uint16_t *c1,
                      uint32_t m, uint32_t n, uint32_t k) {
    if (!m || !n) return 1;
    const uint32_t cus = gpu->num_cus > 0 ? (uint32_t)gpu->num_cus : 256u;
    const uint32_t tiles = ((m + HK_BM - 1) / HK_BM) * ((n + HK_BN - 1) / HK_BN);
    const uint32_t k_steps = k / HK_BK;
    const bool paired =
        m > 64 && k_steps >= 8 && tiles * 4 <= cus &&
        hk_gemm_mfma_ok(gpu, x, w0, b0, c0, m, n, k, HK_EPI_STORE) &&
        hk_gemm_mfma_ok(gpu, x, w1, b1, c1, m, n, k, HK_EPI_STORE);
    if (!paired)
        return hk_gemm_bf16(gpu, x, w0, b0, c0, m, n, k, HK_EPI_STORE) &&
               hk_gemm_bf16(gpu, x, w1, b1, c1, m, n, k, HK_EPI_STORE);
    hk_gemm_lds_setup(gpu);
    hk_gemm_args g;
    g.x = x; g.w = w0; g.bias = b0; g.c = c0;
    g.m = m; g.n = n; g.k = k;
    g.tiles_m = (m + HK_BM - 1) / HK_BM;
    g.tiles_n = (n + HK_BN - 1) / HK_BN;
    g.x_bytes = (uint32_t)((uint64_t)m * k * 2);
    g.w_bytes = (uint32_t)((uint64_t)n * k * 2);
    const uint32_t parts = 2 * tiles;
    uint32_t splits = min(cus / parts, k_steps / 4);
    const uint32_t steps = (k_steps + splits - 1) / splits;
    splits = (k_steps + steps - 1) / steps;
    float *partial = (float *)hk_splitk_space(
        gpu, (size_t)splits * parts * HK_BM * HK_BN * 4);
    if (!partial) return 0;
    g.partial = partial;
    g.split_steps = steps;
    g.tile_base = 0;
    g.part_tiles = parts;
    g.tile_count = parts * splits;
    g.pair_tiles = tiles;
    g.w1 = w1; g.bias1 = b1; g.c1 = c1;
    g.group_tiles = 0;
    g.group = NULL;
    hipLaunchKernelGGL(hk_gemm_mfma<HK_EPI_PARTIAL>, dim3(parts * splits),
                       dim3(HK_GEMM_THREADS), HK_GEMM_LDS, gpu->stream, g);
    hipLaunchKernelGGL(hk_splitk_reduce<HK_EPI_STORE>, dim3(parts * 64),
                       dim3(256), 0, gpu->stream, g, splits);
    return 1;
}

/* A group of `count` problems C_p = X . W_p^T + bias_p of one shape and one
 * X, in one data-parallel launch: the problems' tiles are dealt out like
 * one GEMM's.  `table` is device memory holding (W, bias, C) device
 * addresses per problem. */
static int hk_gemm_bf16_group(struct h3_gpu *gpu, const uint16_t *x,
                              const uint64_t *table, uint32_t count,
                              uint32_t m, uint32_t n, uint32_t k) {
    if (!m || !n || !count) return 1;
    hk_gemm_lds_setup(gpu);
    hk_gemm_args g;
    memset(&g, 0, sizeof(g));
    g.x = x;
    g.m = m; g.n = n; g.k = k;
    g.tiles_m = (m + HK_BM - 1) / HK_BM;
    g.tiles_n = (n + HK_BN - 1) / HK_BN;
    g.x_bytes = (uint32_t)((uint64_t)m * k * 2);
    g.w_bytes = (uint32_t)((uint64_t)n * k * 2);
    g.group_tiles = g.tiles_m * g.tiles_n;
    g.group = table;
    g.tile_count = count * g.group_tiles;
    const uint32_t cus = gpu->num_cus > 0 ? (uint32_t)gpu->num_cus : 256u;
    hipLaunchKernelGGL((hk_gemm_mfma<HK_EPI_STORE, true>),
                       dim3(hk_gemm_grid(g.tile_count, cus)),
                       dim3(HK_GEMM_THREADS), HK_GEMM_LDS, gpu->stream, g);
    return 1;
}

/* ================================================== allocation-free linear
 *
 * h3_hip_linear_bf16_noalloc's split-K partials live in this file-scope
 * device array instead of the context's on-demand scratch, so the call
 * makes no allocation.  Each device holds its own copy from the library's
 * load until the process ends; its address on a device comes from
 * hipGetSymbolAddress (the host-side name is only a stand-in and must never
 * reach a kernel), looked up once per device with that device current.
 * The partial tiles are written in full by the split pieces before the
 * reduction reads them, so the array needs no clearing between calls; calls
 * that overlap on one device share it and race. */
#define HK_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
/* worst case on MI355X: a split never has more pieces than the 256 CUs,
 * each an f32 256x256 partial tile (256 KiB), so 256 x 256 KiB = 64 MiB.
 * Resident on every device the library loads on, called or not. */
static_assert(HK_NOALLOC_SCRATCH_BYTES ==
                  (size_t)256 * HK_BM * HK_BN * sizeof(float),
              "no-alloc scratch sized for 256 CUs of 256x256 f32 partials");
static __device__ __align__(256) float
    scratch[HK_NOALLOC_SCRATCH_BYTES / sizeof(float)];

static float *hk_scratch_ptr[64];
static pthread_mutex_t hk_scratch_lock = PTHREAD_MUTEX_INITIALIZER;

static float *hk_noalloc_scratch(struct h3_gpu *gpu) {
    if (gpu->device < 0 || gpu->device >= 64) {
        hk_fail(gpu, "device ordinal %d out of range", gpu->device);
        return NULL;
    }
    pthread_mutex_lock(&hk_scratch_lock);
    float *ptr = hk_scratch_ptr[gpu->device];
    if (!ptr) {
        int current = -1;
        hipError_t status = hipGetDevice(&current);
        if (status == hipSuccess && current != gpu->device)
            status = hipSetDevice(gpu->device);
        if (status == hipSuccess)
            status = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
        if (current >= 0 && current != gpu->device)
            (void)hipSetDevice(current);
        if (status != hipSuccess || !ptr) {
            pthread_mutex_unlock(&hk_scratch_lock);
            hk_fail_hip(gpu, "static scratch address lookup",
                        status != hipSuccess ? status : hipErrorUnknown);
            return NULL;
        }
        hk_scratch_ptr[gpu->device] = ptr;
    }
    pthread_mutex_unlock(&hk_scratch_lock);
    return ptr;
}

/* ================================================================ ops */

extern "C" {

static int hk_linear_kind(uint32_t rows, uint32_t in, uint32_t out) {
    return rows >= 32 && in >= 256 && out >= 256 ? HK_KIND_LINEAR
                                                 : HK_KIND_DIRECT;
}

int h3_gpu_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                       const h3_gpu_tensor *input, const h3_gpu_tensor *weight,
                       const h3_gpu_tensor *bias, uint32_t rows,
                       uint32_t input_dim, uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "linear input") ||
        !hk_require(gpu, weight, (size_t)output_dim * input_dim, H3_GPU_BF16,
                    "linear weight") ||
        !hk_require(gpu, output, (size_t)rows * output_dim, H3_GPU_BF16,
                    "linear output") ||
        (bias && !hk_require(gpu, bias, output_dim, H3_GPU_BF16,
                             "linear bias")) ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "gemm");
    if (!hk_gemm_bf16(gpu, HK_CBF16(input), HK_CBF16(weight),
                      bias ? HK_CBF16(bias) : NULL, HK_BF16(output), rows,
                      output_dim, input_dim, HK_EPI_STORE))
        return 0;
    return hk_op_end(gpu, "gemm", hk_linear_kind(rows, input_dim, output_dim));
}

int h3_hip_linear_bf16_noalloc(h3_gpu *gpu, h3_gpu_tensor *output,
                               const h3_gpu_tensor *input,
                               const h3_gpu_tensor *weight,
                               const h3_gpu_tensor *bias, uint32_t rows,
                               uint32_t input_dim, uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "linear input") ||
        !hk_require(gpu, weight, (size_t)output_dim * input_dim, H3_GPU_BF16,
                    "linear weight") ||
        !hk_require(gpu, output, (size_t)rows * output_dim, H3_GPU_BF16,
                    "linear output") ||
        (bias && !hk_require(gpu, bias, output_dim, H3_GPU_BF16,
                             "linear bias")) ||
        !hk_require_active(gpu))
        return 0;
    float *partial = hk_noalloc_scratch(gpu);
    if (!partial) return 0;
    hk_op_begin(gpu, "gemm");
    if (!hk_gemm_bf16(gpu, HK_CBF16(input), HK_CBF16(weight),
                      bias ? HK_CBF16(bias) : NULL, HK_BF16(output), rows,
                      output_dim, input_dim, HK_EPI_STORE, partial,
                      HK_NOALLOC_SCRATCH_BYTES))
        return 0;
    return hk_op_end(gpu, "gemm", hk_linear_kind(rows, input_dim, output_dim));
}

h3_gpu_tensor *h3_hip_linear_group_table(h3_gpu *gpu,
                                         h3_gpu_tensor *const *outputs,
                                         const h3_gpu_tensor *const *weights,
                                         const h3_gpu_tensor *const *biases,
                                         uint32_t count, uint32_t rows,
                                         uint32_t input_dim,
                                         uint32_t output_dim) {
    if (!gpu) return NULL;
    if (!count || !outputs || !weights) {
        hk_fail(gpu, "grouped linear table needs at least one problem");
        return NULL;
    }
    uint64_t *entries = (uint64_t *)calloc((size_t)count * 3, sizeof(uint64_t));
    if (!entries) {
        hk_fail(gpu, "out of host memory");
        return NULL;
    }
    for (uint32_t p = 0; p < count; p++) {
        const h3_gpu_tensor *bias = biases ? biases[p] : NULL;
        if (!hk_require(gpu, weights[p], (size_t)output_dim * input_dim,
                        H3_GPU_BF16, "grouped linear weight") ||
            !hk_require(gpu, outputs[p], (size_t)rows * output_dim,
                        H3_GPU_BF16, "grouped linear output") ||
            (bias && !hk_require(gpu, bias, output_dim, H3_GPU_BF16,
                                 "grouped linear bias"))) {
            free(entries);
            return NULL;
        }
        /* the MFMA path's alignment and range rules, checked once here
         * (the input's at each launch) */
        if (!hk_gemm_mfma_ok(gpu, weights[p]->data, weights[p]->data,
                             bias ? bias->data : NULL, outputs[p]->data, rows,
                             output_dim, input_dim, HK_EPI_STORE) &&
            !gpu->reference_kernels) {
            free(entries);
            hk_fail(gpu, "grouped linear problem %u: tensors not aligned for "
                         "the MFMA kernel, or sizes out of its range", p);
            return NULL;
        }
        entries[3 * p] = (uint64_t)(uintptr_t)weights[p]->data;
        entries[3 * p + 1] = bias ? (uint64_t)(uintptr_t)bias->data : 0;
        entries[3 * p + 2] = (uint64_t)(uintptr_t)outputs[p]->data;
    }
    h3_gpu_tensor *table = h3_gpu_tensor_from_u32(
        gpu, (const uint32_t *)entries, (size_t)count * 6);
    free(entries);
    if (table) {
        table->group_shape[0] = rows;
        table->group_shape[1] = input_dim;
        table->group_shape[2] = output_dim;
        table->group_shape[3] = count;
    }
    return table;
}

int h3_hip_linear_group_bf16(h3_gpu *gpu, const h3_gpu_tensor *table,
                             uint32_t first, uint32_t count,
                             const h3_gpu_tensor *input, uint32_t rows,
                             uint32_t input_dim, uint32_t output_dim) {
    /* the table's addresses were validated for one shape: running them at
     * another would read and write past the problems' tensors */
    if (table && table->group_shape[3] == 0)
        return hk_fail(gpu, "grouped linear: the table was not built by "
                            "h3_hip_linear_group_table");
    if (table && (rows != table->group_shape[0] || input_dim != table->group_shape[1] ||
        output_dim != table->group_shape[2]))
        return hk_fail(gpu, "grouped linear: shape %ux%ux%u differs from the "
                            "table's %ux%ux%u", rows, input_dim, output_dim,
                       table->group_shape[0], table->group_shape[1],
                       table->group_shape[2]);
    if (table && (uint64_t)first + count > table->group_shape[3])
        return hk_fail(gpu, "grouped linear: problems [%u, %u) past the "
                            "table's %u", first, first + count,
                       table->group_shape[3]);
    if (!hk_require(gpu, table, ((size_t)first + count) * 6, H3_GPU_U32,
                    "grouped linear table") ||
        !hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "grouped linear input") ||
        !hk_require_active(gpu))
        return 0;
    if (!count) return 1;
    const uint64_t *dev = (const uint64_t *)table->data + (size_t)first * 3;
    const bool mfma = rows > 64 &&
                      hk_gemm_mfma_ok(gpu, input->data, input->data, NULL,
                                      input->data, rows, output_dim,
                                      input_dim, HK_EPI_STORE);
    hk_op_begin(gpu, "gemm_group");
    int ok = 1;
    if (mfma) {
        ok = hk_gemm_bf16_group(gpu, HK_CBF16(input), dev, count, rows,
                                output_dim, input_dim);
    } else {
        /* reference kernels (or a shape the MFMA kernel does not take):
         * the problems one by one, from a host copy of the table */
        uint64_t *entries =
            (uint64_t *)calloc((size_t)count * 3, sizeof(uint64_t));
        if (!entries) return hk_fail(gpu, "out of host memory");
        hipError_t status = hipMemcpyAsync(
            entries, dev, (size_t)count * 3 * sizeof(uint64_t),
            hipMemcpyDeviceToHost, gpu->stream);
        if (status == hipSuccess) status = hipStreamSynchronize(gpu->stream);
        if (status != hipSuccess) {
            free(entries);
            (void)hipGetLastError();
            return hk_fail_hip(gpu, "grouped linear table read", status);
        }
        for (uint32_t p = 0; p < count && ok; p++)
            ok = hk_gemm_bf16(gpu, HK_CBF16(input),
                              (const uint16_t *)(uintptr_t)entries[3 * p],
                              (const uint16_t *)(uintptr_t)entries[3 * p + 1],
                              (uint16_t *)(uintptr_t)entries[3 * p + 2], rows,
                              output_dim, input_dim, HK_EPI_STORE);
        free(entries);
    }
    if (!ok) return 0;
    return hk_op_end(gpu, "gemm_group",
                     hk_linear_kind(rows, input_dim, output_dim));
}

int h3_hip_linear_pair_bf16(h3_gpu *gpu, h3_gpu_tensor *output0,
                            h3_gpu_tensor *output1,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *weight0,
                            const h3_gpu_tensor *bias0,
                            const h3_gpu_tensor *weight1,
                            const h3_gpu_tensor *bias1, uint32_t rows,
                            uint32_t input_dim, uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "linear input") ||
        !hk_require(gpu, weight0, (size_t)output_dim * input_dim,
                    H3_GPU_BF16, "linear weight") ||
        !hk_require(gpu, weight1, (size_t)output_dim * input_dim,
                    H3_GPU_BF16, "linear weight") ||
        !hk_require(gpu, output0, (size_t)rows * output_dim, H3_GPU_BF16,
                    "linear output") ||
        !hk_require(gpu, output1, (size_t)rows * output_dim, H3_GPU_BF16,
                    "linear output") ||
        (bias0 && !hk_require(gpu, bias0, output_dim, H3_GPU_BF16,
                              "linear bias")) ||
        (bias1 && !hk_require(gpu, bias1, output_dim, H3_GPU_BF16,
                              "linear bias")) ||
        !hk_require_active(gpu))
        return 0;
    if (output0 == output1)
        return hk_fail(gpu, "paired linear outputs must be distinct");
    hk_op_begin(gpu, "gemm_pair");
    if (!hk_gemm_bf16_pair(gpu, HK_CBF16(input), HK_CBF16(weight0),
                           bias0 ? HK_CBF16(bias0) : NULL, HK_BF16(output0),
                           HK_CBF16(weight1), bias1 ? HK_CBF16(bias1) : NULL,
                           HK_BF16(output1), rows, output_dim, input_dim))
        return 0;
    return hk_op_end(gpu, "gemm_pair",
                     hk_linear_kind(rows, input_dim, output_dim));
}

int h3_gpu_linear_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                            const h3_gpu_tensor *input,
                            const h3_gpu_tensor *weight,
                            const h3_gpu_tensor *bias, uint32_t rows,
                            uint32_t input_dim, uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "linear input") ||
        !hk_require(gpu, weight, (size_t)output_dim * input_dim, H3_GPU_BF16,
                    "linear weight") ||
        !hk_require(gpu, output, (size_t)rows * output_dim, H3_GPU_BF16,
                    "linear output") ||
        (bias && !hk_require(gpu, bias, output_dim, H3_GPU_BF16,
                             "linear bias")) ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, "gemm_gelu");
    if (!hk_gemm_bf16(gpu, HK_CBF16(input), HK_CBF16(weight),
                      bias ? HK_CBF16(bias) : NULL, HK_BF16(output), rows,
                      output_dim, input_dim, HK_EPI_GELU))
        return 0;
    return hk_op_end(gpu, "gemm_gelu",
                     hk_linear_kind(rows, input_dim, output_dim));
}

int h3_gpu_mlp_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                    const h3_gpu_tensor *input,
                    const h3_gpu_tensor *fc1_weight,
                    const h3_gpu_tensor *fc2_weight, uint32_t rows,
                    uint32_t input_dim, uint32_t hidden_dim,
                    uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "MLP input") ||
        !hk_require(gpu, fc1_weight, (size_t)hidden_dim * 2 * input_dim,
                    H3_GPU_BF16, "MLP fc1 weight") ||
        !hk_require(gpu, fc2_weight, (size_t)output_dim * hidden_dim,
                    H3_GPU_BF16, "MLP fc2 weight") ||
        !hk_require(gpu, output, (size_t)rows * output_dim, H3_GPU_BF16,
                    "MLP output") ||
        !hk_require_active(gpu))
        return 0;
    size_t activated_bytes = (size_t)rows * hidden_dim * 2;
    /* the reference-kernel SwiGLU path also needs 2x that for the fused
     * projection; keep the activation after it */
    size_t fused_bytes = gpu->reference_kernels ? activated_bytes * 2 : 0;
    fused_bytes = (fused_bytes + 255) & ~(size_t)255;
    uint8_t *base = (uint8_t *)hk_workspace(gpu, fused_bytes + activated_bytes);
    if (!base) return 0;
    uint16_t *activated = (uint16_t *)(base + fused_bytes);
    hk_op_begin(gpu, "gemm_swiglu");
    if (!hk_gemm_bf16(gpu, HK_CBF16(input), HK_CBF16(fc1_weight), NULL,
                      activated, rows, hidden_dim, input_dim, HK_EPI_SWIGLU))
        return 0;
    if (!hk_op_end(gpu, "gemm_swiglu", HK_KIND_LINEAR)) return 0;
    hk_op_begin(gpu, "gemm");
    if (!hk_gemm_bf16(gpu, activated, HK_CBF16(fc2_weight), NULL,
                      HK_BF16(output), rows, output_dim, hidden_dim,
                      HK_EPI_STORE))
        return 0;
    return hk_op_end(gpu, "gemm", HK_KIND_LINEAR);
}

int h3_gpu_ffn_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         h3_gpu_tensor *activated,
                         const h3_gpu_tensor *input,
                         const h3_gpu_tensor *fc1_weight,
                         const h3_gpu_tensor *fc1_bias,
                         const h3_gpu_tensor *fc2_weight,
                         const h3_gpu_tensor *fc2_bias, uint32_t rows,
                         uint32_t input_dim, uint32_t hidden_dim,
                         uint32_t output_dim) {
    if (!hk_require(gpu, input, (size_t)rows * input_dim, H3_GPU_BF16,
                    "FFN input") ||
        !hk_require(gpu, fc1_weight, (size_t)hidden_dim * input_dim,
                    H3_GPU_BF16, "FFN fc1 weight") ||
        !hk_require(gpu, fc2_weight, (size_t)output_dim * hidden_dim,
                    H3_GPU_BF16, "FFN fc2 weight") ||
        (fc1_bias && !hk_require(gpu, fc1_bias, hidden_dim, H3_GPU_BF16,
                                 "FFN fc1 bias")) ||
        (fc2_bias && !hk_require(gpu, fc2_bias, output_dim, H3_GPU_BF16,
                                 "FFN fc2 bias")) ||
        (activated && !hk_require(gpu, activated, (size_t)rows * hidden_dim,
                                  H3_GPU_BF16, "FFN activation")) ||
        !hk_require(gpu, output, (size_t)rows * output_dim, H3_GPU_BF16,
                    "FFN output") ||
        !hk_require_active(gpu))
        return 0;
    uint16_t *act = activated ? HK_BF16(activated)
                              : (uint16_t *)hk_workspace(
                                    gpu, (size_t)rows * hidden_dim * 2);
    if (!act) return 0;
    hk_op_begin(gpu, "gemm_gelu");
    if (!hk_gemm_bf16(gpu, HK_CBF16(input), HK_CBF16(fc1_weight),
                      fc1_bias ? HK_CBF16(fc1_bias) : NULL, act, rows,
                      hidden_dim, input_dim, HK_EPI_GELU))
        return 0;
    if (!hk_op_end(gpu, "gemm_gelu", HK_KIND_LINEAR)) return 0;
    hk_op_begin(gpu, "gemm");
    if (!hk_gemm_bf16(gpu, act, HK_CBF16(fc2_weight),
                      fc2_bias ? HK_CBF16(fc2_bias) : NULL, HK_BF16(output),
                      rows, output_dim, hidden_dim, HK_EPI_STORE))
        return 0;
    return hk_op_end(gpu, "gemm", HK_KIND_LINEAR);
}

int h3_gpu_grouped_qkv_linear_rope_bf16(
    h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
    h3_gpu_tensor *value, h3_gpu_tensor *qkv, const h3_gpu_tensor *input,
    const h3_gpu_tensor *weight, const h3_gpu_tensor *q_norm,
    const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos,
    const h3_gpu_tensor *rope_sin, uint32_t rows, uint32_t input_dim,
    uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon) {
    uint32_t out_dim = heads * head_dim * 3;
    return h3_gpu_linear_bf16(gpu, qkv, input, weight, NULL, rows, input_dim,
                              out_dim) &&
           h3_gpu_grouped_qkv_rope_bf16(gpu, query, key, value, qkv, q_norm,
                                        k_norm, rope_cos, rope_sin, rows,
                                        heads, head_dim, rope_half, epsilon);
}

} /* extern "C" */

/* The bf16 MFMA rate this GPU sustains with nothing else running: every CU
 * runs one workgroup of four waves (one per SIMD, the GEMM's occupancy),
 * each issuing v_mfma_f32_32x32x16_bf16 back to back into the 16
 * accumulators of the GEMM's 128x128 wave tile, operands held in
 * registers (no LDS, no memory).  The measured ceiling next to the vendor
 * peak; the sums go to `sink` so that nothing is folded away. */
__global__ void __launch_bounds__(HK_GEMM_THREADS, 1)
__attribute__((amdgpu_waves_per_eu(1, 1)))
hk_mfma_loop(float *sink, uint32_t iterations) {
    hk_f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    hk_bf16x8 fa[4], fb[4];
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            /* small values of the order 2^-7: sums stay finite */
            fa[i][e] = (__bf16)(0.0078125f * (float)((lane + i + e) & 7u));
            fb[i][e] = (__bf16)(0.0078125f * (float)((lane * 3u + i + e) & 7u));
        }
    for (uint32_t it = 0; it < iterations; it++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) total += acc[i][j][r];
    sink[blockIdx.x * HK_GEMM_THREADS + threadIdx.x] = total;
}

extern "C" int h3_hip_mfma_loop(h3_gpu *gpu, h3_gpu_tensor *sink,
                                uint32_t iterations, double *flops) {
    if (!hk_require_active(gpu)) return 0;
    const uint32_t cus = gpu->num_cus > 0 ? (uint32_t)gpu->num_cus : 256u;
    if (!hk_require(gpu, sink, (size_t)cus * HK_GEMM_THREADS, H3_GPU_F32,
                    "MFMA loop sink"))
        return 0;
    hk_op_begin(gpu, "mfma_loop");
    hipLaunchKernelGGL(hk_mfma_loop, dim3(cus), dim3(HK_GEMM_THREADS), 0,
                       gpu->stream, (float *)sink->data, iterations);
    /* 16 MFMAs of 32 x 32 x 16 (2 flops each) per iteration and wave */
    if (flops)
        *flops = (double)cus * 4.0 * iterations * 16.0 * 2.0 * 32 * 32 * 16;
    return hk_op_end(gpu, "mfma_loop", 0);
}
