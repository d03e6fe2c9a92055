/* Flash attention forward for gfx950, head_dim 128, non-causal, bf16 in/out
 * with an F32 online softmax: joint self-attention (q_rows == kv_rows) and
 * cross attention (q_rows != kv_rows) share one kernel.
 *
 * Reference semantics (h3_cuda_attention.cu:1508-1812): scores scaled by
 * `scale`, exp2-domain softmax with scale*log2(e) folded in, running max and
 * sum in F32, P rounded to bf16 (RNE) before P.V, the sum taken over the
 * unrounded P, output = O / l rounded to bf16, keys past the end masked.
 *
 * MI355X design (not the reference's warp tiling):
 *   - the score tile is computed transposed, S^T = K . Q^T, with
 *     v_mfma_f32_32x32x16_bf16: K fragments come from LDS, Q fragments stay
 *     in registers for the whole key loop.  Each lane then owns one query
 *     column and 16 keys of it, so the row max / row sum are in-lane
 *     reductions plus a single exchange with the lane 32 away;
 *   - O^T = V^T . P^T: the P^T operand is the S^T accumulator itself, packed
 *     to bf16 in place.  The accumulator's key order inside a lane is
 *     {4h..4h+3, 8+4h..8+4h+3, ...}; the V^T operand is read in exactly that
 *     key order from the row-major V tile by gfx950's transposing LDS read
 *     (two ds_read_b64_tr_b16 per fragment), so P never goes through LDS;
 *   - K and V are staged row-major by direct-to-LDS loads, with XOR
 *     swizzles on 16-byte chunks (hk_k_swz, hk_v_swz);
 *   - 8 wave64s x 32 queries = 256 queries per workgroup (4 wave64s and
 *     two workgroups per CU for cross attention over at most 1024 keys
 *     and for block-sparse attention, one CSR query block each),
 *     64-key tiles,
 *     double-buffered LDS (2 x 32 KiB) with the next tile's global loads in
 *     flight during the current tile's 32 MFMAs per wave.  At 32 queries a
 *     wave needs under 256 registers, so two waves share each SIMD and the
 *     hardware overlaps one wave's softmax (VALU) with the other's MFMAs;
 *   - the grid is 1-D and regrouped per XCD so the query blocks of one head
 *     run on one XCD and share its L2 copy of that head's K and V;
 *   - the softmax is VALU-bound, so its instruction count is kept low:
 *     P is taken against the running max as it stands and the tile's own
 *     max is only computed (O and l rescaled) when a P sum passes 2^32,
 *     the scale is folded into one FMA per score, and the key-range mask
 *     is compiled only into the last tile's step;
 *   - the V^T reads are inline assembly (hk_vt_read), so the compiler does
 *     not wait for the next tile's direct-to-LDS loads before them.
 *
 * A two-pass reference kernel (hk_attn_ref.hip, built with the default
 * floating-point semantics) serves other head sizes, H3_HIP_REFERENCE=1 and
 * the naive-SDPA knob.
 */
#include "hk_common.h"
#include "hk_internal.h"
#include "hk_attn.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <type_traits>

/* 8 waves per workgroup for self-attention; 4-wave workgroups (two
 * 128-query workgroups per CU, each with its own barrier) were 3% slower
 * there and serve short cross attention (hk_flash_fwd<..., 4>) */
#ifndef HK_WAVES
#define HK_WAVES 8            /* waves per workgroup (two per SIMD) */
#endif
#define HK_THREADS (HK_WAVES * 64)
#define HK_QB (HK_WAVES * 32) /* queries per workgroup */
#define HK_WG_PER_CU (8 / HK_WAVES) /* workgroups per CU: two waves per SIMD */
#define HK_STAGE_BYTES (2 * HK_TILE_BYTES)     /* K tile, then V tile */
#define HK_ATTN_LDS (2 * HK_STAGE_BYTES)       /* 64 KiB */
/* block-sparse launches add one flag word per key tile: up to 64 KiB more,
 * 16384 tiles (1 Mi keys) */
#define HK_ATTN_SPARSE_TILES 16384u
#define HK_ATTN_SPARSE_LDS (HK_ATTN_LDS + 4u * HK_ATTN_SPARSE_TILES)




/* The reference's RoPE pair rotation (h3_cuda_attention.cu:218-233) on 8
 * pairs, x' = x c - y s and y' = y c + x s, rounded to bf16.  With bf16
 * inputs both products are exact in F32, so one two-term dot product
 * (v_dot2_f32_bf16, (x, y) . (c, -s) and (x, y) . (s, c)) rounds exactly
 * once, as the reference's fma over a rounded (exact) product does.
 * t[0..3] hold the packed table entries of the 8 dims, two per 16 bytes:
 * dword 0 / 2 = (c, -s), dword 1 / 3 = (s, c). */
__device__ __forceinline__ void hk_rope8(hk_v4i &x, hk_v4i &y,
                                         const hk_v4i t[4]) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    float xo[8], yo[8];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t xw = (uint32_t)x[w], yw = (uint32_t)y[w];
        /* (x_2w, y_2w) and (x_2w+1, y_2w+1) */
        const uint32_t a0 = __builtin_amdgcn_perm(yw, xw, 0x05040100u);
        const uint32_t a1 = __builtin_amdgcn_perm(yw, xw, 0x07060302u);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t av = h ? a1 : a0;
            const hk_v4i tv = t[w];
            const uint32_t b1 = (uint32_t)tv[2 * h], b2 = (uint32_t)tv[2 * h + 1];
            xo[2 * w + h] = __builtin_amdgcn_fdot2_f32_bf16(
                __builtin_bit_cast(bf2, av), __builtin_bit_cast(bf2, b1),
                0.0f, false);
            yo[2 * w + h] = __builtin_amdgcn_fdot2_f32_bf16(
                __builtin_bit_cast(bf2, av), __builtin_bit_cast(bf2, b2),
                0.0f, false);
        }
    }
    x = __builtin_bit_cast(hk_v4i, hk_pack8(xo));
    y = __builtin_bit_cast(hk_v4i, hk_pack8(yo));
}

/* Correctly rounded square root of a positive normal float (the inputs
 * here are at least the norm's epsilon).  This file's fast-math flags turn
 * sqrtf (and __fsqrt_rn) into the bare v_sqrt_f32, which can be an ulp
 * off; the row kernels' sqrtf is the IEEE one.  The hardware estimate s is
 * within an ulp, and the residuals x - s' s of its two neighbours s' pick
 * the correctly rounded one (the expansion the compiler uses for IEEE
 * sqrtf). */
__device__ __forceinline__ float hk_sqrt_rn(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float down = __uint_as_float(__float_as_uint(s) - 1u);
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    float r = __builtin_fmaf(-down, s, x) <= 0.0f ? down : s;
    return __builtin_fmaf(-up, s, x) > 0.0f ? up : r;
}

/* Packs bf16 cos / sin tables [rows][48] into the (c, -s), (s, c) pairs
 * the in-kernel rotation takes. */
__global__ void __launch_bounds__(256)
hk_rope_pack(const uint16_t *cosines, const uint16_t *sines, uint64_t *out,
             uint32_t count) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= count) return;
    const uint32_t c = cosines[i], sn = sines[i];
    const uint32_t cs = c | ((sn ^ 0x8000u) << 16);
    const uint32_t sc = sn | (c << 16);
    out[i] = (uint64_t)cs | ((uint64_t)sc << 32);
}

/* Rotates every key row once: K [rows][heads][128] -> out, the RoPE pairs
 * (d, d + 48), d < 48, through hk_rope8 and dims 96..127 copied.  Thread
 * t of a (row, head) handles part t & 7: chunk pair (p, p + 6) for p < 6,
 * chunks (12, 13) and (14, 15) for parts 6 and 7.  Rotating the keys in the
 * attention kernel instead repeats it for every query block that reads
 * them (24 at 6144 rows, 38 at 9720). */
__global__ void __launch_bounds__(256)
hk_rope_keys(const uint16_t *k, const uint64_t *table, uint16_t *out,
             uint32_t rows, uint32_t heads) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t part = i & 7u, rh = i >> 3;
    if (rh >= rows * heads) return;
    const uint32_t row = rh / heads;
    const uint32_t c0 = part < 6 ? part : (part == 6 ? 12u : 14u);
    const uint32_t c1 = part < 6 ? part + 6u : c0 + 1u;
    const hk_v4i *src = (const hk_v4i *)(k + (size_t)rh * HK_HD);
    hk_v4i *dst = (hk_v4i *)(out + (size_t)rh * HK_HD);
    hk_v4i x = src[c0], y = src[c1];
    if (part < 6) {
        const hk_v4i *t =
            (const hk_v4i *)(table + (size_t)row * HK_ROPE_HALF + part * 8u);
        const hk_v4i tv[4] = {t[0], t[1], t[2], t[3]};
        hk_rope8(x, y, tv);
    }
    dst[c0] = x;
    dst[c1] = y;
}

template <bool SPARSE, bool SPLIT, int NW = HK_WAVES>
__global__ void __launch_bounds__(NW * 64, 8 / NW)
hk_flash_fwd(hk_attn_args a) {
    constexpr uint32_t NW_QB = NW * 32;   /* queries per workgroup */
    constexpr int NW_DMA = 16 / NW;       /* 1-KiB loads per wave, tile and operand */
    extern __shared__ __attribute__((aligned(16))) uint8_t hk_lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t col = lane & 31u, half = lane >> 5;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t item = SPLIT ? a.full_units + pid / a.pieces : pid;
    const uint32_t qblock = item % a.q_blocks, head = item / a.q_blocks;
    const uint32_t row_stride = a.in_stride; /* elements, Q / K / V rows */

    const __amdgpu_buffer_rsrc_t qr = hk_attn_rsrc(a.q, a.q_bytes);
    __amdgpu_buffer_rsrc_t tr;
    /* a runtime branch (once per workgroup) rather than a template
     * argument: a separate instance came out 3-5% slower in its main loop */
    if (a.rope_pk) tr = hk_attn_rsrc(a.rope_pk, a.rope_bytes);

    /* ---- staging plan ----
     * K and V go from global memory straight into LDS with direct-to-LDS
     * buffer loads: wave w fills rows 8 w .. 8 w + 7 of a tile in two
     * 1-KiB loads, lane l writing physical chunk l & 15 of row 4 i + l / 16;
     * the swizzles are applied on the global side.  (With the RoPE table, K arrives
     * already rotated by hk_rope_keys.) */
    /* sized for the 4-wave build; the 8-wave one uses the first two */
    uint32_t k_dma_off[4], v_dma_off[4];
#pragma unroll
    for (int i = 0; i < NW_DMA; i++) {
        const uint32_t row = (wave * NW_DMA + i) * 4u + (lane >> 4);
        const uint32_t kc = (lane & 15u) ^ (row & 15u);
        const uint32_t vc = (lane & 15u) ^ ((row & 3u) << 2);
        k_dma_off[i] = (row * row_stride + head * HK_HD) * 2u + kc * 16u;
        v_dma_off[i] = (row * row_stride + head * HK_HD) * 2u + vc * 16u;
    }
    auto issue_tile = [&](uint32_t kv0, uint32_t stage) {
        const size_t base = (size_t)kv0 * row_stride;
        const uint32_t left = a.kv_bytes - kv0 * row_stride * 2u;
        const __amdgpu_buffer_rsrc_t vr =
            hk_attn_rsrc(a.v + base, a.v_bytes - kv0 * row_stride * 2u);
        uint8_t *st = hk_lds + stage * HK_STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < NW_DMA; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                vr, (hk_lds_void *)(st + HK_TILE_BYTES +
                                    (wave * NW_DMA + i) * 1024u),
                16, v_dma_off[i], 0, 0, 0);
        const __amdgpu_buffer_rsrc_t kr = hk_attn_rsrc(a.k + base, left);
#pragma unroll
        for (int i = 0; i < NW_DMA; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                kr, (hk_lds_void *)(st + (wave * NW_DMA + i) * 1024u), 16,
                k_dma_off[i], 0, 0, 0);
    };

    const uint32_t all_tiles = (a.kv_rows + HK_KT - 1) / HK_KT;
    /* a split piece covers key tiles [first_tile, dense) */
    const uint32_t piece_tiles =
        SPLIT ? (all_tiles + a.pieces - 1) / a.pieces : all_tiles;
    const uint32_t first_tile = SPLIT ? (pid % a.pieces) * piece_tiles : 0;
    const uint32_t dense =
        SPLIT ? min(all_tiles, first_tile + piece_tiles) : all_tiles;
    /* dense: the first key tile's loads go out before the Q fragments'
     * (its latency then overlaps theirs) */
    if constexpr (!SPARSE) issue_tile(first_tile * HK_KT, 0);

    /* ---- Q fragments: B operand of S^T = K . Q^T ----
     * k-step ks: Q[q][16 ks + 8 half .. +8]; with the RoPE table, dims d < 48 pair
     * with d + 48, i.e. k-step ks < 3 with ks + 3 in the same lane */
    const uint32_t qbase = qblock * NW_QB + wave * 32u;
    hk_bf16x8 qf[8];
    {
        const uint32_t q = qbase + col;
        const uint32_t off = q < a.q_rows
            ? ((q * row_stride + head * HK_HD + half * 8u) * 2u)
            : 0xfffffff0u;
        hk_v4i raw[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            raw[ks] = __builtin_amdgcn_raw_buffer_load_b128(
                qr, off == 0xfffffff0u ? off : off + ks * 32u, 0, 0);
        if (a.rope_pk) {
            /* dims 16 ks + 8 half + e, e < 8: 64 bytes of the table */
            const uint32_t roff = q < a.q_rows
                ? (q * HK_ROPE_HALF + half * 8u) * 8u : 0xfffffff0u;
#pragma unroll
            for (int ks = 0; ks < 3; ks++) {
                hk_v4i t[4];
#pragma unroll
                for (int p = 0; p < 4; p++)
                    t[p] = __builtin_amdgcn_raw_buffer_load_b128(
                        tr, roff == 0xfffffff0u ? roff
                                                : roff + ks * 128u + p * 16u,
                        0, 0);
                hk_rope8(raw[ks], raw[ks + 3], t);
            }
        }
        if (a.q_norm) {
            /* the row kernels' lanes hold dims 8 j .. 8 j + 7, j < 16, and
             * sum them with a fma chain, then over j with an xor tree
             * (8, 4, 2, 1); chunk j here is k-step j / 2 of the lane half
             * j % 2, so the tree's first three levels pair k-steps
             * (ks, ks + 4), (ks, ks ^ 2), (ks, ks ^ 1) in the lane and the
             * last pairs the two halves. */
            float x[8][8], part[8];
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                part[ks] = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t bits = (uint32_t)raw[ks][w];
                    x[ks][2 * w] = hk_bf2f(bits & 0xffffu);
                    x[ks][2 * w + 1] = hk_bf2f(bits >> 16);
                }
#pragma unroll
                for (int e = 0; e < 8; e++)
                    part[ks] = __builtin_fmaf(x[ks][e], x[ks][e], part[ks]);
                /* this file's -fassociative-math would otherwise merge the
                 * partial sums into one chain: each sum is pinned */
                asm volatile("" : "+v"(part[ks]));
            }
            float l1[4];
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                l1[ks] = part[ks] + part[ks + 4];
                asm volatile("" : "+v"(l1[ks]));
            }
            float l2a = l1[0] + l1[2], l2b = l1[1] + l1[3];
            asm volatile("" : "+v"(l2a), "+v"(l2b));
            float l3 = l2a + l2b;
            asm volatile("" : "+v"(l3));
            const auto sw = __builtin_amdgcn_permlane32_swap(
                __float_as_uint(l3), __float_as_uint(l3), false, false);
            /* lanes < 32 find the other half's value in the second
             * result, lanes >= 32 in the first */
            const float other = __uint_as_float(half ? sw[0] : sw[1]);
            float total = l3 + other;
            asm volatile("" : "+v"(total));
            const float inv = __fdiv_rn(
                1.0f, hk_sqrt_rn(__builtin_fmaf(total, 0.0078125f, a.q_eps)));
            const hk_v4i *wv = (const hk_v4i *)a.q_norm;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const hk_v4i wr = wv[2 * ks + half];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t bits = (uint32_t)wr[w];
                    /* (x inv) w, rounded in that order (pinned, or the
                     * flags would let it become x (inv w)) */
                    float lo = x[ks][2 * w] * inv, hi = x[ks][2 * w + 1] * inv;
                    asm volatile("" : "+v"(lo), "+v"(hi));
                    x[ks][2 * w] = lo * hk_bf2f(bits & 0xffffu);
                    x[ks][2 * w + 1] = hi * hk_bf2f(bits >> 16);
                }
            }
            if (a.q_cos) {
                const bool live = q < a.q_rows;
                const hk_v4i *cv = (const hk_v4i *)(a.q_cos +
                    (size_t)(live ? q : 0) * HK_ROPE_HALF + half * 8u);
                const hk_v4i *sv = (const hk_v4i *)(a.q_sin +
                    (size_t)(live ? q : 0) * HK_ROPE_HALF + half * 8u);
#pragma unroll
                for (int ks = 0; ks < 3; ks++) {
                    const hk_v4i cr = cv[2 * ks], sr = sv[2 * ks];
#pragma unroll
                    for (int w = 0; w < 4; w++) {
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const uint32_t cb = (uint32_t)cr[w], sb = (uint32_t)sr[w];
                            const float c = hk_bf2f(h ? cb >> 16 : cb & 0xffffu);
                            const float sn = hk_bf2f(h ? sb >> 16 : sb & 0xffffu);
                            const int e = 2 * w + h;
                            const float lo = x[ks][e], hi = x[ks + 3][e];
                            float hs = hi * sn, ls = lo * sn;
                            asm volatile("" : "+v"(hs), "+v"(ls));
                            x[ks][e] = __builtin_fmaf(lo, c, -hs);
                            x[ks + 3][e] = __builtin_fmaf(hi, c, ls);
                        }
                    }
                }
            }
#pragma unroll
            for (int ks = 0; ks < 8; ks++)
                raw[ks] = __builtin_bit_cast(hk_v4i, hk_pack8(x[ks]));
        }
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            qf[ks] = __builtin_bit_cast(hk_bf16x8, raw[ks]);
    }

    /* fragment addresses (lane parts; the stage and tile sub-block go in
     * the instructions' offset fields) */
    const uint32_t lds_base =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)
            hk_lds;
    uint32_t k_frag[8];
#pragma unroll
    for (int kk = 0; kk < 8; kk++)
        k_frag[kk] = lds_base + hk_k_swz(col, kk * 2u + half);
    /* V^T operand of O^T = V^T . P^T: lane l needs, for dim 32 d + l % 32,
     * keys 4 half + {0..3} and 8 + 4 half + {0..3} of a 16-key step (the
     * key order of the P^T operand).  ds_read_b64_tr_b16 hands lane i of a
     * 16-lane group the column i of a 4-row x 16-column block whose rows
     * source lanes 4 r .. 4 r + 3 address (4 columns each): source lane
     * j = l & 15 addresses row 4 half + j / 4, columns 16 (l / 16 & 1) +
     * 4 (j & 3) of dim block d. */
    uint32_t v_frag[4];
    {
        const uint32_t j = lane & 15u, g1 = (lane >> 4) & 1u;
        const uint32_t vrow = 4u * half + (j >> 2);
        const uint32_t low = 2u * g1 + ((j & 3u) >> 1);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const uint32_t chunk = (uint32_t)d * 4u + low;
            v_frag[d] = lds_base + HK_TILE_BYTES + hk_v_swz(vrow, chunk) +
                        8u * (j & 1u);
        }
    }

    hk_f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = 0.0f;
    float m_run = -INFINITY, l_part = 0.0f;

    /* a wave whose 32 queries all lie past q_rows (the last query block of
     * a ragged sequence) still stages its share of every tile and meets
     * every barrier, but skips the MFMAs and the softmax: its output is
     * never stored, and its split partials keep weight 0 */
    const bool live = qbase < a.q_rows;

    /* ---- key-tile schedule ----
     * Dense: every 64-key tile in order.  Block-sparse (128-query
     * workgroups, one 128-row block of the CSR each): the kept tiles of
     * [first_tile, dense) in order.  The list's length is clamped to the
     * dense tile count, as in the reference kernel.  It becomes one flag
     * word per key tile in LDS past the two stages, set by the whole
     * workgroup once per work item, and each step finds the next tile with
     * LDS reads: reading the list from global memory at every step put a
     * load's latency before each tile's loads. */
    static_assert(!SPARSE || NW == 4, "block-sparse walks one 128-row block");
    uint32_t *flags = (uint32_t *)(hk_lds + HK_ATTN_LDS);
    if (SPARSE) {
        const uint32_t first = a.sparse_ptr[qblock];
        const uint32_t end = min(a.sparse_ptr[qblock + 1], first + all_tiles);
        const uint32_t span = dense - first_tile;
        for (uint32_t t = tid; t < span; t += NW * 64u) flags[t] = 0u;
        __syncthreads();
        for (uint32_t j = first + tid; j < end; j += NW * 64u) {
            const uint32_t t = a.sparse_idx[j];
            if (t >= first_tile && t < dense) flags[t - first_tile] = 1u;
        }
        __syncthreads();
    }
    /* the first flagged tile at or after `from`, or dense when none */
    auto next_tile = [&](uint32_t from) -> uint32_t {
        uint32_t t = from;
        while (t < dense && flags[t - first_tile] == 0u) t++;
        return t;
    };

    /* one tile: MFMAs and softmax on stage STAGE (compile-time, so every
     * LDS address is a lane register plus an immediate), with the next
     * tile's loads in flight into the other stage */
    auto tile_step = [&](auto stage_tag, uint32_t tile, uint32_t next_tile,
                         bool more, bool mine, auto tail_tag) {
        constexpr uint32_t stage = decltype(stage_tag)::value;
        constexpr bool tail = decltype(tail_tag)::value;
        if (more) issue_tile(next_tile * HK_KT, stage ^ 1u);

        if (mine) {
        /* S^T[kt]: keys kt*32 + .., queries col */
        hk_f32x16 s[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[kt][r] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                const hk_bf16x8 kf = *(const hk_bf16x8 *)(
                    (__attribute__((address_space(3))) uint8_t *)(uintptr_t)
                        (k_frag[kk] + stage * HK_STAGE_BYTES +
                         kt * 32u * 256u));
                s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    kf, qf[kk], s[kt], 0, 0, 0);
            }
        }

        /* online softmax per query column.  P = exp2(s - m_run) is taken
         * against the running maximum m_run as it stands; the tile's own
         * maximum is only computed, and m_run moved (O and l rescaled),
         * when that leaves a lane's P sum above 2^32 (some score above
         * m_run + 32 in the exp2 domain) or m_run is still unset.  So P <=
         * 2^32 always, which keeps O and l far from f32 overflow, and the
         * common tile runs its exponentials straight off the scores.  The
         * stale maximum is not the row's true maximum and the gap between
         * them is not a power of two, so bf16(P) can round differently
         * from the reference's P (relative to the row maximum) by up to
         * half a bf16 ulp per element: O matches to the bf16 rounding of P
         * (the bound the tests apply), while l, summed over the unrounded
         * P, is exact up to f32 rounding. */
        const uint32_t kv0 = tile * HK_KT;
        hk_bf16x8 pf[2][2]; /* [kt][step] */
        /* only the last tile has keys past kv_rows; the block-sparse
         * walk, whose steps all take this path, skips it on the others */
        if (tail && tile + 1u == all_tiles && (a.kv_rows & (HK_KT - 1u))) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t key = kv0 + kt * 32u + (r >> 2) * 8u +
                                         half * 4u + (r & 3);
                    if (key >= a.kv_rows) s[kt][r] = -INFINITY;
                }
        }
        auto exps = [&]() -> float {
            const float neg = -m_run;
            float sum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                float p[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = __builtin_amdgcn_exp2f(
                        __builtin_fmaf(s[kt][r], a.scale_log2, neg));
                    sum += p[r];
                }
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    hk_bf16x8 v;
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = (__bf16)p[st * 8 + e];
                    pf[kt][st] = v;
                }
            }
            return sum;
        };
        /* (with m_run unset the sum is not looked at: it may hold
         * inf - inf) */
        const bool unset = m_run == -INFINITY;
        float sum = unset ? 0.0f : exps();
        if (__builtin_amdgcn_ballot_w64(unset || sum > 0x1p32f)) {
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r += 2)
                    mx = __builtin_fmaxf(
                        mx, __builtin_fmaxf(s[kt][r], s[kt][r + 1]));
            /* the column's other 16 keys sit in the lane 32 away: one
             * v_permlane32_swap (no LDS round trip) hands each half the
             * other's value */
            const auto sw = __builtin_amdgcn_permlane32_swap(
                __float_as_uint(mx), __float_as_uint(mx), false, false);
            mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) *
                 a.scale_log2;
            const float m_new = fmaxf(m_run, mx);
            const float ref = m_new == -INFINITY ? 0.0f : m_new;
            const float c = __builtin_amdgcn_exp2f(m_run - ref);
            m_run = ref;
            l_part *= c;
#pragma unroll
            for (int d = 0; d < 4; d++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[d][r] *= c;
            sum = exps();
        }
        l_part += sum;

        /* O^T[d] += V^T[d, keys] . P^T[keys]: the V^T operand comes from
         * the row-major V tile through two transposing 8-byte reads per
         * fragment, a 16-key step's four fragments read while the MFMAs
         * of the step before run (hk_vt_read) */
        hk_v2i vt[2][4][2];
        hk_vt_read(vt[0], v_frag, stage * HK_STAGE_BYTES);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int kt = i >> 1, st = i & 1;
            if (i < 3) {
                hk_vt_read(vt[(i + 1) & 1], v_frag,
                           stage * HK_STAGE_BYTES +
                               (((i + 1) >> 1) * 32u + ((i + 1) & 1) * 16u) *
                                   256u);
                hk_vt_wait<8>(vt[i & 1]);
            } else {
                hk_vt_wait<0>(vt[i & 1]);
            }
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const hk_v4i both = {vt[i & 1][d][0][0], vt[i & 1][d][0][1],
                                     vt[i & 1][d][1][0], vt[i & 1][d][1][1]};
                o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(hk_bf16x8, both), pf[kt][st], o[d], 0,
                    0, 0);
            }
        }
        } /* mine */

        /* the next stage's direct-to-LDS loads (issued by every wave) have
         * landed once every wave has waited for its own */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };

    using S0 = std::integral_constant<uint32_t, 0>;
    using S1 = std::integral_constant<uint32_t, 1>;
    using NT = std::integral_constant<bool, false>;
    using TT = std::integral_constant<bool, true>;
    if constexpr (!SPARSE) {
        /* the key-range mask is compiled only into the step of the last
         * tile, the only one with keys past kv_rows */
        const uint32_t n = dense - first_tile;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        uint32_t i = 0;
        for (; i + 2 < n; i += 2) {
            const uint32_t t = first_tile + i;
            tile_step(S0(), t, t + 1, true, live, NT());
            tile_step(S1(), t + 1, t + 2, true, live, NT());
        }
        if (i + 2 == n) {
            tile_step(S0(), first_tile + i, first_tile + i + 1, true, live,
                      NT());
            tile_step(S1(), first_tile + i + 1, 0, false, live, TT());
        } else {
            tile_step(S0(), first_tile + i, 0, false, live, TT());
        }
    } else {
        uint32_t cur = next_tile(first_tile);
        if (cur < dense) issue_tile(cur * HK_KT, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        /* one instantiation per stage (register pressure) */
        while (cur < dense) {
            uint32_t nxt = next_tile(cur + 1u);
            tile_step(S0(), cur, nxt, nxt < dense, live, TT());
            cur = nxt;
            if (cur >= dense) break;
            nxt = next_tile(cur + 1u);
            tile_step(S1(), cur, nxt, nxt < dense, live, TT());
            cur = nxt;
        }
    }

    if constexpr (SPLIT) {
        /* unnormalised partials for the combine kernel, through the
         * wave's 8 KiB of LDS in two halves of 64 dims (16-byte chunk c of
         * row r at c ^ (r % 16)), leaving as whole 256-byte row halves */
        const uint32_t ql = wave * 32u + col;
        float *pw = (float *)(hk_lds + wave * (32u * 64u * 4u));
#pragma unroll
        for (int hd = 0; hd < 2; hd++) {
#pragma unroll
            for (int dd = 0; dd < 2; dd++)
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    const int d = 2 * hd + dd;
                    const uint32_t c = dd * 8u + blk * 2u + half;
                    *(float4 *)(pw + col * 64u + ((c ^ (col & 15u)) << 2)) =
                        make_float4(o[d][blk * 4 + 0], o[d][blk * 4 + 1],
                                    o[d][blk * 4 + 2], o[d][blk * 4 + 3]);
                }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t r = i * 4u + (lane >> 4), c = lane & 15u;
                const float4 v =
                    *(const float4 *)(pw + r * 64u + ((c ^ (r & 15u)) << 2));
                *(float4 *)(a.part_o +
                            ((size_t)pid * NW_QB + wave * 32u + r) * HK_HD +
                            hd * 64u + c * 4u) = v;
            }
        }
        const float l = l_part + __shfl_xor(l_part, 32, 64);
        if (half == 0)
            *(float2 *)(a.part_ml + ((size_t)pid * NW_QB + ql) * 2u) =
                make_float2(m_run, l);
        return;
    }
    /* ---- normalise and store ----
     * The lane owns query column `col` and dims d*32 + (r/4)*8 + 4*half +
     * r%4; stored directly, each store would write 16 bytes into each of
     * 32 rows (20% of a 512-key cross-attention's time).  The wave's 32
     * rows go through its own 8 KiB of LDS instead (free after the last
     * tile's barrier; 16-byte chunk c of row r at c ^ (r % 16)) and leave
     * as whole 256-byte rows, four rows per store. */
    const float l = l_part + __shfl_xor(l_part, 32, 64);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    uint8_t *ow = hk_lds + wave * (32u * HK_HD * 2u);
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int blk = 0; blk < 4; blk++) {
            const uint32_t dim = d * 32u + blk * 8u + half * 4u;
            uint2 packed = {hk_pack2(o[d][blk * 4 + 0] * inv,
                                     o[d][blk * 4 + 1] * inv),
                            hk_pack2(o[d][blk * 4 + 2] * inv,
                                     o[d][blk * 4 + 3] * inv)};
            *(uint2 *)(ow + col * 256u + (((dim >> 3) ^ (col & 15u)) << 4) +
                       (dim & 7u) * 2u) = packed;
        }
    /* the wave's own rows: its LDS operations run in order */
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t r = i * 4u + (lane >> 4), c = lane & 15u;
        const uint4 v = *(const uint4 *)(ow + r * 256u + ((c ^ (r & 15u)) << 4));
        const uint32_t q = qbase + r;
        if (q >= a.q_rows) continue;
        uint16_t *out = a.head_major
            ? a.o + ((size_t)head * a.q_rows + q) * HK_HD
            : a.o + (size_t)q * a.heads * HK_HD + (size_t)head * HK_HD;
        *(uint4 *)(out + c * 8u) = v;
    }
}

/* Combines the key-range pieces of the split work items: per query, with
 * the pieces' running maxima m_p (exp2 domain), sums l_p and unnormalised
 * O_p, O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p, M = max_p m_p.
 * 8 queries per workgroup, 4 dims per thread; QB queries per work item. */
template <uint32_t QB>
__global__ void __launch_bounds__(256) hk_flash_combine(hk_attn_args a) {
    const uint32_t titem = blockIdx.x / (QB / 8u);
    const uint32_t ql = (blockIdx.x % (QB / 8u)) * 8u + (threadIdx.x >> 5);
    const uint32_t d4 = (threadIdx.x & 31u) * 4u;
    const uint32_t item = a.full_units + titem;
    const uint32_t qblock = item % a.q_blocks, head = item / a.q_blocks;
    const uint32_t q = qblock * QB + ql;
    if (q >= a.q_rows) return;
    const size_t first = (size_t)titem * a.pieces;
    float top = -INFINITY;
    for (uint32_t p = 0; p < a.pieces; p++)
        top = fmaxf(top, a.part_ml[((first + p) * QB + ql) * 2u]);
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float l = 0.0f;
    for (uint32_t p = 0; p < a.pieces; p++) {
        const float2 ml =
            *(const float2 *)(a.part_ml + ((first + p) * QB + ql) * 2u);
        /* a sparse piece may hold no key tile of this query block */
        const float w =
            ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - top);
        const float4 op = *(const float4 *)(a.part_o +
                                            ((first + p) * QB + ql) * HK_HD +
                                            d4);
        sum.x += w * op.x; sum.y += w * op.y;
        sum.z += w * op.z; sum.w += w * op.w;
        l += w * ml.y;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    uint16_t *out = a.head_major
        ? a.o + ((size_t)head * a.q_rows + q) * HK_HD
        : a.o + (size_t)q * a.heads * HK_HD + (size_t)head * HK_HD;
    *(uint2 *)(out + d4) = make_uint2(hk_pack2(sum.x * inv, sum.y * inv),
                                      hk_pack2(sum.z * inv, sum.w * inv));
}

/* devices (bit = ordinal) whose attention kernels have their LDS limit
 * raised */
static uint64_t hk_attn_lds_ready = 0;

template <bool SPARSE, bool SPLIT, int NW = HK_WAVES>
static void hk_flash_set_lds() {
    (void)hipFuncSetAttribute(
        (const void *)hk_flash_fwd<SPARSE, SPLIT, NW>,
        hipFuncAttributeMaxDynamicSharedMemorySize,
        SPARSE ? HK_ATTN_SPARSE_LDS : HK_ATTN_LDS);
}

template <bool SPLIT>
static void hk_flash_launch(struct h3_gpu *gpu, const hk_attn_args &a,
                            bool masked, uint32_t grid, bool four) {
    const dim3 g(grid), b(HK_THREADS);
    const uint32_t sparse_lds =
        HK_ATTN_LDS + 4u * ((a.kv_rows + HK_KT - 1u) / HK_KT);
    if (four && masked)
        hipLaunchKernelGGL((hk_flash_fwd<true, SPLIT, 4>), g, dim3(256),
                           sparse_lds, gpu->stream, a);
    else if (four)
        hipLaunchKernelGGL((hk_flash_fwd<false, false, 4>), g, dim3(256),
                           HK_ATTN_LDS, gpu->stream, a);
    else
        hipLaunchKernelGGL((hk_flash_fwd<false, SPLIT>), g, b, HK_ATTN_LDS,
                           gpu->stream, a);
}

int hk_attention_bf16(struct h3_gpu *gpu, const uint16_t *q,
                      const uint16_t *k, const uint16_t *v, uint16_t *o,
                      uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                      uint32_t head_dim, float scale, int head_major,
                      int sparse, const uint16_t *rope_cos,
                      const uint16_t *rope_sin, int fused_qkv,
                      const uint16_t *q_norm, const uint16_t *q_cos,
                      const uint16_t *q_sin, float q_eps) {
    if (!q_rows || !heads) return 1;
    /* fused: q, k, v are the three thirds of each [rows][3][heads][hd] row */
    const uint64_t inner = (uint64_t)heads * head_dim;
    const uint64_t in_stride = fused_qkv ? 3 * inner : inner;
    const uint64_t q_bytes = (uint64_t)q_rows * in_stride * 2;
    const uint64_t kv_bytes =
        (uint64_t)kv_rows * in_stride * 2 - (fused_qkv ? inner * 2 : 0);
    const uint64_t v_bytes =
        (uint64_t)kv_rows * in_stride * 2 - (fused_qkv ? inner * 4 : 0);
    const bool rope = rope_cos != NULL;
    /* the reference's debugging knob H3_CUDA_SDPA_NAIVE=1 (read per call,
     * like its backend: h3_cuda_attention.cu) selects the two-pass kernel;
     * H3_HIP_SDPA_NAIVE is the same knob under this backend's prefix */
    const char *naive = getenv("H3_CUDA_SDPA_NAIVE");
    if (!naive || !*naive) naive = getenv("H3_HIP_SDPA_NAIVE");
    const bool naive_on = naive && *naive && strcmp(naive, "0") != 0;
    const bool flash = !gpu->reference_kernels && !naive_on &&
                       head_dim == HK_HD &&
                       kv_rows > 0 && q_bytes < 0xfffff000ull &&
                       kv_bytes < 0xfffff000ull &&
                       ((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 &&
                       ((uintptr_t)v & 15) == 0 && ((uintptr_t)o & 7) == 0;
    if (q_norm && (!flash || rope || ((uintptr_t)q_norm & 15) ||
                   ((uintptr_t)q_cos & 15) || ((uintptr_t)q_sin & 15) ||
                   (!q_cos) != (!q_sin)))
        return hk_fail(gpu, "attention with the Q norm in the kernel needs "
                            "the flash kernel (head_dim 128, 16-byte aligned "
                            "operands, no reference or naive mode), "
                            "16-byte aligned weight and tables, and no "
                            "in-kernel RoPE of the unnormalised Q");
    if (fused_qkv && (!flash || rope || q_rows != kv_rows))
        return hk_fail(gpu, "attention on the fused QKV rows needs the flash "
                            "kernel (head_dim 128, 16-byte aligned rows, no "
                            "reference or naive mode), no RoPE tables and "
                            "q_rows == kv_rows");
    if (rope && (!flash || q_rows != kv_rows))
        return hk_fail(gpu, "attention with in-kernel RoPE needs the flash "
                            "kernel (head_dim 128, 16-byte aligned operands, "
                            "no reference or naive mode) and q_rows == "
                            "kv_rows");
    if (flash) {
        const uint64_t lds_bit = 1ull << (gpu->device & 63);
        if (!(hk_attn_lds_ready & lds_bit)) {
            hk_flash_set_lds<false, false>();
            hk_flash_set_lds<false, true>();
            hk_flash_set_lds<false, false, 4>();
            hk_flash_set_lds<true, false, 4>();
            hk_flash_set_lds<true, true, 4>();
            hk_attn_lds_ready |= lds_bit;
        }
        hk_attn_args a;
        a.q = q; a.k = k; a.v = v; a.o = o;
        a.q_rows = q_rows; a.kv_rows = kv_rows; a.heads = heads;
        const bool masked = sparse && gpu->sparse_ptr &&
                            gpu->sparse_rows == q_rows && q_rows == kv_rows;
        if (masked && (kv_rows + HK_KT - 1u) / HK_KT > HK_ATTN_SPARSE_TILES)
            return hk_fail(gpu, "block-sparse attention takes at most %u "
                                "key tiles of %u rows, got %u rows",
                           HK_ATTN_SPARSE_TILES, HK_KT, kv_rows);
        /* Short cross attention (a text of at most 1024 keys) runs 4-wave,
         * 128-query workgroups, two per CU: each workgroup walks few key
         * tiles, so its Q load and O store are a large share of its time,
         * and the second workgroup's tiles overlap them. */
        const bool narrow = !masked && q_rows != kv_rows && kv_rows <= 1024;
        /* Block-sparse attention runs the same 128-query workgroups: each
         * then walks its own query block's tile list.  A 256-query
         * workgroup would walk the union of two blocks' lists, and where they
         * differ (the window mask keeps 38 and 27 of 38 tiles in adjacent
         * blocks) half of its waves idle on the other block's tiles. */
        const bool four = narrow || masked;
        const uint32_t qb_rows = four ? 128u : HK_QB;
        a.q_blocks = (q_rows + qb_rows - 1) / qb_rows;
        a.q_bytes = (uint32_t)q_bytes;
        a.kv_bytes = (uint32_t)kv_bytes;
        a.v_bytes = (uint32_t)v_bytes;
        a.in_stride = (uint32_t)in_stride;
        a.q_norm = q_norm;
        a.q_cos = q_cos;
        a.q_sin = q_sin;
        a.q_eps = q_eps;
        a.scale_log2 = scale * 1.4426950408889634f;
        a.head_major = head_major;
        a.sparse_ptr = masked ? gpu->sparse_ptr : NULL;
        a.sparse_idx = masked ? gpu->sparse_idx : NULL;
        a.sparse_blocks = (q_rows + 127u) / 128u;
        a.rope_pk = NULL;
        a.rope_bytes = rope ? q_rows * HK_ROPE_HALF * 8u : 0u;
        const uint32_t units = a.q_blocks * heads;
        a.full_units = units;
        a.pieces = 1;
        a.part_o = a.part_ml = NULL;
        /* With one workgroup per CU the items run in rounds of num_cus.  A
         * sparse last round (the H3 block at 2378 rows: 560 items = 2
         * rounds + 48) is cut along the keys into pieces that fill the
         * CUs, when that takes at most 0.6 of a round instead of one; a
         * combine kernel merges the pieces' partial softmax. */
        const uint32_t cus = (gpu->num_cus > 0 ? (uint32_t)gpu->num_cus
                                               : 256u) *
                             (four ? 2u : (uint32_t)HK_WG_PER_CU);
        const uint32_t kv_tiles = (kv_rows + HK_KT - 1) / HK_KT;
        const uint32_t tail = units % cus;
        uint32_t pieces = 1;
        float best = 1.0f;
        for (uint32_t s = 2; tail && s <= 8 && kv_tiles >= 2 * s; s++) {
            const float cost = (float)((tail * s + cus - 1) / cus) / (float)s;
            if (cost < best - 1e-6f) {
                best = cost;
                pieces = s;
            }
        }
        if (best > 0.6f || narrow) pieces = 1;
        /* scratch: the packed RoPE table, the rotated keys, then the split
         * pieces' partials */
        const size_t table_bytes = ((size_t)a.rope_bytes + 255) & ~(size_t)255;
        const size_t keys_bytes = rope ? ((kv_bytes + 255) & ~(uint64_t)255) : 0;
        size_t parts = 0;
        if (pieces > 1) {
            /* every piece non-empty */
            const uint32_t per = (kv_tiles + pieces - 1) / pieces;
            pieces = (kv_tiles + per - 1) / per;
            parts = (size_t)tail * pieces;
        }
        const size_t part_bytes = parts * qb_rows * (HK_HD + 2) * sizeof(float);
        if (table_bytes + keys_bytes + part_bytes) {
            uint8_t *buf = (uint8_t *)hk_splitk_space(
                gpu, table_bytes + keys_bytes + part_bytes);
            if (!buf) return 0;
            if (rope) {
                a.rope_pk = (const uint64_t *)buf;
                const uint32_t count = q_rows * HK_ROPE_HALF;
                hipLaunchKernelGGL(hk_rope_pack, dim3((count + 255) / 256),
                                   dim3(256), 0, gpu->stream, rope_cos,
                                   rope_sin, (uint64_t *)buf, count);
                uint16_t *keys = (uint16_t *)(buf + table_bytes);
                const uint32_t threads = kv_rows * heads * 8u;
                hipLaunchKernelGGL(hk_rope_keys, dim3((threads + 255) / 256),
                                   dim3(256), 0, gpu->stream, k,
                                   (const uint64_t *)buf, keys, kv_rows,
                                   heads);
                a.k = keys;
            }
            if (parts) {
                float *pf = (float *)(buf + table_bytes + keys_bytes);
                a.part_o = pf;
                a.part_ml = pf + parts * qb_rows * HK_HD;
                a.full_units = units - tail;
                a.pieces = pieces;
            }
        }
        if (a.full_units)
            hk_flash_launch<false>(gpu, a, masked, a.full_units, four);
        if (pieces > 1) {
            hk_flash_launch<true>(gpu, a, masked, tail * pieces, four);
            if (four)
                hipLaunchKernelGGL(hk_flash_combine<128>,
                                   dim3(tail * (128 / 8)), dim3(256), 0,
                                   gpu->stream, a);
            else
                hipLaunchKernelGGL(hk_flash_combine<HK_QB>,
                                   dim3(tail * (HK_QB / 8)), dim3(256), 0,
                                   gpu->stream, a);
        }
        return 1;
    }
    return hk_attention_reference(gpu, q, k, v, o, q_rows, kv_rows, heads,
                                  head_dim, scale, head_major);
}

extern "C" {

static int hk_sdpa(h3_gpu *gpu, h3_gpu_tensor *output,
                   const h3_gpu_tensor *query, const h3_gpu_tensor *key,
                   const h3_gpu_tensor *value, uint32_t q_rows,
                   uint32_t kv_rows, uint32_t heads, uint32_t head_dim,
                   float scale, int head_major, int sparse,
                   const char *name) {
    size_t q_count = (size_t)q_rows * heads * head_dim;
    size_t kv_count = (size_t)kv_rows * heads * head_dim;
    if (!hk_require(gpu, query, q_count, H3_GPU_BF16, "SDPA query") ||
        !hk_require(gpu, key, kv_count, H3_GPU_BF16, "SDPA key") ||
        !hk_require(gpu, value, kv_count, H3_GPU_BF16, "SDPA value") ||
        !hk_require(gpu, output, q_count, H3_GPU_BF16, "SDPA output") ||
        !hk_require_active(gpu))
        return 0;
    hk_op_begin(gpu, name);
    if (!hk_attention_bf16(gpu, HK_CBF16(query), HK_CBF16(key),
                           HK_CBF16(value), HK_BF16(output), q_rows, kv_rows,
                           heads, head_dim, scale, head_major, sparse, NULL,
                           NULL))
        return 0;
    return hk_op_end(gpu, name, HK_KIND_SDPA);
}

int h3_gpu_sdpa_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                     const h3_gpu_tensor *query, const h3_gpu_tensor *key,
                     const h3_gpu_tensor *value, uint32_t sequence,
                     uint32_t heads, uint32_t head_dim, float scale) {
    return hk_sdpa(gpu, output, query, key, value, sequence, sequence, heads,
                   head_dim, scale, 0, 1, "attention");
}

int h3_gpu_sdpa_bf16_head_major_output(h3_gpu *gpu, h3_gpu_tensor *output,
                                       const h3_gpu_tensor *query,
                                       const h3_gpu_tensor *key,
                                       const h3_gpu_tensor *value,
                                       uint32_t sequence, uint32_t heads,
                                       uint32_t head_dim, float scale) {
    return hk_sdpa(gpu, output, query, key, value, sequence, sequence, heads,
                   head_dim, scale, 1, 1, "attention");
}

int h3_hip_sdpa_qkv_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                         const h3_gpu_tensor *qkv, uint32_t sequence,
                         uint32_t heads, uint32_t head_dim, float scale) {
    const size_t count = (size_t)sequence * heads * head_dim;
    if (!hk_require(gpu, qkv, count * 3, H3_GPU_BF16, "SDPA QKV") ||
        !hk_require(gpu, output, count, H3_GPU_BF16, "SDPA output") ||
        !hk_require_active(gpu))
        return 0;
    const uint16_t *base = HK_CBF16(qkv);
    const size_t inner = (size_t)heads * head_dim;
    hk_op_begin(gpu, "attention");
    if (!hk_attention_bf16(gpu, base, base + inner, base + 2 * inner,
                           HK_BF16(output), sequence, sequence, heads,
                           head_dim, scale, 0, 1, NULL, NULL, 1))
        return 0;
    return hk_op_end(gpu, "attention", HK_KIND_SDPA);
}

int h3_hip_sdpa_qkv_norm_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                   const h3_gpu_tensor *qkv,
                                   const h3_gpu_tensor *q_norm,
                                   const h3_gpu_tensor *rope_cos,
                                   const h3_gpu_tensor *rope_sin,
                                   uint32_t sequence, uint32_t heads,
                                   uint32_t head_dim, uint32_t rope_half,
                                   float epsilon, float scale) {
    const size_t count = (size_t)sequence * heads * head_dim;
    if (!hk_require(gpu, qkv, count * 3, H3_GPU_BF16, "SDPA QKV") ||
        !hk_require(gpu, output, count, H3_GPU_BF16, "SDPA output") ||
        !hk_require(gpu, q_norm, head_dim, H3_GPU_BF16, "Q norm") ||
        (rope_cos && !hk_require(gpu, rope_cos, (size_t)sequence * rope_half,
                                 H3_GPU_BF16, "RoPE cos")) ||
        (rope_sin && !hk_require(gpu, rope_sin, (size_t)sequence * rope_half,
                                 H3_GPU_BF16, "RoPE sin")) ||
        !hk_require_active(gpu))
        return 0;
    if (head_dim != HK_HD || (rope_cos && rope_half != HK_ROPE_HALF) ||
        (!rope_cos) != (!rope_sin))
        return hk_fail(gpu, "attention with the Q norm in the kernel supports "
                            "head_dim 128 and RoPE tables of rope_half 48 "
                            "(got %u / %u)", head_dim, rope_half);
    const uint16_t *base = HK_CBF16(qkv);
    const size_t inner = (size_t)heads * head_dim;
    hk_op_begin(gpu, "attention");
    if (!hk_attention_bf16(gpu, base, base + inner, base + 2 * inner,
                           HK_BF16(output), sequence, sequence, heads,
                           head_dim, scale, 0, 1, NULL, NULL, 1,
                           HK_CBF16(q_norm),
                           rope_cos ? HK_CBF16(rope_cos) : NULL,
                           rope_sin ? HK_CBF16(rope_sin) : NULL, epsilon))
        return 0;
    return hk_op_end(gpu, "attention", HK_KIND_SDPA);
}

int h3_hip_sdpa_cross_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                                const h3_gpu_tensor *query,
                                const h3_gpu_tensor *key,
                                const h3_gpu_tensor *value,
                                const h3_gpu_tensor *q_norm, uint32_t q_rows,
                                uint32_t kv_rows, uint32_t heads,
                                uint32_t head_dim, float epsilon,
                                float scale) {
    const size_t qc = (size_t)q_rows * heads * head_dim;
    const size_t kc = (size_t)kv_rows * heads * head_dim;
    if (!hk_require(gpu, query, qc, H3_GPU_BF16, "SDPA query") ||
        !hk_require(gpu, key, kc, H3_GPU_BF16, "SDPA key") ||
        !hk_require(gpu, value, kc, H3_GPU_BF16, "SDPA value") ||
        !hk_require(gpu, output, qc, H3_GPU_BF16, "SDPA output") ||
        !hk_require(gpu, q_norm, head_dim, H3_GPU_BF16, "Q norm") ||
        !hk_require_active(gpu))
        return 0;
    if (head_dim != HK_HD)
        return hk_fail(gpu, "attention with the Q norm in the kernel supports "
                            "head_dim 128 (got %u)", head_dim);
    hk_op_begin(gpu, "attention_cross");
    if (!hk_attention_bf16(gpu, HK_CBF16(query), HK_CBF16(key),
                           HK_CBF16(value), HK_BF16(output), q_rows, kv_rows,
                           heads, head_dim, scale, 0, 0, NULL, NULL, 0,
                           HK_CBF16(q_norm), NULL, NULL, epsilon))
        return 0;
    return hk_op_end(gpu, "attention_cross", HK_KIND_SDPA);
}

int h3_hip_sdpa_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                          const h3_gpu_tensor *query,
                          const h3_gpu_tensor *key,
                          const h3_gpu_tensor *value,
                          const h3_gpu_tensor *rope_cos,
                          const h3_gpu_tensor *rope_sin, uint32_t sequence,
                          uint32_t heads, uint32_t head_dim,
                          uint32_t rope_half, float scale) {
    const size_t count = (size_t)sequence * heads * head_dim;
    if (!hk_require(gpu, query, count, H3_GPU_BF16, "SDPA query") ||
        !hk_require(gpu, key, count, H3_GPU_BF16, "SDPA key") ||
        !hk_require(gpu, value, count, H3_GPU_BF16, "SDPA value") ||
        !hk_require(gpu, output, count, H3_GPU_BF16, "SDPA output") ||
        !hk_require(gpu, rope_cos, (size_t)sequence * rope_half, H3_GPU_BF16,
                    "RoPE cos") ||
        !hk_require(gpu, rope_sin, (size_t)sequence * rope_half, H3_GPU_BF16,
                    "RoPE sin") ||
        !hk_require_active(gpu))
        return 0;
    if (rope_half != HK_ROPE_HALF || head_dim != HK_HD)
        return hk_fail(gpu, "attention with in-kernel RoPE supports head_dim "
                            "128 with rope_half 48 (got %u / %u)", head_dim,
                       rope_half);
    hk_op_begin(gpu, "attention_rope");
    if (!hk_attention_bf16(gpu, HK_CBF16(query), HK_CBF16(key),
                           HK_CBF16(value), HK_BF16(output), sequence,
                           sequence, heads, head_dim, scale, 0, 1,
                           HK_CBF16(rope_cos), HK_CBF16(rope_sin)))
        return 0;
    return hk_op_end(gpu, "attention_rope", HK_KIND_SDPA);
}

int h3_gpu_sdpa_cross_bf16(h3_gpu *gpu, h3_gpu_tensor *output,
                           const h3_gpu_tensor *query,
                           const h3_gpu_tensor *key,
                           const h3_gpu_tensor *value, uint32_t q_rows,
                           uint32_t kv_rows, uint32_t heads,
                           uint32_t head_dim, float scale) {
    return hk_sdpa(gpu, output, query, key, value, q_rows, kv_rows, heads,
                   head_dim, scale, 0, 0, "attention_cross");
}

} /* extern "C" */
