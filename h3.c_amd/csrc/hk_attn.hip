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
 *     key order (two 8-byte LDS reads), so P never goes through LDS;
 *   - V is transposed once per tile while being staged into LDS
 *     (V^T rows of 64 keys, 136-byte pitch), K is staged row-major with an
 *     XOR swizzle on 16-byte chunks;
 *   - 8 wave64s x 32 queries = 256 queries per workgroup, 64-key tiles,
 *     double-buffered LDS (2 x 33 KiB) with the next tile's global loads in
 *     flight during the current tile's 32 MFMAs per wave.  At 32 queries a
 *     wave needs under 256 registers, so two waves share each SIMD and the
 *     hardware overlaps one wave's softmax (VALU) with the other's MFMAs;
 *   - the grid is 1-D and regrouped per XCD so the query blocks of one head
 *     run on one XCD and share its L2 copy of that head's K and V;
 *   - the softmax is VALU-bound, so its instruction count is kept low: the
 *     running max only moves (rescaling O and l) when a tile's max exceeds
 *     it by more than 2^8, the scale is folded into one FMA per score, row
 *     maxima take two scores per med3 (compiler-visible, so the MFMA ->
 *     VALU result hazards get their wait states), and the key-range mask
 *     is compiled only into the last tile's step.
 *
 * A two-pass reference kernel (hk_attn_ref.hip, built with the default
 * floating-point semantics) serves other head sizes, H3_HIP_REFERENCE=1 and
 * the naive-SDPA knob.
 */
#include "hk_common.h"
#include "hk_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <type_traits>

#define HK_HD 128
#define HK_QG 1               /* 32-query groups per wave */
#define HK_WAVES 8            /* waves per workgroup (two per SIMD) */
#define HK_THREADS (HK_WAVES * 64)
#define HK_QB (HK_WAVES * 32 * HK_QG) /* queries per workgroup */
#define HK_KPT (64 / (HK_THREADS / 16)) /* staged key rows per thread */
#define HK_KT 64              /* keys per tile */
#define HK_K_BYTES (HK_KT * HK_HD * 2)        /* 16 KiB, 256-B rows */
#define HK_VT_PITCH 136                        /* bytes per V^T row */
#define HK_VT_BYTES (HK_HD * HK_VT_PITCH)      /* 17 KiB */
#define HK_STAGE_BYTES (HK_K_BYTES + HK_VT_BYTES)
#define HK_ATTN_LDS (2 * HK_STAGE_BYTES)

typedef int hk_v4i __attribute__((ext_vector_type(4)));
typedef int hk_v2i __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t hk_attn_rsrc(
    const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base),
                                             (short)0, (int)bytes,
                                             0x00020000);
}

/* K tile: row = key (256 B), 16 chunks, chunk ^= row & 15 */
__device__ __forceinline__ uint32_t hk_k_swz(uint32_t row, uint32_t chunk) {
    return row * 256u + ((chunk ^ (row & 15u)) << 4);
}

struct hk_attn_args {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    uint32_t q_rows, kv_rows, heads, q_blocks;
    uint32_t q_bytes, kv_bytes;
    float scale_log2;
    int head_major;
    /* block-sparse mask: CSR over 128-row query blocks of 64-row key tiles
     * (lists sorted), or null for dense */
    const uint32_t *sparse_ptr, *sparse_idx;
    uint32_t sparse_blocks; /* query blocks in the CSR */
    /* split launch (SPLIT): work item full_units + pid / pieces, key tiles
     * of piece pid % pieces; unnormalised f32 O into part_o[pid][256][128],
     * (running max in the exp2 domain, sum) into part_ml[pid][256] */
    uint32_t full_units, pieces;
    float *part_o, *part_ml;
};

template <bool SPARSE, bool SPLIT>
__global__ void __launch_bounds__(HK_THREADS, 1) hk_flash_fwd(hk_attn_args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t hk_lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t col = lane & 31u, half = lane >> 5;

    uint32_t pid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) pid = (pid & 7u) * (nwg >> 3) + (pid >> 3);
    const uint32_t item = SPLIT ? a.full_units + pid / a.pieces : pid;
    const uint32_t qblock = item % a.q_blocks, head = item / a.q_blocks;
    const uint32_t row_stride = a.heads * HK_HD; /* elements */

    const __amdgpu_buffer_rsrc_t qr = hk_attn_rsrc(a.q, a.q_bytes);
    const __amdgpu_buffer_rsrc_t kr = hk_attn_rsrc(a.k, a.kv_bytes);
    const __amdgpu_buffer_rsrc_t vr = hk_attn_rsrc(a.v, a.kv_bytes);

    /* ---- Q fragments: B operand of S^T = K . Q^T ----
     * group g, k-step ks: Q[q][16 ks + 8 half .. +8] */
    const uint32_t qbase = qblock * HK_QB + wave * (32u * HK_QG);
    hk_bf16x8 qf[HK_QG][8];
#pragma unroll
    for (int g = 0; g < HK_QG; g++) {
        const uint32_t q = qbase + g * 32u + col;
        const uint32_t off = q < a.q_rows
            ? ((q * row_stride + head * HK_HD + half * 8u) * 2u)
            : 0xfffffff0u;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            hk_v4i raw = __builtin_amdgcn_raw_buffer_load_b128(
                qr, off == 0xfffffff0u ? off : off + ks * 32u, 0, 0);
            qf[g][ks] = __builtin_bit_cast(hk_bf16x8, raw);
        }
    }

    /* ---- staging plan ----
     * K: thread t loads chunk (t & 15) of key rows (t >> 4) + 16 i
     * V: thread t loads chunk dc = t & 15 of key rows 4 kg .. 4 kg + 3,
     *    kg = t >> 4, and writes them transposed */
    const uint32_t sc = tid & 15u, sr = tid >> 4;
    hk_v4i kreg[HK_KPT], vreg[HK_KPT];
    auto load_tile = [&](uint32_t kv0) {
#pragma unroll
        for (int i = 0; i < HK_KPT; i++) {
            const uint32_t krow = kv0 + sr + (HK_THREADS / 16u) * i;
            const uint32_t koff = krow < a.kv_rows
                ? ((krow * row_stride + head * HK_HD + sc * 8u) * 2u)
                : 0xfffffff0u;
            kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, koff, 0, 0);
            const uint32_t vrow = kv0 + sr * HK_KPT + i;
            const uint32_t voff = vrow < a.kv_rows
                ? ((vrow * row_stride + head * HK_HD + sc * 8u) * 2u)
                : 0xfffffff0u;
            vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, voff, 0, 0);
        }
    };
    auto store_tile = [&](uint32_t stage) {
        uint8_t *ks = hk_lds + stage * HK_STAGE_BYTES;
        uint8_t *vt = ks + HK_K_BYTES;
#pragma unroll
        for (int i = 0; i < HK_KPT; i++)
            *(hk_v4i *)(ks + hk_k_swz(sr + (HK_THREADS / 16u) * i, sc)) =
                kreg[i];
        /* transpose KPT keys x 8 dims -> 8 rows of KPT keys */
        const uint16_t *v16[HK_KPT];
#pragma unroll
        for (int i = 0; i < HK_KPT; i++) v16[i] = (const uint16_t *)&vreg[i];
#pragma unroll
        for (int d = 0; d < 8; d++) {
            uint8_t *dst = vt + (sc * 8u + d) * HK_VT_PITCH + sr * (2u * HK_KPT);
            if (HK_KPT == 4) {
                uint2 packed;
                packed.x = (uint32_t)v16[0][d] | ((uint32_t)v16[1][d] << 16);
                packed.y = (uint32_t)v16[2][d] | ((uint32_t)v16[3][d] << 16);
                *(uint2 *)dst = packed;
            } else {
                *(uint32_t *)dst =
                    (uint32_t)v16[0][d] | ((uint32_t)v16[HK_KPT - 1][d] << 16);
            }
        }
    };

    hk_f32x16 o[4][HK_QG];
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
        for (int g = 0; g < HK_QG; g++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[d][g][r] = 0.0f;
    float m_run[HK_QG], l_part[HK_QG];
#pragma unroll
    for (int g = 0; g < HK_QG; g++) {
        m_run[g] = -INFINITY;
        l_part[g] = 0.0f;
    }

    /* ---- key-tile schedule ----
     * Dense: every 64-key tile in order.  Block-sparse: the workgroup's
     * 256 queries are two 128-row query blocks of the CSR; it walks the
     * merged (sorted) union of their tile lists, staging each tile once,
     * and waves 0-3 (first block) / 4-7 (second block) run the MFMAs and
     * softmax only on tiles of their own block's list.  A list's length is
     * clamped to the dense tile count, as in the reference kernel. */
    const uint32_t all_tiles = (a.kv_rows + HK_KT - 1) / HK_KT;
    /* a split piece covers key tiles [first_tile, dense) */
    const uint32_t piece_tiles =
        SPLIT ? (all_tiles + a.pieces - 1) / a.pieces : all_tiles;
    const uint32_t first_tile = SPLIT ? (pid % a.pieces) * piece_tiles : 0;
    const uint32_t dense =
        SPLIT ? min(all_tiles, first_tile + piece_tiles) : all_tiles;
    uint32_t dense_next = first_tile, ia = 0, ea = 0, ib = 0, eb = 0;
    if (SPARSE) {
        const uint32_t qa = qblock * 2u, qb = qa + 1u;
        ia = a.sparse_ptr[qa];
        ea = min(a.sparse_ptr[qa + 1], ia + all_tiles);
        if (qb < a.sparse_blocks) {
            ib = a.sparse_ptr[qb];
            eb = min(a.sparse_ptr[qb + 1], ib + all_tiles);
        }
        if (SPLIT) {
            /* this piece's key tiles [first_tile, dense) of the sorted
             * lists */
            while (ia < ea && a.sparse_idx[ia] < first_tile) ia++;
            uint32_t e = ia;
            while (e < ea && a.sparse_idx[e] < dense) e++;
            ea = e;
            while (ib < eb && a.sparse_idx[ib] < first_tile) ib++;
            e = ib;
            while (e < eb && a.sparse_idx[e] < dense) e++;
            eb = e;
        }
    }
    const bool first_block = wave < HK_WAVES / 2;
    /* next tile of the schedule: false when done; in_a / in_b say whose
     * list holds it */
    auto advance = [&](uint32_t &tile, bool &in_a, bool &in_b) -> bool {
        if (!SPARSE) {
            if (dense_next >= dense) return false;
            tile = dense_next++;
            in_a = in_b = true;
            return true;
        }
        const uint32_t ta = ia < ea ? a.sparse_idx[ia] : 0xffffffffu;
        const uint32_t tb = ib < eb ? a.sparse_idx[ib] : 0xffffffffu;
        if (ta == 0xffffffffu && tb == 0xffffffffu) return false;
        tile = min(ta, tb);
        in_a = ta == tile;
        in_b = tb == tile;
        if (in_a) ia++;
        if (in_b) ib++;
        return true;
    };
    uint32_t cur = 0, nxt = 0;
    bool cur_a = false, cur_b = false, nxt_a = false, nxt_b = false;
    bool have = advance(cur, cur_a, cur_b);
    if (have) {
        load_tile(cur * HK_KT);
        store_tile(0);
    }
    __syncthreads();

    auto tile_step = [&](uint32_t t, uint32_t tile, uint32_t next_tile,
                         bool more, bool mine, auto tail_tag) {
        constexpr bool tail = decltype(tail_tag)::value;
        const uint32_t stage = t & 1u;
        if (more) load_tile(next_tile * HK_KT);
        const uint8_t *ks = hk_lds + stage * HK_STAGE_BYTES;
        const uint8_t *vt = ks + HK_K_BYTES;

        if (mine) {
        /* S^T[kt][g]: keys kt*32 + .., queries g*32 + col */
        hk_f32x16 s[2][HK_QG];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int g = 0; g < HK_QG; g++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[kt][g][r] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                hk_bf16x8 kf = *(const hk_bf16x8 *)(
                    ks + hk_k_swz(kt * 32u + col, kk * 2u + half));
#pragma unroll
                for (int g = 0; g < HK_QG; g++)
                    s[kt][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        kf, qf[g][kk], s[kt][g], 0, 0, 0);
            }
        }

        /* online softmax per query column.  The running maximum is only
         * moved (and O, l rescaled) when a score exceeds it by more than
         * 2^8 in the exp2 domain; otherwise P = exp2(s - m_stale) <= 256.
         * The stale maximum is not the row's true maximum and the gap
         * between them is not a power of two, so bf16(P) can round
         * differently from the reference's P (relative to the row maximum)
         * by up to half a bf16 ulp per element: O matches to the bf16
         * rounding of P (the bound the tests apply), while l, summed over
         * the unrounded P, is exact up to f32 rounding. */
        const uint32_t kv0 = tile * HK_KT;
        hk_bf16x8 pf[2][2][HK_QG]; /* [kt][step][g] */
#pragma unroll
        for (int g = 0; g < HK_QG; g++) {
            float mx = -INFINITY;
            if constexpr (tail) {
#pragma unroll
                for (int kt = 0; kt < 2; kt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const uint32_t key = kv0 + kt * 32u + (r >> 2) * 8u +
                                             half * 4u + (r & 3);
                        if (key >= a.kv_rows) s[kt][g][r] = -INFINITY;
                    }
            }
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r += 2)
                    mx = __builtin_fmaxf(
                        mx, __builtin_fmaxf(s[kt][g][r], s[kt][g][r + 1]));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * a.scale_log2;
            const bool grow = mx > m_run[g] + 8.0f;
            if (__builtin_amdgcn_ballot_w64(grow)) {
                const float m_new = fmaxf(m_run[g], mx);
                const float ref = m_new == -INFINITY ? 0.0f : m_new;
                const float c = __builtin_amdgcn_exp2f(m_run[g] - ref);
                m_run[g] = ref;
                l_part[g] *= c;
#pragma unroll
                for (int d = 0; d < 4; d++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[d][g][r] *= c;
            }
            const float neg = -m_run[g];
            float sum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; kt++) {
                float p[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = __builtin_amdgcn_exp2f(
                        __builtin_fmaf(s[kt][g][r], a.scale_log2, neg));
                    sum += p[r];
                }
#pragma unroll
                for (int st = 0; st < 2; st++) {
                    hk_bf16x8 v;
#pragma unroll
                    for (int e = 0; e < 8; e++) v[e] = (__bf16)p[st * 8 + e];
                    pf[kt][st][g] = v;
                }
            }
            l_part[g] += sum;
        }

        /* O^T[d][g] += V^T[d, keys] . P^T[keys, g] */
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const uint32_t key = kt * 32u + st * 16u + half * 4u;
#pragma unroll
                for (int d = 0; d < 4; d++) {
                    const uint8_t *row = vt + (d * 32u + col) * HK_VT_PITCH;
                    hk_v2i lo = *(const hk_v2i *)(row + key * 2u);
                    hk_v2i hi = *(const hk_v2i *)(row + (key + 8u) * 2u);
                    hk_v4i both = {lo[0], lo[1], hi[0], hi[1]};
                    hk_bf16x8 vf = __builtin_bit_cast(hk_bf16x8, both);
#pragma unroll
                    for (int g = 0; g < HK_QG; g++)
                        o[d][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            vf, pf[kt][st][g], o[d][g], 0, 0, 0);
                }
            }
        } /* mine */

        if (more) store_tile(stage ^ 1u);
        __syncthreads();
    };
    /* the key-range mask is compiled only into the step of the last dense
     * tile, the only tile with keys past kv_rows */
    if constexpr (!SPARSE) {
        for (uint32_t t = first_tile; t + 1 < dense; t++)
            tile_step(t - first_tile, t, t + 1, true, true,
                      std::integral_constant<bool, false>());
        tile_step(dense - 1 - first_tile, dense - 1, 0, false, true,
                  std::integral_constant<bool, true>());
    } else {
        for (uint32_t t = 0; have; t++) {
            const bool more = advance(nxt, nxt_a, nxt_b);
            const bool mine = first_block ? cur_a : cur_b;
            /* one instantiation (register pressure): the key-range mask is
             * a no-op except on the last dense tile */
            tile_step(t, cur, nxt, more, mine,
                      std::integral_constant<bool, true>());
            cur = nxt;
            cur_a = nxt_a;
            cur_b = nxt_b;
            have = more;
        }
    }

    if constexpr (SPLIT) {
        /* unnormalised partials for the combine kernel */
#pragma unroll
        for (int g = 0; g < HK_QG; g++) {
            const uint32_t ql = wave * (32u * HK_QG) + g * 32u + col;
            float *po = a.part_o + ((size_t)pid * HK_QB + ql) * HK_HD;
#pragma unroll
            for (int d = 0; d < 4; d++)
#pragma unroll
                for (int blk = 0; blk < 4; blk++)
                    *(float4 *)(po + d * 32u + blk * 8u + half * 4u) =
                        make_float4(o[d][g][blk * 4 + 0], o[d][g][blk * 4 + 1],
                                    o[d][g][blk * 4 + 2], o[d][g][blk * 4 + 3]);
            const float l = l_part[g] + __shfl_xor(l_part[g], 32, 64);
            if (half == 0)
                *(float2 *)(a.part_ml + ((size_t)pid * HK_QB + ql) * 2u) =
                    make_float2(m_run[g], l);
        }
        return;
    }
    /* ---- normalise and store: lane owns query column `col` of group g and
     * dims d*32 + (r/4)*8 + 4*half + r%4 */
#pragma unroll
    for (int g = 0; g < HK_QG; g++) {
        const float l = l_part[g] + __shfl_xor(l_part[g], 32, 64);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const uint32_t q = qbase + g * 32u + col;
        if (q >= a.q_rows) continue;
        uint16_t *out = a.head_major
            ? a.o + ((size_t)head * a.q_rows + q) * HK_HD
            : a.o + (size_t)q * row_stride + (size_t)head * HK_HD;
#pragma unroll
        for (int d = 0; d < 4; d++)
#pragma unroll
            for (int blk = 0; blk < 4; blk++) {
                const uint32_t dim = d * 32u + blk * 8u + half * 4u;
                uint2 packed = {
                    hk_pack2(o[d][g][blk * 4 + 0] * inv,
                             o[d][g][blk * 4 + 1] * inv),
                    hk_pack2(o[d][g][blk * 4 + 2] * inv,
                             o[d][g][blk * 4 + 3] * inv)};
                *(uint2 *)(out + dim) = packed;
            }
    }
}

/* Combines the key-range pieces of the split work items: per query, with
 * the pieces' running maxima m_p (exp2 domain), sums l_p and unnormalised
 * O_p, O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p, M = max_p m_p.
 * 8 queries per workgroup, 4 dims per thread. */
__global__ void __launch_bounds__(256) hk_flash_combine(hk_attn_args a) {
    const uint32_t titem = blockIdx.x >> 5;
    const uint32_t ql = (blockIdx.x & 31u) * 8u + (threadIdx.x >> 5);
    const uint32_t d4 = (threadIdx.x & 31u) * 4u;
    const uint32_t item = a.full_units + titem;
    const uint32_t qblock = item % a.q_blocks, head = item / a.q_blocks;
    const uint32_t q = qblock * HK_QB + ql;
    if (q >= a.q_rows) return;
    const size_t first = (size_t)titem * a.pieces;
    float top = -INFINITY;
    for (uint32_t p = 0; p < a.pieces; p++)
        top = fmaxf(top, a.part_ml[((first + p) * HK_QB + ql) * 2u]);
    float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float l = 0.0f;
    for (uint32_t p = 0; p < a.pieces; p++) {
        const float2 ml =
            *(const float2 *)(a.part_ml + ((first + p) * HK_QB + ql) * 2u);
        /* a sparse piece may hold no key tile of this query block */
        const float w =
            ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - top);
        const float4 op = *(const float4 *)(a.part_o +
                                            ((first + p) * HK_QB + ql) * HK_HD +
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
/* the comma in a template argument list confuses hipLaunchKernelGGL */
#define HK_FLASH(sparse, split) (hk_flash_fwd<sparse, split>)

int hk_attention_bf16(struct h3_gpu *gpu, const uint16_t *q,
                      const uint16_t *k, const uint16_t *v, uint16_t *o,
                      uint32_t q_rows, uint32_t kv_rows, uint32_t heads,
                      uint32_t head_dim, float scale, int head_major,
                      int sparse) {
    if (!q_rows || !heads) return 1;
    const uint64_t q_bytes = (uint64_t)q_rows * heads * head_dim * 2;
    const uint64_t kv_bytes = (uint64_t)kv_rows * heads * head_dim * 2;
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
    if (flash) {
        const uint64_t lds_bit = 1ull << (gpu->device & 63);
        if (!(hk_attn_lds_ready & lds_bit)) {
            (void)hipFuncSetAttribute(
                (const void *)hk_flash_fwd<false, false>,
                hipFuncAttributeMaxDynamicSharedMemorySize, HK_ATTN_LDS);
            (void)hipFuncSetAttribute(
                (const void *)hk_flash_fwd<true, false>,
                hipFuncAttributeMaxDynamicSharedMemorySize, HK_ATTN_LDS);
            (void)hipFuncSetAttribute(
                (const void *)hk_flash_fwd<false, true>,
                hipFuncAttributeMaxDynamicSharedMemorySize, HK_ATTN_LDS);
            (void)hipFuncSetAttribute(
                (const void *)hk_flash_fwd<true, true>,
                hipFuncAttributeMaxDynamicSharedMemorySize, HK_ATTN_LDS);
            hk_attn_lds_ready |= lds_bit;
        }
        hk_attn_args a;
        a.q = q; a.k = k; a.v = v; a.o = o;
        a.q_rows = q_rows; a.kv_rows = kv_rows; a.heads = heads;
        a.q_blocks = (q_rows + HK_QB - 1) / HK_QB;
        a.q_bytes = (uint32_t)q_bytes;
        a.kv_bytes = (uint32_t)kv_bytes;
        a.scale_log2 = scale * 1.4426950408889634f;
        a.head_major = head_major;
        const bool masked = sparse && gpu->sparse_ptr &&
                            gpu->sparse_rows == q_rows && q_rows == kv_rows;
        a.sparse_ptr = masked ? gpu->sparse_ptr : NULL;
        a.sparse_idx = masked ? gpu->sparse_idx : NULL;
        a.sparse_blocks = (q_rows + 127u) / 128u;
        const uint32_t units = a.q_blocks * heads;
        a.full_units = units;
        a.pieces = 1;
        a.part_o = a.part_ml = NULL;
        /* With one workgroup per CU the items run in rounds of num_cus.  A
         * sparse last round (the H3 block at 2378 rows: 560 items = 2
         * rounds + 48) is cut along the keys into pieces that fill the
         * CUs, when that takes at most 0.6 of a round instead of one; a
         * combine kernel merges the pieces' partial softmax. */
        const uint32_t cus = gpu->num_cus > 0 ? (uint32_t)gpu->num_cus : 256u;
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
        if (best > 0.6f) pieces = 1;
        if (pieces > 1) {
            /* every piece non-empty */
            const uint32_t per = (kv_tiles + pieces - 1) / pieces;
            pieces = (kv_tiles + per - 1) / per;
            const size_t parts = (size_t)tail * pieces;
            float *buf = (float *)hk_splitk_space(
                gpu, parts * HK_QB * (HK_HD + 2) * sizeof(float));
            if (!buf) return 0;
            a.part_o = buf;
            a.part_ml = buf + parts * HK_QB * HK_HD;
            a.full_units = units - tail;
            a.pieces = pieces;
        }
        if (a.full_units) {
            if (masked)
                hipLaunchKernelGGL(HK_FLASH(true, false), dim3(a.full_units),
                                   dim3(HK_THREADS), HK_ATTN_LDS, gpu->stream,
                                   a);
            else
                hipLaunchKernelGGL(HK_FLASH(false, false), dim3(a.full_units),
                                   dim3(HK_THREADS), HK_ATTN_LDS, gpu->stream,
                                   a);
        }
        if (pieces > 1) {
            if (masked)
                hipLaunchKernelGGL(HK_FLASH(true, true), dim3(tail * pieces),
                                   dim3(HK_THREADS), HK_ATTN_LDS, gpu->stream,
                                   a);
            else
                hipLaunchKernelGGL(HK_FLASH(false, true), dim3(tail * pieces),
                                   dim3(HK_THREADS), HK_ATTN_LDS, gpu->stream,
                                   a);
            hipLaunchKernelGGL(hk_flash_combine, dim3(tail * 32), dim3(256),
                               0, gpu->stream, a);
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
                           heads, head_dim, scale, head_major, sparse))
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
