/* Shared by the flash attention kernels: the launch arguments, the LDS
 * tile swizzles, the buffer resources and the V^T fragment reads. */
#pragma once
#include "hk_common.h"

#define HK_HD 128
#define HK_KT 64                          /* keys per tile */
#define HK_TILE_BYTES (HK_KT * HK_HD * 2) /* 16 KiB, 256-B rows */
#define HK_ROPE_HALF 48 /* RoPE pairs (d, d + 48), d < 48 */

typedef int hk_v4i __attribute__((ext_vector_type(4)));
typedef int hk_v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void hk_lds_void;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t hk_attn_rsrc(
    const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base),
                                             (short)0, (int)bytes,
                                             0x00020000);
}

/* K tile: row = key (256 B = 16 chunks of 16 B); logical chunk c of row r
 * sits at physical chunk c ^ (r & 15), so the 32-key fragment reads (one
 * chunk of 16 consecutive rows per 16 lanes) hit 16 distinct chunks. */
__device__ __forceinline__ uint32_t hk_k_swz(uint32_t row, uint32_t chunk) {
    return row * 256u + ((chunk ^ (row & 15u)) << 4);
}

/* V tile: row-major like K, chunk c of row r at c ^ 4 (r & 3).  The
 * transposing reads take 4 consecutive rows x 32 B per 16 lanes; the XOR
 * puts the four rows' 32-byte pieces in four different 64-byte bank
 * groups. */
__device__ __forceinline__ uint32_t hk_v_swz(uint32_t row, uint32_t chunk) {
    return row * 256u + ((chunk ^ ((row & 3u) << 2)) << 4);
}

/* The transposing V^T fragment reads of one 16-key step (rows base ..
 * base + 15 of the V tile at LDS offset `off`): for each 32-dim block d,
 * two ds_read_b64_tr_b16 (keys 0-7 of the step at lo, 8-15 at hi).  They
 * are inline assembly because the compiler's wait insertion takes the
 * ds_read_tr builtin as possibly aliasing the direct-to-LDS loads in
 * flight and waits for all of them (vmcnt(0)) first -- the next tile's
 * loads, which then no longer overlap the current tile.  Their completion
 * is the caller's to wait for, with hk_vt_wait. */
__device__ __forceinline__ void hk_vt_read(hk_v2i (&vt)[4][2],
                                           const uint32_t (&v_frag)[4],
                                           uint32_t off) {
#pragma unroll
    for (int d = 0; d < 4; d++)
        asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\t"
                     "ds_read_b64_tr_b16 %1, %2 offset:%4"
                     : "=v"(vt[d][0]), "=v"(vt[d][1])
                     : "v"(v_frag[d]), "i"(off), "i"(off + 8u * 256u));
}

/* Waits until at most N LDS operations are outstanding, which completes
 * the reads of vt when N more were issued after them. */
template <int N>
__device__ __forceinline__ void hk_vt_wait(hk_v2i (&vt)[4][2]) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(vt[0][0]), "+v"(vt[0][1]), "+v"(vt[1][0]),
                   "+v"(vt[1][1]), "+v"(vt[2][0]), "+v"(vt[2][1]),
                   "+v"(vt[3][0]), "+v"(vt[3][1])
                 : "i"(N));
}

struct hk_attn_args {
    const uint16_t *q, *k, *v;
    uint16_t *o;
    uint32_t q_rows, kv_rows, heads, q_blocks;
    /* bytes readable from q, k and v; elements from one Q / K / V row to
     * the next (heads * 128, or 3 heads * 128 when the three are read from
     * the fused QKV projection output) */
    uint32_t q_bytes, kv_bytes, v_bytes, in_stride;
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
    /* RoPE: the joint sequence's cos / sin tables packed per (row, dim) as
     * the two bf16 pairs (c, -s), (s, c) of the rotation ([rows][48]
     * uint64, hk_rope_pack); Q arrives unrotated and is rotated as the
     * kernel loads its fragments, K was rotated by hk_rope_keys */
    const uint64_t *rope_pk;
    uint32_t rope_bytes;
    /* Q_NORM: the per-head RMS norm of Q (weight q_norm[128], epsilon
     * q_eps) applied as the Q fragments are loaded, then, with q_cos /
     * q_sin ([rows][48] bf16), the RoPE pairs (d, d + 48) -- the arithmetic
     * and rounding of hk_head_rms128 / hk_qk_norm_rope128v, so the result
     * equals normalising (and rotating) Q first */
    const uint16_t *q_norm, *q_cos, *q_sin;
    float q_eps;
};

