"""Block-sparse joint attention on the GPU (h3_gpu_sdpa_set_sparse,
reference h3_gpu.h:44-52 and h3_cuda_attention.cu:1652-1673, 1812-1857)
against the oracle, plus the H3 block with the layout's window mask
(h3_dit.c:1006-1132)."""
import ctypes as C
import math

import numpy as np
import pytest

import h3hip
import oracle
from conftest import assert_close, cosine_rel_l2, rand_bf16, \
    sdpa_p_rounding_bound
from test_host_math import layout
from test_sparse_mask import mask

pytestmark = pytest.mark.gpu

L = h3hip.lib()


def register(gpu, ptr, idx, rows):
    p = np.ascontiguousarray(ptr, np.uint32)
    i = np.ascontiguousarray(idx, np.uint32)
    return L.h3_gpu_sdpa_set_sparse(gpu.h, h3hip.ptr(p), p.size,
                                    h3hip.ptr(i), i.size, rows)


def clear(gpu):
    assert L.h3_gpu_sdpa_set_sparse(gpu.h, None, 0, None, 0, 0)


def random_mask(rng, rows, keep=0.5):
    qb, kt = (rows + 127) // 128, (rows + 63) // 64
    ptr, idx = [0], []
    for q in range(qb):
        tiles = [t for t in range(kt) if rng.random() < keep] or [kt - 1]
        rng.shuffle(tiles)                   # registration sorts the lists
        idx += tiles
        ptr.append(len(idx))
    return ptr, idx


@pytest.mark.parametrize("rows,heads,head_major", [(300, 2, False),
                                                    (700, 2, True),
                                                    (512, 1, False)])
def test_sparse_sdpa_matches_oracle(gpu, rows, heads, head_major):
    rng = np.random.default_rng(rows)
    hd = 128
    q, k, v = (rand_bf16(rng, rows * heads * hd) for _ in range(3))
    ptr, idx = random_mask(rng, rows)
    assert register(gpu, ptr, idx, rows), gpu.error()
    try:
        out = gpu.new_bf16(rows * heads * hd)
        scale = 1.0 / math.sqrt(hd)
        name = ("h3_gpu_sdpa_bf16_head_major_output" if head_major
                else "h3_gpu_sdpa_bf16")
        gpu.run(name, out, gpu.bf16(q), gpu.bf16(k), gpu.bf16(v), rows,
                heads, hd, C.c_float(scale))
        want = oracle.sdpa_sparse(q, k, v, rows, heads, hd, scale, ptr, idx,
                                  head_major=head_major)
        assert_close(gpu.read_bf16(out), want, what="sparse SDPA",
                     extra_abs=2 * sdpa_p_rounding_bound(
                         q, k, v, rows, rows, heads, hd, scale, head_major))
    finally:
        clear(gpu)


def test_sparse_split_pieces_with_empty_block(gpu):
    """700 rows, 2 heads: 6 work items on 256 CUs, so each is cut into
    key-range pieces; query block 2 keeps no tile at all (its rows are
    zeros, as in the reference) and block 4 only the last tile (most of its
    pieces are empty)."""
    rows, heads, hd = 700, 2, 128
    rng = np.random.default_rng(41)
    q, k, v = (rand_bf16(rng, rows * heads * hd) for _ in range(3))
    lists = [[0, 3, 7], [1, 2, 10], [], [4, 5, 6, 9], [10], [0, 10]]
    ptr, idx = [0], []
    for tiles in lists:
        idx += tiles
        ptr.append(len(idx))
    assert register(gpu, ptr, idx, rows), gpu.error()
    try:
        out = gpu.new_bf16(rows * heads * hd)
        scale = 1.0 / math.sqrt(hd)
        gpu.run("h3_gpu_sdpa_bf16", out, gpu.bf16(q), gpu.bf16(k),
                gpu.bf16(v), rows, heads, hd, C.c_float(scale))
        got = gpu.read_bf16(out)
        want = oracle.sdpa_sparse(q, k, v, rows, heads, hd, scale, ptr, idx)
        assert not got.reshape(rows, -1)[256:384].any()
        assert_close(got, want, what="sparse SDPA, split pieces",
                     extra_abs=2 * sdpa_p_rounding_bound(
                         q, k, v, rows, rows, heads, hd, scale))
    finally:
        clear(gpu)


def test_mask_only_applies_to_its_row_count(gpu):
    """Other sequence lengths and cross attention stay dense; clearing the
    mask restores dense attention."""
    rng = np.random.default_rng(8)
    hd, heads, rows = 128, 2, 300
    ptr, idx = random_mask(rng, 400, keep=0.3)
    assert register(gpu, ptr, idx, 400)
    try:
        q, k, v = (rand_bf16(rng, rows * heads * hd) for _ in range(3))
        scale = 1.0 / math.sqrt(hd)
        out = gpu.new_bf16(rows * heads * hd)
        gpu.run("h3_gpu_sdpa_bf16", out, gpu.bf16(q), gpu.bf16(k),
                gpu.bf16(v), rows, heads, hd, C.c_float(scale))
        want = oracle.sdpa(q, k, v, rows, rows, heads, hd, scale)
        bound = sdpa_p_rounding_bound(q, k, v, rows, rows, heads, hd, scale)
        assert_close(gpu.read_bf16(out), want, extra_abs=bound,
                     what="dense at another length")
        gpu.run("h3_gpu_sdpa_cross_bf16", out, gpu.bf16(q), gpu.bf16(k),
                gpu.bf16(v), rows, rows, heads, hd, C.c_float(scale))
        assert_close(gpu.read_bf16(out), want, extra_abs=bound,
                     what="cross attention stays dense")
    finally:
        clear(gpu)


def test_registration_validation(gpu):
    """The reference's CSR checks (h3_cuda_attention.cu:1826-1834)."""
    rows = 300                                 # 3 query blocks, 5 tiles
    assert not register(gpu, [1, 2, 3, 4], [0, 1, 2, 3], rows)   # ptr[0]
    assert not register(gpu, [0, 2, 1, 4], [0, 1, 2, 3], rows)   # decreasing
    assert not register(gpu, [0, 1, 2, 3], [0, 1, 2, 3], rows)   # end != n
    assert not register(gpu, [0, 1, 2, 3], [0, 1, 5], rows)      # tile 5
    assert not register(gpu, [0, 1, 2], [0, 1], rows)            # 2 blocks
    assert register(gpu, [0, 1, 2, 3], [0, 4, 2], rows)
    clear(gpu)


def test_h3_block_with_window_mask_matches_oracle(gpu):
    """One H3 block on the 256x256x22f t2va layout (256 text, 74 audio,
    448 video rows) with the 0:1:1 window: the joint attention of the
    video blocks is sparse, everything else global."""
    ok, lay, err = layout(256, 7, 16, 16, 37, 22)
    assert ok, err
    hidden, heads, ffn = 256, 2, 512
    n = lay.seq_len
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, hidden, heads, ffn, n, blocks=1,
                           time_rows=1)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=6, weight_std=0.05, mod_std=0.1)
        ptr, idx = mask(lay, 0, 1, 1, 0)
        kept = dit.gpu.L.h3hip_dit_set_sparse_window(dit.h, C.byref(lay), 0,
                                                     1, 1, 0, 0)
        assert kept == len(idx) and kept < ((n + 127) // 128) * \
            ((n + 63) // 64)
        names = ["norm1", "norm2", "qkv", "q_norm", "k_norm", "out", "fc1",
                 "fc2", "modulation"]
        w = [{k: dit.read(k, 0) for k in names}]
        x0 = dit.read("hidden")
        cos = dit.read("rope_cos")[:n * 48]
        sin = dit.read("rope_sin")[:n * 48]
        dit.run_blocks(0, 1)
        got = dit.read("hidden")
        row_map = np.zeros(n, np.uint32)
        want = oracle.h3_blocks(x0, w, row_map, cos, sin, n, hidden, heads,
                                ffn, sparse=(ptr, idx))
        c, r = cosine_rel_l2(got, want)
        assert c >= 0.999 and r <= 1e-2, (c, r)
        dense = oracle.h3_blocks(x0, w, row_map, cos, sin, n, hidden, heads,
                                 ffn)
        # the mask changes the result measurably (it is really applied)
        assert cosine_rel_l2(got, dense)[1] > 1e-3
    finally:
        assert dit.gpu.L.h3hip_dit_set_sparse_window(dit.h, None, 0, 0, 0, 0,
                                                     1) == 0
        dit.close()
        L.h3hip_layout_free(C.byref(lay))
