"""Host restatement of the reference's block-sparse attention mask
(h3_dit.c:1006-1132) and the oracle's sparse SDPA: properties that pin
them without a GPU."""
import ctypes as C

import numpy as np

import h3hip
import oracle
from test_host_math import layout

L = h3hip.lib()


def mask(lay, rt, rh, rw, g):
    qblocks = (lay.seq_len + 127) // 128
    ptr = np.zeros(qblocks + 1, np.uint32)
    total = L.h3hip_sparse_mask(C.byref(lay), rt, rh, rw, g, h3hip.ptr(ptr),
                                None, 0)
    assert total >= 0
    idx = np.zeros(max(total, 1), np.uint32)
    assert L.h3hip_sparse_mask(C.byref(lay), rt, rh, rw, g, h3hip.ptr(ptr),
                               h3hip.ptr(idx), total) == total
    return ptr, idx[:total]


def lists(ptr, idx):
    return [set(idx[ptr[q]:ptr[q + 1]].tolist()) for q in range(len(ptr) - 1)]


def test_sparse_mask_structure_on_the_real_layout():
    """512x512x22f t2va layout: text 0..511, audio 512..585, video
    586..2377.  Tiles/blocks holding any non-video row are global both ways;
    huge radii keep everything; the mask grows with the radii; every video
    tile overlapping a query block's rows is kept (gap 0); a global stride
    G adds exactly the tiles k % G == 0."""
    ok, lay, err = layout(512, 7, 32, 32, 37, 22)
    assert ok, err
    try:
        n = lay.seq_len
        qb, kt = (n + 127) // 128, (n + 63) // 64
        ptr, idx = mask(lay, 100, 100, 100, 0)
        assert all(s == set(range(kt)) for s in lists(ptr, idx))
        small = lists(*mask(lay, 0, 1, 1, 0))
        mid = lists(*mask(lay, 1, 4, 4, 0))
        assert all(a <= b for a, b in zip(small, mid))
        assert sum(map(len, small)) < qb * kt
        global_tiles = set(range((586 + 63) // 64))      # tiles 0..9
        for q, s in enumerate(small):
            if q * 128 < 586:                            # blocks 0..4
                assert s == set(range(kt))
            else:
                assert global_tiles <= s
                lo, hi = q * 128, min(n, q * 128 + 128)
                own = {t for t in range(kt) if t * 64 < hi and t * 64 + 64 > lo}
                assert own <= s
        strided = lists(*mask(lay, 0, 1, 1, 4))
        for a, b in zip(small, strided):
            assert b == a | {t for t in range(kt) if t % 4 == 0}
        # the offsets are consistent
        ptr, idx = mask(lay, 0, 1, 1, 0)
        assert ptr[0] == 0 and ptr[-1] == len(idx)
        assert np.all(np.diff(ptr.astype(np.int64)) >= 0)
        assert np.all(idx < kt)
    finally:
        L.h3hip_layout_free(C.byref(lay))


def test_oracle_sparse_sdpa_pins():
    """Full lists reproduce the dense oracle bit for bit; a block with one
    listed tile equals dense attention over that tile's keys alone; an
    empty list gives zeros."""
    rng = np.random.default_rng(4)
    n, h, hd = 200, 2, 128
    q, k, v = (oracle.bf16(rng.standard_normal(n * h * hd).astype(np.float32))
               for _ in range(3))
    scale = hd ** -0.5
    full = oracle.sdpa_sparse(q, k, v, n, h, hd, scale, [0, 4, 8],
                              [0, 1, 2, 3] * 2)
    assert np.array_equal(full, oracle.sdpa(q, k, v, n, n, h, hd, scale))
    one = oracle.sdpa_sparse(q, k, v, n, h, hd, scale, [0, 1, 2], [2, 0])
    # block 0 (rows 0..127) sees keys 128..191 only
    ks = k.reshape(n, h, hd)[128:192].ravel()
    vs = v.reshape(n, h, hd)[128:192].ravel()
    want = oracle.sdpa(q.reshape(n, h, hd)[:128].ravel(), ks, vs, 128, 64, h,
                       hd, scale)
    got = one.reshape(n, h, hd)[:128].ravel()
    assert np.array_equal(got, want)
    # a block whose list is empty outputs zeros (the reference's l = 0
    # guard, h3_cuda_attention.cu:1789)
    empty = oracle.sdpa_sparse(q, k, v, n, h, hd, scale, [0, 0, 1], [3])
    assert not empty.reshape(n, h, hd)[:128].any()
    assert empty.reshape(n, h, hd)[128:].any()
