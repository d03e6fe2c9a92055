"""Token reduction on the GPU (reference h3_cuda_dit.cu:336-535 and the
h3_gpu.h:557-612 entry points) against the oracle: pooling and expansion
bit for bit, the fused adaLN variants within the adaLN row tolerance."""
import numpy as np
import pytest

import oracle
from conftest import adaln_terms, assert_row_close, rand_bf16

pytestmark = pytest.mark.gpu


def plan(rng, input_rows, rows, baseline_rows):
    """pairs covering input rows (some singletons), baseline indices for the
    first baseline_rows reduced rows, parents mapping every full row back."""
    order = rng.permutation(input_rows)
    pairs, parents = [], np.zeros(input_rows, np.uint32)
    i = 0
    for r in range(rows):
        left = input_rows - i
        need = rows - r
        take = 2 if left > need else 1
        x = order[i]
        y = order[i + 1] if take == 2 else x
        pairs += [x, y]
        parents[x] = parents[y] = r
        i += take
    assert i == input_rows
    bidx = np.full(rows, 0xFFFFFFFF, np.uint32)
    sel = rng.choice(rows, baseline_rows, replace=False)
    bidx[sel] = np.arange(baseline_rows, dtype=np.uint32)
    return np.array(pairs, np.uint32), parents, bidx


@pytest.mark.parametrize("width", [512, 5376])
def test_token_pool_and_expand(gpu, width):
    rng = np.random.default_rng(width)
    input_rows, rows, baseline_rows = 300, 180, 150
    pairs, parents, bidx = plan(rng, input_rows, rows, baseline_rows)
    x = rand_bf16(rng, input_rows * width)
    off = 3 * width                      # nonzero input / original offsets
    tin = gpu.bf16(np.concatenate([np.zeros(off, np.uint16), x]))
    out = gpu.new_bf16(rows * width)
    orig = gpu.bf16(np.zeros(off + input_rows * width, np.uint16))
    base = gpu.bf16(np.zeros(width + baseline_rows * width, np.uint16))
    tb, tp = gpu.u32(bidx), gpu.u32(pairs)
    gpu.run("h3_gpu_token_pool_bf16", out, tin, off, orig, off, base, width,
            tb, tp, input_rows, rows, baseline_rows, width)
    w_out, w_orig, w_base = oracle.token_pool(x, pairs, bidx, input_rows,
                                              rows, baseline_rows, width)
    assert np.array_equal(gpu.read_bf16(out), w_out)
    assert np.array_equal(gpu.read_bf16(orig)[off:], w_orig)
    assert np.array_equal(gpu.read_bf16(base)[width:], w_base)

    # the reduced stack moves on; expand with the delta rule
    reduced = oracle.bf16(oracle.f32(w_out) +
                          0.1 * rng.standard_normal(rows * width)
                          .astype(np.float32))
    tred = gpu.bf16(reduced)
    full = gpu.new_bf16(input_rows * width)
    prefix, scale = 7, 0.75
    gpu.run("h3_gpu_token_expand_delta_bf16", full, orig, off, tred, base,
            width, tb, gpu.u32(parents), input_rows, rows, baseline_rows,
            width, prefix, np.float32(scale))
    want = oracle.token_expand(w_orig, reduced, w_base, bidx, parents,
                               input_rows, width, prefix, scale)
    assert np.array_equal(gpu.read_bf16(full), want)


def test_token_fused_adaln(gpu):
    rng = np.random.default_rng(11)
    width, input_rows, rows, baseline_rows = 5376, 200, 120, 100
    slots, mod_rows, eps = 6, 4, 1e-5
    pairs, parents, bidx = plan(rng, input_rows, rows, baseline_rows)
    x = rand_bf16(rng, input_rows * width)
    norm = rand_bf16(rng, width, 0.02, 1.0)
    mod = rand_bf16(rng, mod_rows * slots * width, 0.3)
    rmap_r = rng.integers(0, mod_rows, rows).astype(np.uint32)
    rmap_f = rng.integers(0, mod_rows, input_rows).astype(np.uint32)
    tin, tnorm, tmod = gpu.bf16(x), gpu.bf16(norm), gpu.bf16(mod)
    orig = gpu.new_bf16(input_rows * width)
    base = gpu.new_bf16(baseline_rows * width)
    res = gpu.new_bf16(rows * width)
    out = gpu.new_bf16(rows * width)
    tb = gpu.u32(bidx)
    gpu.run("h3_gpu_token_pool_adaln_bf16", res, out, tin, 0, orig, 0, base,
            0, tb, gpu.u32(pairs), tnorm, tmod, gpu.u32(rmap_r), input_rows,
            rows, baseline_rows, width, slots, 0, 1, np.float32(eps))
    w_res, w_orig, w_base = oracle.token_pool(x, pairs, bidx, input_rows,
                                              rows, baseline_rows, width)
    assert np.array_equal(gpu.read_bf16(res), w_res)
    want = oracle.adaln(w_res, norm, mod, rmap_r, rows, width, slots, 0, 1,
                        eps)
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(w_res, norm, mod, rmap_r, rows, width,
                                 slots, 0, 1, eps), what="pool adaLN")

    reduced = rand_bf16(rng, rows * width)
    full = gpu.new_bf16(input_rows * width)
    fout = gpu.new_bf16(input_rows * width)
    gpu.run("h3_gpu_token_expand_adaln_bf16", full, fout, orig, 0,
            gpu.bf16(reduced), base, 0, tb, gpu.u32(parents), tnorm, tmod,
            gpu.u32(rmap_f), input_rows, rows, baseline_rows, width, 5,
            np.float32(0.5), slots, 3, 4, np.float32(eps))
    w_full = oracle.token_expand(w_orig, reduced, w_base, bidx, parents,
                                 input_rows, width, 5, 0.5)
    assert np.array_equal(gpu.read_bf16(full), w_full)
    want = oracle.adaln(w_full, norm, mod, rmap_f, input_rows, width, slots,
                        3, 4, eps)
    assert_row_close(gpu.read_bf16(fout), want,
                     adaln_terms(w_full, norm, mod, rmap_f, input_rows, width,
                                 slots, 3, 4, eps), what="expand adaLN")


def test_token_validation(gpu):
    """Shape rules of the reference (h3_cuda_dit.cu:797-1074) plus this
    backend's 16-byte row chunks (width % 8 == 0)."""
    t = gpu.new_bf16(64 * 16)
    u = gpu.u32(np.zeros(64, np.uint32))
    L = gpu.L
    gpu.begin()
    try:
        assert not L.h3_gpu_token_pool_bf16(gpu.h, t, t, 0, t, 0, t, 0, u, u,
                                            8, 9, 0, 16)    # rows > input
        assert not L.h3_gpu_token_pool_bf16(gpu.h, t, t, 0, t, 0, t, 0, u, u,
                                            8, 4, 0, 12)    # width % 8
        assert not L.h3_gpu_token_expand_delta_bf16(
            gpu.h, t, t, 0, t, t, 0, u, u, 8, 4, 2, 16, 5,
            np.float32(1))                                  # prefix > reduced
        assert not L.h3_gpu_token_expand_adaln_bf16(
            gpu.h, t, t, t, 0, t, t, 0, u, u, t, t, u, 8, 4, 2, 16, 0,
            np.float32(1), 6, 6, 1, np.float32(1e-5))      # slot 6 of 6
    finally:
        gpu.submit()
