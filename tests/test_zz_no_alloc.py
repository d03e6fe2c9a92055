"""h3_hip_linear_bf16_noalloc (static split-K scratch, no allocation)
against h3_gpu_linear_bf16 through the C ABI: bit-identical outputs on
consecutive calls whose second and third inputs are smaller than the first,
so each call reuses the static scratch the previous one left filled."""
import ctypes as C

import numpy as np
import pytest

import h3hip
import oracle
from conftest import assert_close, rand_bf16

pytestmark = pytest.mark.gpu


def _pair(gpu, rng, rows, k, n, bias):
    x = rand_bf16(rng, rows * k)
    w = rand_bf16(rng, n * k, 0.02)
    b = rand_bf16(rng, n, 0.1) if bias else None
    tx, tw = gpu.bf16(x), gpu.bf16(w)
    tb = gpu.bf16(b) if bias else None
    ref, got = gpu.new_bf16(rows * n), gpu.new_bf16(rows * n)
    gpu.run("h3_gpu_linear_bf16", ref, tx, tw, tb, rows, k, n)
    gpu.run("h3_hip_linear_bf16_noalloc", got, tx, tw, tb, rows, k, n)
    out = gpu.read_bf16(got), gpu.read_bf16(ref)
    for t in (tx, tw, ref, got) + ((tb,) if bias else ()):
        gpu.free(t)
    return out, (x, w, b)


def test_noalloc_linear_matches_linear_on_consecutive_calls(gpu):
    rng = np.random.default_rng(71)
    # 1: the 512-row text K/V projection shape (40 tiles, every tile split
    #    along K); 2: a smaller split launch (6 tiles x 4 pieces);
    # 3: a launch with full rounds and no split (skinny rows)
    for rows, k, n, bias in ((512, 5120, 5120, True), (300, 1024, 768, False),
                             (40, 512, 1024, True)):
        print(f"noalloc linear {rows}x{k}x{n}", flush=True)
        (got, ref), (x, w, b) = _pair(gpu, rng, rows, k, n, bias)
        np.testing.assert_array_equal(got, ref)
        if rows * k * n <= 300 * 1024 * 768:
            assert_close(got, oracle.linear(x, w, b, rows, k, n),
                         what=f"noalloc {rows}x{k}x{n}")


def test_noalloc_linear_leaves_no_allocation():
    """In a fresh context (no split-K scratch yet) a split-K call of the
    allocation-free entry point makes no device allocation, while the
    ordinary entry point's first split-K call grows its scratch."""
    rng = np.random.default_rng(72)
    rows, k, n = 512, 2048, 1536
    x, w = rand_bf16(rng, rows * k), rand_bf16(rng, n * k, 0.02)
    with h3hip.Gpu() as g:
        tx, tw = g.bf16(x), g.bf16(w)
        out, ref = g.new_bf16(rows * n), g.new_bf16(rows * n)
        before = g.L.h3_hip_device_allocations(g.h)
        g.run("h3_hip_linear_bf16_noalloc", out, tx, tw, None, rows, k, n)
        assert g.L.h3_hip_device_allocations(g.h) == before
        g.run("h3_gpu_linear_bf16", ref, tx, tw, None, rows, k, n)
        assert g.L.h3_hip_device_allocations(g.h) == before + 1
        got = g.read_bf16(out)
        np.testing.assert_array_equal(got, g.read_bf16(ref))
    assert_close(got, oracle.linear(x, w, None, rows, k, n),
                 what="noalloc 512x2048x1536")
