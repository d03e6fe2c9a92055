"""Modulation precompute on the GPU against the oracle (reference
h3_dit_schedule.c:78-337): timestep features -> F32 time MLP -> bf16 SiLU
-> per-block and final adaLN projections."""
import numpy as np
import pytest

import h3hip
import oracle
from conftest import assert_close
from test_sampler_gpu import make_model

pytestmark = pytest.mark.gpu

L = h3hip.lib()


def fill_bf16(gpu, count, seed, std):
    t = gpu.new_bf16(count)
    gpu.run("h3_gpu_fill_normal_bf16", t, 0, count, seed, 0.0, std)
    return gpu.read_bf16(t)


def test_schedule_precompute_matches_oracle(gpu):
    steps, hidden, blocks, seed = 4, 256, 2, 900
    dit, lay, m, (v_sig, a_sig, vr, ar) = make_model(gpu, steps=steps,
                                                     reuse=1, hidden=hidden,
                                                     blocks=blocks)
    try:
        dit.schedule_precompute(seed, weight_std=0.05)
        # host side: time rows (t = 1 - sigma) and sinusoid features, both
        # pinned against the reference in test_host_math
        n = dit.cfg.time_rows
        times = np.zeros(n, np.float32)
        a, b = np.zeros(steps, np.uint32), np.zeros(steps, np.uint32)
        assert L.h3hip_time_rows(steps, h3hip.ptr(v_sig), h3hip.ptr(a_sig), 0,
                                 0, h3hip.ptr(a), h3hip.ptr(b), None, None,
                                 h3hip.ptr(times)) == n
        feat = np.zeros(n * 256, np.float32)
        L.h3hip_timestep_features(h3hip.ptr(times), n, h3hip.ptr(feat))
        th, td = hidden, hidden // 2
        rd = lambda name: gpu.read_f32(dit.tensor(name))  # noqa: E731
        time = oracle.time_embedding(feat, rd("time_in_w"), rd("time_in_b"),
                                     rd("time_out_w"), rd("time_out_b"), n,
                                     256, th, td)
        block_out = 3 * 6 * hidden
        for blk in range(blocks):
            w = fill_bf16(gpu, block_out * td, seed + 16 + 2 * blk, 0.05)
            bias = fill_bf16(gpu, block_out, seed + 17 + 2 * blk, 0.02)
            want = oracle.linear(time, w, bias, n, td, block_out)
            assert_close(dit.read("modulation", blk), want,
                         what=f"block {blk} modulation", chained=1)
        w = fill_bf16(gpu, 2 * hidden * td, seed + 8, 0.05)
        bias = fill_bf16(gpu, 2 * hidden, seed + 9, 0.02)
        want = oracle.linear(time, w, bias, n, td, 2 * hidden)
        assert_close(dit.read("final_modulation"), want,
                     what="final modulation", chained=1)
    finally:
        dit.close()
        L.h3hip_layout_free(__import__("ctypes").byref(lay))
