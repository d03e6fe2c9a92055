"""Every BASELINE configuration at its own size on the GPU, against the CPU
oracle where the oracle finishes in seconds and through size-independent
properties where it cannot (the 50-block forwards, the full-size denoise).

  config 1  Wan block, 5120 hidden, 6x16x16 = 1536 video + 256 text rows
  config 2  Wan block at 512x512x22f: 6x32x32 = 6144 video + 512 text rows
  config 3  SDPA, 40 heads x 128: self 6144 / 9720 with the 3D RoPE applied
            in the kernel, cross 6144 / 9720 x 512
  config 4  Wan block at 864x480x22f: 6x30x54 = 9720 + 512 rows (one block
            against the oracle, the 50-block forward through properties)
  config 5  20-step Euler denoise, velocity reuse 2 (the small layout against
            the oracle forward; the H3 512x512x22f layout, 2378 rows and 50
            blocks, against the oracle's sampler loop driven by the device
            forward)

Block bar: cosine >= 0.999 and relative L2 <= 1e-2.
SDPA bar: the reference's |g - r| <= 1e-3 + 1e-2 |r|
(tests/test_cuda_attention.c:79-114) plus the bf16 P-rounding bound, on a
subset of heads (the device runs all 40, so the launch is the real one).
"""
import ctypes as C
import math

import numpy as np
import pytest

import h3hip
import oracle
from conftest import assert_close, cosine_rel_l2, rand_bf16, to_f32

pytestmark = pytest.mark.gpu

L = h3hip.lib()

WAN_NAMES = ["norm3", "norm3_bias", "qkv", "qkv_bias", "q_norm", "k_norm",
             "out", "out_bias", "fc1", "fc1_bias", "fc2", "fc2_bias", "cq",
             "cq_bias", "ck", "ck_bias", "cv", "cv_bias", "cq_norm",
             "ck_norm", "co", "co_bias", "modulation"]
H3_NAMES = ["norm1", "norm2", "qkv", "q_norm", "k_norm", "out", "fc1", "fc2",
            "modulation"]


def _bar(got, want, what):
    cos, rel = cosine_rel_l2(got, want)
    print(f"{what}: cosine {cos:.6f} rel-L2 {rel:.3e}", flush=True)
    assert cos >= 0.999 and rel <= 1e-2, f"{what}: cos {cos:.6f} rel {rel:.3g}"


def _wan_block_vs_oracle(gpu, t, h, w, text, seed):
    rows = t * h * w
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, 5120, 40, 13824, rows,
                           blocks=1, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=seed, weight_std=0.02, mod_std=0.1)
        cos, sin = h3hip.rope_tables(h3hip.wan_positions(t, h, w))
        dit.set_rope(cos, sin)
        wts = {n: dit.read(n, 0) for n in WAN_NAMES}
        x0, ctx = dit.read("hidden"), dit.read("context")
        dit.run_blocks(0, 1)
        got = dit.read("hidden")
    finally:
        dit.close()
    want = oracle.wan_block(x0, ctx, wts, np.zeros(rows, np.uint32),
                            oracle.bf16(cos), oracle.bf16(sin), rows, text,
                            5120, 40, 13824)
    _bar(got, want, f"Wan block {rows} + {text}")


def test_config1_wan_block_1536_plus_256(gpu):
    _wan_block_vs_oracle(gpu, 6, 16, 16, 256, seed=101)


def test_config2_wan_block_6144_plus_512(gpu):
    _wan_block_vs_oracle(gpu, 6, 32, 32, 512, seed=102)


def test_config4_wan_block_9720_plus_512(gpu):
    _wan_block_vs_oracle(gpu, 6, 30, 54, 512, seed=104)


def test_config4_wan_50_block_forward_properties(gpu):
    """The full config-4 forward (50 blocks, 9720 + 512 rows, ~35 GB of
    weights resident): finite, bit-identical on a re-run, and with every
    residual branch switched off (gate slots 2 and 5 zero; the ungated
    cross-attention branch off through a zero out-projection and bias) the
    50 blocks return their input bit for bit."""
    rows, text, blocks = 9720, 512, 50
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, 5120, 40, 13824, rows,
                           blocks=blocks, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=4, weight_std=0.02, mod_std=0.1)
        cos, sin = h3hip.rope_tables(h3hip.wan_positions(6, 30, 54))
        dit.set_rope(cos, sin)
        x0 = dit.read("hidden")
        dit.run_blocks(0, blocks)
        y1 = dit.read("hidden")
        f = to_f32(y1)
        assert np.isfinite(f).all()
        assert not np.array_equal(y1, x0)
        dit.write("hidden", x0)
        dit.run_blocks(0, blocks)
        assert np.array_equal(dit.read("hidden"), y1), "not deterministic"
        zero_co = np.zeros(5120 * 5120, np.uint16)
        zero_b = np.zeros(5120, np.uint16)
        for blk in range(blocks):
            mod = dit.read("modulation", blk).reshape(-1, 6, 5120).copy()
            mod[:, 2, :] = 0
            mod[:, 5, :] = 0
            dit.write("modulation", mod.ravel(), blk)
            dit.write("co", zero_co, blk)
            dit.write("co_bias", zero_b, blk)
        dit.write("hidden", x0)
        dit.run_blocks(0, blocks)
        assert np.array_equal(dit.read("hidden"), x0)
    finally:
        dit.close()


# ------------------------------------------------------------- config 3

def _sdpa_bound(q, k, v, q_rows, kv_rows, hd, scale):
    """sdpa_p_rounding_bound for one head, in query chunks (float64)."""
    Q = to_f32(q).astype(np.float64).reshape(q_rows, hd)
    K = to_f32(k).astype(np.float64).reshape(kv_rows, hd)
    V = np.abs(to_f32(v).astype(np.float64).reshape(kv_rows, hd))
    out = np.empty((q_rows, hd))
    for i in range(0, q_rows, 2048):
        s = Q[i:i + 2048] @ K.T * scale
        p = np.exp(s - s.max(-1, keepdims=True))
        out[i:i + 2048] = 2.0 ** -8 * (p @ V) / p.sum(-1, keepdims=True)
    return out


@pytest.mark.parametrize("q_rows,kv_rows,grid", [
    (6144, 6144, (6, 32, 32)), (9720, 9720, (6, 30, 54)), (6144, 512, None),
    (9720, 512, None)])
def test_config3_sdpa_full_size(gpu, q_rows, kv_rows, grid):
    """Self-attention with the grid's 3D RoPE applied in the kernel
    (h3_hip_sdpa_rope_bf16) against the oracle's rotation then attention;
    cross-attention (no RoPE) against the oracle's attention."""
    heads, hd = 40, 128
    scale = 1.0 / math.sqrt(hd)
    rng = np.random.default_rng(q_rows + kv_rows)
    q = rand_bf16(rng, q_rows * heads * hd)
    k = rand_bf16(rng, kv_rows * heads * hd)
    v = rand_bf16(rng, kv_rows * heads * hd)
    tq, tk, tv = gpu.bf16(q), gpu.bf16(k), gpu.bf16(v)
    to = gpu.new_bf16(q_rows * heads * hd)
    extra = []
    try:
        if grid:
            cos, sin = h3hip.rope_tables(h3hip.wan_positions(*grid))
            cos, sin = oracle.bf16(cos), oracle.bf16(sin)
            tc, ts = gpu.bf16(cos), gpu.bf16(sin)
            extra = [tc, ts]
            gpu.run("h3_hip_sdpa_rope_bf16", to, tq, tk, tv, tc, ts, q_rows,
                    heads, hd, 48, C.c_float(scale))
        else:
            gpu.run("h3_gpu_sdpa_cross_bf16", to, tq, tk, tv, q_rows, kv_rows,
                    heads, hd, C.c_float(scale))
        got = gpu.read_bf16(to).reshape(q_rows, heads, hd)
    finally:
        for t in [tq, tk, tv, to] + extra:
            gpu.free(t)
    q3 = q.reshape(q_rows, heads, hd)
    k3 = k.reshape(kv_rows, heads, hd)
    v3 = v.reshape(kv_rows, heads, hd)
    for h in (0, 23, 39):
        qh = np.ascontiguousarray(q3[:, h])
        kh = np.ascontiguousarray(k3[:, h])
        vh = np.ascontiguousarray(v3[:, h])
        if grid:
            qh = oracle.rope_rotate(qh, cos, sin, q_rows, 1)
            kh = oracle.rope_rotate(kh, cos, sin, kv_rows, 1)
        want = oracle.sdpa(qh, kh, vh, q_rows, kv_rows, 1, hd, scale)
        assert_close(np.ascontiguousarray(got[:, h]).ravel(), want,
                     what=f"SDPA {q_rows}x{kv_rows} head {h}",
                     extra_abs=_sdpa_bound(qh, kh, vh, q_rows, kv_rows, hd,
                                           scale).ravel())


# ------------------------------------------------------- H3 real shapes

def _h3_layout(latent_h=32, latent_w=32):
    lay = h3hip.Layout()
    err = C.create_string_buffer(256)
    assert L.h3hip_layout_build(512, 7, latent_h, latent_w, 37, 22, None, 0,
                                None, 0, C.byref(lay), err, 256), err.value
    return lay


def _h3_schedule(steps):
    v = np.zeros(steps + 1, np.float32)
    a = np.zeros(steps + 1, np.float32)
    assert L.h3hip_serving_schedule_build(steps, h3hip.ptr(v), h3hip.ptr(a))
    vr = np.zeros(steps, np.uint32)
    ar = np.zeros(steps, np.uint32)
    n = L.h3hip_time_rows(steps, h3hip.ptr(v), h3hip.ptr(a), 0, 0,
                          h3hip.ptr(vr), h3hip.ptr(ar), None, None, None)
    return v, a, n, vr, ar


def _layout_rope(lay):
    n = lay.seq_len
    pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                     lay.positions[i].w] for i in range(n)], np.float64)
    return h3hip.rope_tables(pos)


def test_h3_block_real_shape_2378_rows(gpu):
    """One H3 block at its 512x512x22f shape (5376 hidden, 56 heads, SwiGLU
    14336, 2378 packed rows) with the layout's own 3D RoPE tables and the
    step-0 row map, against the oracle."""
    lay = _h3_layout()
    try:
        rows = lay.seq_len
        assert rows == 2378
        _, _, n_time, vr, ar = _h3_schedule(20)
        row_map = np.zeros(rows, np.uint32)
        assert L.h3hip_row_map(C.byref(lay), int(vr[0]), int(ar[0]),
                               0xFFFFFFFF, 0xFFFFFFFF, None, 0,
                               h3hip.ptr(row_map), rows)
        cos, sin = _layout_rope(lay)
    finally:
        L.h3hip_layout_free(C.byref(lay))
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, 5376, 56, 14336, rows, blocks=1,
                           time_rows=n_time)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=23, weight_std=0.02, mod_std=0.1)
        dit.set_rope(cos, sin)
        dit.set_row_map(row_map)
        wts = [{n: dit.read(n, 0) for n in H3_NAMES}]
        x0 = dit.read("hidden")
        dit.run_blocks(0, 1)
        got = dit.read("hidden")
    finally:
        dit.close()
    want = oracle.h3_blocks(x0, wts, row_map, oracle.bf16(cos),
                            oracle.bf16(sin), rows, 5376, 56, 14336)
    _bar(got, want, "H3 block 2378 rows")


def test_h3_50_block_drift_against_oracle(gpu):
    """Drift through a full 50-block stack (hidden 512, 4 heads, 300 rows):
    the hidden state after blocks 9, 19, 29, 39 and 49 against the oracle
    run over the same blocks (the checkpoints of the reference's full-step
    test, tests/test_real_dit_block.c:539-552, 653-662).  The device runs the
    stack in five calls of ten blocks; each oracle segment starts from the
    oracle's own previous output, so errors accumulate on both sides
    independently."""
    rows, hidden, heads, ffn, blocks = 300, 512, 4, 1024, 50
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, hidden, heads, ffn, rows,
                           blocks=blocks, time_rows=2)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=50, weight_std=0.02, mod_std=0.1)
        rng = np.random.default_rng(50)
        ang = rng.uniform(-40, 40, rows * 48).astype(np.float32)
        cos, sin = np.cos(ang), np.sin(ang)
        dit.set_rope(cos, sin)
        row_map = rng.integers(0, 6, rows).astype(np.uint32)
        dit.set_row_map(row_map)
        wts = [{n: dit.read(n, b) for n in H3_NAMES} for b in range(blocks)]
        want = dit.read("hidden")
        for first in range(0, blocks, 10):
            dit.run_blocks(first, 10)
            got = dit.read("hidden")
            want = oracle.h3_blocks(want, wts[first:first + 10], row_map,
                                    oracle.bf16(cos), oracle.bf16(sin), rows,
                                    hidden, heads, ffn)
            _bar(got, want, f"after block {first + 9}")
    finally:
        dit.close()


def test_wan_50_block_drift_against_oracle(gpu):
    """The Wan stack's drift through 50 blocks (hidden 512, 4 heads, 300
    video + 77 text rows): the hidden state after blocks 9, 19, 29, 39 and
    49 against the oracle over the same blocks (the reference's full-step
    checkpoints, tests/test_real_dit_block.c:539-552, 653-662).  The device
    runs the stack in five calls of ten blocks, each fusing the FFN gate
    with the next block's adaLN across its blocks and starting with the
    grouped launch of its blocks' text K/V; each oracle segment starts from
    the oracle's own previous output."""
    rows, text, hidden, heads, ffn, blocks = 300, 77, 512, 4, 1024, 50
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, hidden, heads, ffn, rows,
                           blocks=blocks, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=51, weight_std=0.02, mod_std=0.1)
        rng = np.random.default_rng(51)
        ang = rng.uniform(-40, 40, rows * 48).astype(np.float32)
        cos, sin = np.cos(ang), np.sin(ang)
        dit.set_rope(cos, sin)
        wts = [{n: dit.read(n, b) for n in WAN_NAMES} for b in range(blocks)]
        want, ctx = dit.read("hidden"), dit.read("context")
        zero_map = np.zeros(rows, np.uint32)
        for first in range(0, blocks, 10):
            dit.run_blocks(first, 10)
            got = dit.read("hidden")
            for w in wts[first:first + 10]:
                want = oracle.wan_block(want, ctx, w, zero_map,
                                        oracle.bf16(cos), oracle.bf16(sin),
                                        rows, text, hidden, heads, ffn)
            _bar(got, want, f"Wan after block {first + 9}")
    finally:
        dit.close()


# -------------------------------------------------------------- config 5

def test_config5_denoise_20_steps_reuse_2_matches_oracle(gpu):
    """The 20-step serving schedule with velocity reuse 2 (11 fresh
    forwards, extrapolated transitions, terminal sigma 0) on the small
    layout, the whole loop against the oracle's."""
    from test_sampler_gpu import make_model
    steps, reuse = 20, 2
    dit, lay, m, (v_sig, a_sig, _, _) = make_model(gpu, steps=steps,
                                                   reuse=reuse)
    try:
        assert v_sig[-1] == 0.0 and a_sig[-1] == 0.0
        v0, a0 = m["video_input"].copy(), m["audio_input"].copy()
        n = dit.denoise()
        assert n == 11 == sum(oracle.reuse_schedule(steps, reuse))
        gv, ga = dit.read_latents()
        wv, wa, n_ref = oracle.h3_denoise(m, v_sig, a_sig, reuse)
        assert n_ref == n
        for got, want, start, what in ((gv, wv, v0, "video"),
                                       (ga, wa, a0, "audio")):
            _bar(h3hip.f32_to_bf16(got - start),
                 h3hip.f32_to_bf16(want - start), f"denoise {what}")
    finally:
        dit.close()
        L.h3hip_layout_free(C.byref(lay))


def test_config5_denoise_full_size_loop(gpu):
    """BASELINE config 5 at its own size: the H3 layout of a 512x512x22f
    clip (2378 rows), 50 blocks, the 20-step serving schedule with reuse 2
    and an N(0,1) start.  The device's denoise must equal, bit for bit, the
    oracle's sampler loop (reuse schedule, extrapolation ratios, Euler
    updates in F32) driven by the device's own forward for each fresh step;
    the result is finite and changes the target rows."""
    steps, reuse, blocks = 20, 2, 50
    lay = _h3_layout()
    try:
        rows = lay.seq_len
        v_sig, a_sig, n_time, _, _ = _h3_schedule(steps)
        cfg = h3hip.dit_config(h3hip.FAMILY_H3, 5376, 56, 14336, rows,
                               blocks=blocks, time_rows=n_time)
        dit = h3hip.Dit(gpu, cfg)
        try:
            dit.init_random(seed=1, weight_std=0.02, mod_std=0.1)
            cos, sin = _layout_rope(lay)
            dit.set_rope(cos, sin)
            dit.sampler_create(lay, v_sig, a_sig, reuse_interval=reuse)
            dit.sampler_init_random(seed=2, weight_std=0.02, mod_std=0.1)
            dit.schedule_precompute(seed=3, weight_std=0.02)
            vrows, arows, vt, at = dit.sampler_rows()
            rng = np.random.default_rng(0)
            v0 = rng.standard_normal(vrows * 96).astype(np.float32)
            a0 = rng.standard_normal(arows * 32).astype(np.float32)
            dit.write_latents(v0, a0)
            assert dit.denoise() == 11
            gv, ga = dit.read_latents()
            assert np.isfinite(gv).all() and np.isfinite(ga).all()

            def device_forward(mm, step):
                dit.write_latents(mm["video_input"], mm["audio_input"])
                dit.forward_step(step)
                return (dit.read("video_velocity")[:vt * 96],
                        dit.read("audio_velocity")[:at * 32])

            m = {"video_input": v0, "audio_input": a0, "video_patch": 96,
                 "audio_channels": 32, "video_conditions": vrows - vt,
                 "audio_conditions": arows - at}
            wv, wa, n = oracle.h3_denoise(m, v_sig, a_sig, reuse,
                                          forward=device_forward)
            assert n == 11
            np.testing.assert_array_equal(gv, wv)
            np.testing.assert_array_equal(ga, wa)
            assert not np.array_equal(gv[-vt * 96:], v0[-vt * 96:])
        finally:
            dit.close()
    finally:
        L.h3hip_layout_free(C.byref(lay))
