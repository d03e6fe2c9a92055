"""The H3 sampler on the GPU against the oracle: patch projection, packing,
blocks, final adaLN heads and the Euler loop with velocity reuse
(reference h3_dit.c encode_forward :2182-2528, denoise_euler_gpu
:2745-2917), on a small layout so the CPU oracle finishes in seconds."""
import ctypes as C

import numpy as np
import pytest

import h3hip
import oracle
from conftest import cosine_rel_l2

pytestmark = pytest.mark.gpu

L = h3hip.lib()


def build_layout(text, lt, lh, lw, at, frames):
    lay = h3hip.Layout()
    err = C.create_string_buffer(256)
    assert L.h3hip_layout_build(text, lt, lh, lw, at, frames, None, 0, None, 0,
                                C.byref(lay), err, 256), err.value
    return lay


def serving_sigmas(steps):
    v = np.zeros(steps + 1, np.float32)
    a = np.zeros(steps + 1, np.float32)
    assert L.h3hip_serving_schedule_build(steps, h3hip.ptr(v), h3hip.ptr(a))
    return v, a


def time_rows(v, a):
    steps = len(v) - 1
    vr = np.zeros(steps, np.uint32)
    ar = np.zeros(steps, np.uint32)
    n = L.h3hip_time_rows(steps, h3hip.ptr(v), h3hip.ptr(a), 0, 0,
                          h3hip.ptr(vr), h3hip.ptr(ar), None, None, None)
    return n, vr, ar


def rope(lay):
    n = lay.seq_len
    pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                     lay.positions[i].w] for i in range(n)], np.float64)
    inv = np.empty(16, np.float32)
    L.h3hip_default_inv_freq(h3hip.ptr(inv))
    cos = np.empty(n * 48, np.float32)
    sin = np.empty(n * 48, np.float32)
    L.h3hip_rope_tables(h3hip.ptr(pos), n, h3hip.ptr(inv), C.c_float(1.0),
                        h3hip.ptr(cos), h3hip.ptr(sin))
    return cos, sin


def host_row_map(lay, video_row, audio_row):
    rows = np.zeros(lay.seq_len, np.uint32)
    assert L.h3hip_row_map(C.byref(lay), video_row, audio_row, 0xFFFFFFFF,
                           0xFFFFFFFF, None, 0, h3hip.ptr(rows), lay.seq_len)
    return rows


def make_model(gpu, steps, reuse, hidden=256, heads=2, ffn=512, blocks=2,
               seed=5):
    """Small H3 DiT + sampler on the 'tiny' layout (12 text, 16 audio,
    2 video rows; reference tests/test_h3.c:176)."""
    lay = build_layout(12, 2, 2, 2, 8, 5)
    v_sig, a_sig = serving_sigmas(steps)
    n_time, vr, ar = time_rows(v_sig, a_sig)
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, hidden, heads, ffn, lay.seq_len,
                           blocks=blocks, time_rows=n_time)
    dit = h3hip.Dit(gpu, cfg)
    dit.init_random(seed, weight_std=0.05, mod_std=0.05)
    cos, sin = rope(lay)
    dit.set_rope(cos, sin)
    dit.sampler_create(lay, v_sig, a_sig, reuse_interval=reuse)
    dit.sampler_init_random(seed + 1, weight_std=0.05, mod_std=0.05)
    vrows, arows, vt, at = dit.sampler_rows()
    rng = np.random.default_rng(seed)
    dit.write_latents(rng.standard_normal(vrows * 96).astype(np.float32),
                      rng.standard_normal(arows * 32).astype(np.float32))
    segs = [(lay.segments[i].start, lay.segments[i].stop,
             lay.segments[i].kind) for i in range(lay.segment_count)]
    names = ["norm1", "norm2", "qkv", "q_norm", "k_norm", "out", "fc1", "fc2",
             "modulation"]
    m = dict(
        hidden=hidden, heads=heads, ffn=ffn, rows=lay.seq_len, eps=1e-5,
        video_patch=96, audio_channels=32, segments=segs,
        blocks=[{k: dit.read(k, b) for k in names} for b in range(blocks)],
        cos=h3hip.f32_to_bf16(cos), sin=h3hip.f32_to_bf16(sin),
        refined_text=dit.read("refined_text"),
        final_norm=dit.read("final_norm"),
        final_modulation=dit.read("final_modulation"),
        final_video_w=dit.read("final_video_w"),
        final_video_b=dit.read("final_video_b"),
        final_audio_w=dit.read("final_audio_w"),
        final_audio_b=dit.read("final_audio_b"),
        video_patch_w=gpu.read_f32(dit.tensor("video_patch_w")),
        video_patch_b=gpu.read_f32(dit.tensor("video_patch_b")),
        audio_patch_w=gpu.read_f32(dit.tensor("audio_patch_w")),
        audio_patch_b=gpu.read_f32(dit.tensor("audio_patch_b")),
        step_maps=[host_row_map(lay, int(vr[s]), int(ar[s]))
                   for s in range(steps)],
        final_video_maps=[np.full(vt, vr[s], np.uint32)
                          for s in range(steps)],
        final_audio_maps=[np.full(at, ar[s], np.uint32)
                          for s in range(steps)],
        video_conditions=0, audio_conditions=0,
        video_targets=vt, audio_targets=at,
        video_target_start=[s for s, e, k in segs if k == 5][0],
        audio_target_start=[s for s, e, k in segs if k == 4][0])
    vin, ain = dit.read_latents()
    m["video_input"], m["audio_input"] = vin, ain
    return dit, lay, m, (v_sig, a_sig, vr, ar)


def test_row_maps_follow_the_schedule(gpu):
    """Per-step maps (reference prepare_maps h3_dit.c:1134-1200) as the
    oracle model uses them: text rows at video_row*3+1, audio at
    audio_row*3+2, video at video_row*3; final maps hold the bare time row.
    The device copies are checked through the forward parity below."""
    dit, lay, m, (v, a, vr, ar) = make_model(gpu, steps=4, reuse=1)
    try:
        for s in range(4):
            rows = m["step_maps"][s]
            assert rows[:12].tolist() == [int(vr[s]) * 3 + 1] * 12
            assert rows[12:28].tolist() == [int(ar[s]) * 3 + 2] * 16
            assert rows[28:30].tolist() == [int(vr[s]) * 3] * 2
            assert m["final_video_maps"][s].tolist() == [int(vr[s])] * 2
            assert m["final_audio_maps"][s].tolist() == [int(ar[s])] * 16
    finally:
        dit.close()
        L.h3hip_layout_free(C.byref(lay))


def test_forward_step_matches_oracle(gpu):
    dit, lay, m, _ = make_model(gpu, steps=3, reuse=1)
    try:
        for step in (0, 2):
            dit.forward_step(step)
            gv = dit.read("video_velocity")[:2 * 96]
            ga = dit.read("audio_velocity")[:16 * 32]
            wv, wa = oracle.h3_forward_step(m, step)
            for got, want, what in ((gv, wv, "video"), (ga, wa, "audio")):
                cos, rel = cosine_rel_l2(got, want)
                assert cos >= 0.999 and rel <= 1e-2, (step, what, cos, rel)
    finally:
        dit.close()
        L.h3hip_layout_free(C.byref(lay))


@pytest.mark.parametrize("steps,reuse", [(5, 2), (4, 1)])
def test_denoise_matches_oracle(gpu, steps, reuse):
    dit, lay, m, (v_sig, a_sig, _, _) = make_model(gpu, steps=steps,
                                                   reuse=reuse)
    try:
        v0, a0 = m["video_input"].copy(), m["audio_input"].copy()
        n = dit.denoise()
        assert n == sum(oracle.reuse_schedule(steps, reuse))
        gv, ga = dit.read_latents()
        wv, wa, n_ref = oracle.h3_denoise(m, v_sig, a_sig, reuse)
        assert n_ref == n
        for got, want, start, what in ((gv, wv, v0, "video"),
                                       (ga, wa, a0, "audio")):
            # compare the change the sampler made; the start is shared
            d_got = h3hip.f32_to_bf16(got - start)
            d_want = h3hip.f32_to_bf16(want - start)
            cos, rel = cosine_rel_l2(d_got, d_want)
            assert cos >= 0.999 and rel <= 1e-2, (what, cos, rel)
    finally:
        dit.close()
        L.h3hip_layout_free(C.byref(lay))


def test_denoise_with_zero_velocity_head_keeps_latents(gpu):
    """Invariant: zero final-head weights and biases give v = 0, so every
    Euler step (fresh or extrapolated) leaves the latents unchanged, bit for
    bit."""
    dit, lay, m, _ = make_model(gpu, steps=5, reuse=2)
    try:
        for name, count in (("final_video_w", 96 * 256), ("final_video_b", 96),
                            ("final_audio_w", 32 * 256),
                            ("final_audio_b", 32)):
            dit.write(name, np.zeros(count, np.uint16))
        v0, a0 = dit.read_latents()
        assert dit.denoise() == 3
        v1, a1 = dit.read_latents()
        assert np.array_equal(v0, v1) and np.array_equal(a0, a1)
    finally:
        dit.close()
        L.h3hip_layout_free(C.byref(lay))
