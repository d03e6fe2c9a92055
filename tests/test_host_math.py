"""Host math of the DiT path (h3.c_amd/host/h3hip_host.c) pinned bit for bit:

  * against tests/golden/host_golden.json, written from the reference's own
    h3_host.c (tests/golden/make_golden.py): temporal shapes, both sigma
    grids, packed layouts with positions, PCG32 / Box-Muller streams;
  * against the literal constants of the reference's tests/test_h3.c;
  * RoPE tables, timestep rows and row maps against restatements of
    h3_dit.c:907-922 and h3_dit_schedule.c:78-161, 434-485 built from libm's
    cosf/sinf and hand-derived row assignments.
These run on the CPU; they load the product library but call no device code.
"""
import ctypes as C
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

import h3hip

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "host_golden.json")))
L = h3hip.lib()


def fbits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32).tolist()


def layout(text, lt, lh, lw, at, frames, keys=(), refs=()):
    karr = (C.c_int * max(1, len(keys)))(*keys)
    rarr = (h3hip.LayoutRef * max(1, len(refs)))(
        *[h3hip.LayoutRef(*r) for r in refs])
    lay = h3hip.Layout()
    err = C.create_string_buffer(256)
    ok = L.h3hip_layout_build(text, lt, lh, lw, at, frames,
                              C.cast(karr, C.c_void_p), len(keys),
                              C.cast(rarr, C.c_void_p), len(refs),
                              C.byref(lay), err, 256)
    return ok, lay, err.value.decode()


# ------------------------------------------------------------- temporal

def test_temporal_matches_reference():
    for req, frames, vt, at in GOLDEN["temporal"]:
        f, v, a = C.c_int(), C.c_int(), C.c_int()
        L.h3hip_temporal(req, C.byref(f), C.byref(v), C.byref(a))
        assert (f.value, v.value, a.value) == (frames, vt, at), req


def test_temporal_literals():
    """reference tests/test_h3.c:34-48"""
    cases = [(5, 5, 2, 8), (6, 22, 7, 37), (22, 22, 7, 37), (23, 39, 12, 65),
             (56, 56, 17, 93), (124, 124, 37, 207), (361, 362, 107, 603)]
    for req, frames, vt, at in cases:
        f, v, a = C.c_int(), C.c_int(), C.c_int()
        L.h3hip_temporal(req, C.byref(f), C.byref(v), C.byref(a))
        assert (f.value, v.value, a.value) == (frames, vt, at)


# ------------------------------------------------------------- schedules

def _grid(fn, n):
    v = np.zeros(n + 1, np.float32)
    a = np.zeros(n + 1, np.float32)
    ok = fn(n, h3hip.ptr(v), h3hip.ptr(a))
    return ok, v, a


@pytest.mark.parametrize("kind", ["schedule", "serving_schedule"])
def test_sigma_grids_bit_exact(kind):
    fn = (L.h3hip_schedule_build if kind == "schedule"
          else L.h3hip_serving_schedule_build)
    for n, want in GOLDEN[kind].items():
        ok, v, a = _grid(fn, int(n))
        if want is None:
            assert not ok
            continue
        assert ok
        assert fbits(v) == want["video"], (kind, n)
        assert fbits(a) == want["audio"], (kind, n)


def test_sigma_literals():
    """reference tests/test_h3.c:77-126"""
    ok, v, a = _grid(L.h3hip_schedule_build, 20)
    assert ok and v[0] == 1.0 and a[0] == 1.0 and v[20] == 0 and a[20] == 0
    assert abs(v[1] - 0.995633185) <= 1e-7 and abs(a[1] - 0.982758582) <= 1e-7
    assert abs(v[19] - 0.387096792) <= 1e-7
    assert abs(a[19] - 0.136363640) <= 1e-7
    ok, v, a = _grid(L.h3hip_serving_schedule_build, 50)
    base = np.float32(0.5)
    assert abs(v[25] - 12 * base / (1 + 11 * base)) <= 1e-7
    assert abs(a[25] - 3 * base / (1 + 2 * base)) <= 1e-7
    ok, v, a = _grid(L.h3hip_serving_schedule_build, 4)
    assert abs(v[1] - 36.0 / 37.0) <= 1e-7 and abs(a[1] - 0.9) <= 1e-7
    assert np.all(np.diff(v) < 0) and np.all(np.diff(a) < 0)
    assert not _grid(L.h3hip_serving_schedule_build, 1)[0]
    assert not _grid(L.h3hip_serving_schedule_build, 1001)[0]


def test_reuse_schedule_literals():
    """reference tests/test_h3.c:128-147"""
    sel = np.zeros(50, np.uint8)
    assert L.h3hip_reuse_schedule(20, 3, h3hip.ptr(sel), 50) == 8
    assert np.flatnonzero(sel[:20]).tolist() == [0, 3, 6, 9, 12, 15, 18, 19]
    assert L.h3hip_reuse_schedule(20, 2, h3hip.ptr(sel), 50) == 11
    assert all(sel[s] == (s % 2 == 0 or s == 19) for s in range(20))
    assert L.h3hip_reuse_schedule(50, 3, h3hip.ptr(sel), 50) == 18
    assert L.h3hip_reuse_schedule(20, 1, h3hip.ptr(sel), 50) == 20
    assert L.h3hip_reuse_schedule(20, 3, h3hip.ptr(sel), 19) == -1


def test_extrapolation_ratio_clamped():
    """h3_dit.c:2644-2655: (s - s_last) / (s_last - s_prev), clamped to
    [-2, 2], 0 without a previous evaluation or a zero denominator."""
    r = L.h3hip_extrapolation_ratio
    assert r(0.5, 0.6, 0.7, 1) == pytest.approx(1.0)
    assert r(0.5, 0.6, 0.7, 0) == 0.0
    assert r(0.5, 0.6, 0.6, 1) == 0.0
    assert r(0.0, 0.6, 0.65, 1) == 2.0
    assert r(1.0, 0.6, 0.65, 1) == -2.0


# --------------------------------------------------------------- layouts

@pytest.mark.parametrize("name", sorted(GOLDEN["layouts"]))
def test_layout_matches_reference(name):
    g = GOLDEN["layouts"][name]
    text, lt, lh, lw, at, frames, keys, refs = g["spec"]
    ok, lay, err = layout(text, lt, lh, lw, at, frames, keys,
                          [tuple(r) for r in refs])
    assert ok, err
    try:
        assert lay.seq_len == g["seq_len"]
        segs = [[lay.segments[i].start, lay.segments[i].stop,
                 lay.segments[i].kind] for i in range(lay.segment_count)]
        assert segs == g["segments"]
        assert [lay.img_cond_rows, lay.img_target_rows, lay.audio_cond_rows,
                lay.audio_target_rows] == g["rows"]
        flat = []
        for i in range(lay.seq_len):
            p = lay.positions[i]
            flat += [p.t, p.h, p.w]
        raw = struct.pack("<%dd" % len(flat), *flat)
        assert hashlib.sha256(raw).hexdigest() == g["positions_sha256"]
        for i, t, h, w in g["sample"]:
            p = lay.positions[i]
            got = [struct.unpack("<Q", struct.pack("<d", x))[0]
                   for x in (p.t, p.h, p.w)]
            assert got == [t, h, w], (name, i)
    finally:
        L.h3hip_layout_free(C.byref(lay))


def test_layout_checksum_literals():
    """reference tests/test_h3.c:176-192 (tiny layout)"""
    ok, lay, _ = layout(12, 2, 2, 2, 8, 5)
    assert ok and lay.seq_len == 30
    t = [lay.positions[i].t for i in range(30)]
    assert abs(sum(t) - 339.6666666666667) <= 1e-10
    assert abs(sum((i + 1) * x for i, x in enumerate(t)) - 6498.0) <= 1e-10
    L.h3hip_layout_free(C.byref(lay))


def test_layout_rejects_bad_input():
    assert not layout(0, 2, 2, 2, 8, 5)[0]
    assert not layout(12, 2, 3, 2, 8, 5)[0]           # odd latent height
    ok, _, err = layout(12, 2, 2, 2, 8, 56, keys=[3])
    assert not ok and "keyframes" in err
    ok, _, err = layout(12, 2, 2, 2, 8, 56, keys=[0],
                        refs=[(0, 0, 2, 2, 0)])
    assert not ok and "exclusive" in err


# ------------------------------------------------------------------- RNG

@pytest.mark.parametrize("seed", sorted(GOLDEN["rng"], key=int))
def test_rng_streams_bit_exact(seed):
    g = GOLDEN["rng"][seed]
    r = h3hip.Rng()
    L.h3hip_rng_seed(C.byref(r), int(seed))
    assert [L.h3hip_rng_u32(C.byref(r)) for _ in range(64)] == g["u32"]
    r = h3hip.Rng()
    L.h3hip_rng_seed(C.byref(r), int(seed))
    vals = np.zeros(65, np.float32)
    L.h3hip_rng_fill_normal(C.byref(r), h3hip.ptr(vals), 65)
    assert fbits(vals) == g["normal"]


def test_pcg32_definition():
    """PCG32 XSH-RR (O'Neill 2014) restated in Python matches the stream."""
    mask = (1 << 64) - 1

    def step(state, inc):
        old = state
        state = (old * 6364136223846793005 + inc) & mask
        xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
        rot = old >> 59
        return state, ((xs >> rot) | (xs << ((-rot) & 31))) & 0xFFFFFFFF

    seed = 42
    inc = ((seed << 1) | 1) & mask
    state, _ = step(0, inc)
    state = (state + (seed ^ 0x9E3779B97F4A7C15)) & mask
    state, _ = step(state, inc)
    want = []
    for _ in range(16):
        state, v = step(state, inc)
        want.append(v)
    assert GOLDEN["rng"]["42"]["u32"][:16] == want


# ------------------------------------------------------------ RoPE tables

def test_rope_tables_match_libm_restatement():
    """h3_dit.c:907-922: angle = (float)axis * inv_freq[f] in float, cosf /
    sinf from libm, index row*48 + axis*16 + f."""
    libm = C.CDLL("libm.so.6")
    libm.cosf.restype = C.c_float
    libm.cosf.argtypes = [C.c_float]
    libm.sinf.restype = C.c_float
    libm.sinf.argtypes = [C.c_float]
    ok, lay, _ = layout(12, 2, 4, 6, 8, 5)
    n = lay.seq_len
    pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                     lay.positions[i].w] for i in range(n)])
    L.h3hip_layout_free(C.byref(lay))
    inv = np.empty(16, np.float32)
    L.h3hip_default_inv_freq(h3hip.ptr(inv))
    np.testing.assert_array_equal(
        inv, np.array([10000.0 ** (-f / 16.0) for f in range(16)], np.float32))
    scale = 0.75
    c = np.empty(n * 48, np.float32)
    s = np.empty(n * 48, np.float32)
    L.h3hip_rope_tables(h3hip.ptr(pos), n, h3hip.ptr(inv), C.c_float(scale),
                        h3hip.ptr(c), h3hip.ptr(s))
    for r in range(n):
        axes = [np.float32(pos[r, 0]), np.float32(np.float32(pos[r, 1]) *
                                                  np.float32(scale)),
                np.float32(np.float32(pos[r, 2]) * np.float32(scale))]
        for a in range(3):
            for f in range(16):
                ang = np.float32(axes[a] * inv[f])
                i = r * 48 + a * 16 + f
                assert c[i] == np.float32(libm.cosf(float(ang)))
                assert s[i] == np.float32(libm.sinf(float(ang)))
    # row 0 is text position (0, 0, 0): identity rotation
    assert np.all(c[:48] == 1.0) and np.all(s[:48] == 0.0)


# ---------------------------------------------- timestep rows and row maps

def test_time_rows_and_row_map():
    """h3_dit_schedule.c:99-160 and 434-485 on the 4-evaluation serving grid:
    video and audio time rows are interleaved by t = 1 - sigma (equal t
    shares a row), then text rows map to video_row*3+1, audio to
    audio_row*3+2, video to video_row*3+0."""
    ok, v, a = _grid(L.h3hip_serving_schedule_build, 4)
    steps = 4
    vr = np.zeros(steps, np.uint32)
    ar = np.zeros(steps, np.uint32)
    n = L.h3hip_time_rows(steps, h3hip.ptr(v), h3hip.ptr(a), 0, 0,
                          h3hip.ptr(vr), h3hip.ptr(ar), None, None, None)
    times = np.zeros(n, np.float32)
    L.h3hip_time_rows(steps, h3hip.ptr(v), h3hip.ptr(a), 0, 0, h3hip.ptr(vr),
                      h3hip.ptr(ar), None, None, h3hip.ptr(times))
    # step 0: sigma 1 for both -> one shared row; later steps: video sigma
    # (shift 12) > audio sigma (shift 3) -> video t < audio t -> video first
    assert vr.tolist() == [0, 1, 3, 5] and ar.tolist() == [0, 2, 4, 6]
    assert n == 7
    for s in range(steps):
        assert times[vr[s]] == np.float32(1) - v[s]
        assert times[ar[s]] == np.float32(1) - a[s]
    ok, lay, _ = layout(12, 2, 2, 2, 8, 5)
    rows = np.zeros(lay.seq_len, np.uint32)
    assert L.h3hip_row_map(C.byref(lay), int(vr[2]), int(ar[2]), 0xFFFFFFFF,
                           0xFFFFFFFF, None, 0, h3hip.ptr(rows), lay.seq_len)
    assert rows[:12].tolist() == [3 * 3 + 1] * 12          # text
    assert rows[12:28].tolist() == [4 * 3 + 2] * 16        # audio
    assert rows[28:30].tolist() == [3 * 3 + 0] * 2         # video
    tags = np.array([0, 1, 2] * 4, np.uint8)
    assert L.h3hip_row_map(C.byref(lay), 1, 2, 0xFFFFFFFF, 0xFFFFFFFF,
                           h3hip.ptr(tags), 12, h3hip.ptr(rows), lay.seq_len)
    assert rows[:12].tolist() == [3 + t for t in tags.tolist()]
    bad = np.array([3] * 12, np.uint8)
    assert not L.h3hip_row_map(C.byref(lay), 1, 2, 0xFFFFFFFF, 0xFFFFFFFF,
                               h3hip.ptr(bad), 12, h3hip.ptr(rows),
                               lay.seq_len)
    L.h3hip_layout_free(C.byref(lay))


def test_timestep_features():
    """h3_dit_schedule.c:146-157: [cos(t f_i), sin(t f_i)], f_i =
    exp(-ln(1e4) i / 128)."""
    times = np.array([0.0, 0.5, 1.0], np.float32)
    feats = np.empty(3 * 256, np.float32)
    L.h3hip_timestep_features(h3hip.ptr(times), 3, h3hip.ptr(feats))
    feats = feats.reshape(3, 256)
    assert np.all(feats[0, :128] == 1.0) and np.all(feats[0, 128:] == 0.0)
    f = np.exp(-math.log(1e4) * np.arange(128) / 128.0)
    np.testing.assert_allclose(feats[1, :128], np.cos(0.5 * f), atol=2e-7)
    np.testing.assert_allclose(feats[2, 128:], np.sin(f), atol=2e-7)


# ------------------------------------------------------ row conversions

def test_patchify_and_pack_known_answers():
    """reference tests/test_h3.c:357-380"""
    C_, T, H, W = 3, 2, 4, 6
    latent = np.arange(C_ * T * H * W, dtype=np.float32)
    rows = np.empty_like(latent)
    assert L.h3hip_patchify_video(h3hip.ptr(latent), C_, T, H, W,
                                  h3hip.ptr(rows), latent.size)
    assert rows[:12].tolist() == [0, 1, 6, 7, 48, 49, 54, 55, 96, 97, 102, 103]
    back = np.empty_like(latent)
    assert L.h3hip_unpatchify_video(h3hip.ptr(rows), C_, T, H, W,
                                    h3hip.ptr(back), latent.size)
    np.testing.assert_array_equal(back, latent)
    assert not L.h3hip_patchify_video(h3hip.ptr(latent), C_, T, H, W,
                                      h3hip.ptr(rows), latent.size - 1)
    AC, AT = 4, 3
    audio = np.arange(AC * 2 * AT, dtype=np.float32)
    packed = np.empty_like(audio)
    assert L.h3hip_pack_audio(h3hip.ptr(audio), AC, AT, h3hip.ptr(packed),
                              audio.size)
    assert packed.tolist() == [0, 6, 12, 18, 1, 7, 13, 19, 2, 8, 14, 20, 3, 9,
                               15, 21, 4, 10, 16, 22, 5, 11, 17, 23]
    un = np.empty_like(audio)
    assert L.h3hip_unpack_audio(h3hip.ptr(packed), AC, AT, h3hip.ptr(un),
                                audio.size)
    np.testing.assert_array_equal(un, audio)


def test_host_euler_literal():
    """reference tests/test_h3.c:324-328"""
    v = np.array([2.0, -4.0], np.float32)
    x = np.array([1.0, 3.0], np.float32)
    assert L.h3hip_euler_velocity_step(h3hip.ptr(x), h3hip.ptr(v), 2,
                                       C.c_float(0.75), C.c_float(0.25))
    assert x.tolist() == [2.0, 1.0]
    assert not L.h3hip_euler_velocity_step(h3hip.ptr(x), h3hip.ptr(v), 2,
                                           C.c_float(0.25), C.c_float(0.25))


def test_safetensors_index_reads_the_header(tmp_path):
    """The header walk used to locate tensors in a safetensors file, checked
    on a file written by the safetensors library itself."""
    np_st = pytest.importorskip("safetensors.numpy")
    import h3hip
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = np.arange(5, dtype=np.uint16)
    path = str(tmp_path / "m.safetensors")
    np_st.save_file({"a": a, "b": b}, path)
    idx = h3hip.safetensors_index(path)
    raw = open(path, "rb").read()
    assert idx["a"][:2] == ("F32", (3, 4)) and idx["b"][:2] == ("U16", (5,))
    for name, arr in (("a", a), ("b", b)):
        _, _, off, nbytes = idx[name]
        assert raw[off:off + nbytes] == arr.tobytes()
