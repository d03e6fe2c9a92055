"""Write tests/golden/host_golden.json from the reference's own host math.

Loads oracle/_ref/libh3ref.so -- /root/reference/h3_host.c compiled as is
by `make -C oracle ref` -- and records its outputs for the functions the DiT
path depends on bit for bit: temporal shapes, both sigma grids, the packed
layout with (t, h, w) positions, and the PCG32 / Box-Muller streams.  Run it
in the container that holds /root/reference:

    make -C oracle ref && python tests/golden/make_golden.py

The fixture is data only (inputs and the reference's outputs); floats are
stored as IEEE bit patterns so the comparison is exact.
"""
import ctypes as C
import hashlib
import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.path.join(ROOT, "oracle", "_ref", "libh3ref.so")
MAX_STEPS = 1000


class Temporal(C.Structure):
    _fields_ = [("frame_count", C.c_int), ("video_t", C.c_int),
                ("audio_t", C.c_int)]


class Position(C.Structure):
    _fields_ = [("t", C.c_double), ("h", C.c_double), ("w", C.c_double)]


class Segment(C.Structure):
    _fields_ = [("start", C.c_size_t), ("stop", C.c_size_t),
                ("kind", C.c_int)]


class LayoutRef(C.Structure):
    _fields_ = [("kind", C.c_int), ("latent_t", C.c_int),
                ("latent_h", C.c_int), ("latent_w", C.c_int),
                ("audio_t", C.c_int)]


class LayoutSpec(C.Structure):
    _fields_ = [("text_len", C.c_int), ("latent_t", C.c_int),
                ("latent_h", C.c_int), ("latent_w", C.c_int),
                ("audio_t", C.c_int), ("frame_count", C.c_int),
                ("keyframes", C.POINTER(C.c_int)),
                ("keyframe_count", C.c_size_t),
                ("references", C.POINTER(LayoutRef)),
                ("reference_count", C.c_size_t)]


class Layout(C.Structure):
    _fields_ = [("seq_len", C.c_size_t), ("segments", C.POINTER(Segment)),
                ("segment_count", C.c_size_t),
                ("positions", C.POINTER(Position)),
                ("img_cond_rows", C.c_size_t),
                ("img_target_rows", C.c_size_t),
                ("audio_cond_rows", C.c_size_t),
                ("audio_target_rows", C.c_size_t),
                ("signature", C.c_int * 5)]


class Sigmas(C.Structure):
    _fields_ = [("steps", C.c_int), ("video", C.c_float * (MAX_STEPS + 1)),
                ("audio", C.c_float * (MAX_STEPS + 1))]


class Rng(C.Structure):
    _fields_ = [("state", C.c_uint64), ("increment", C.c_uint64),
                ("spare", C.c_float), ("has_spare", C.c_int)]


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def dbits(x):
    return struct.unpack("<Q", struct.pack("<d", x))[0]


# Layout cases: (name, text, latent_t, latent_h, latent_w, audio_t, frames,
#                keyframes, references)
LAYOUTS = [
    ("tiny", 12, 2, 2, 2, 8, 5, [], []),                    # test_h3.c:176
    ("fl2va", 128, 17, 30, 54, 93, 56, [0, 55], []),        # test_h3.c:194
    ("ref2va", 192, 17, 30, 54, 93, 56, [],                 # test_h3.c:219
     [(0, 0, 16, 24, 0), (2, 7, 16, 24, 48), (1, 0, 0, 0, 80)]),
    ("t2va_512x512x22", 512, 7, 32, 32, 37, 22, [], []),    # BASELINE 512^2
    ("t2va_864x480x22", 512, 7, 30, 54, 37, 22, [], []),    # BASELINE 864x480
    ("t2va_256x256x22", 256, 7, 16, 16, 37, 22, [], []),    # CPU config
]


def main():
    L = C.CDLL(REF)
    L.h3_temporal.restype = Temporal
    L.h3_temporal.argtypes = [C.c_int]
    L.h3_schedule_build.argtypes = [C.c_int, C.POINTER(Sigmas)]
    L.h3_serving_schedule_build.argtypes = [C.c_int, C.POINTER(Sigmas)]
    L.h3_layout_build.argtypes = [C.POINTER(LayoutSpec), C.POINTER(Layout),
                                  C.c_char_p, C.c_size_t]
    L.h3_layout_free.argtypes = [C.POINTER(Layout)]
    L.h3_rng_seed.argtypes = [C.POINTER(Rng), C.c_uint64]
    L.h3_rng_u32.restype = C.c_uint32
    L.h3_rng_u32.argtypes = [C.POINTER(Rng)]
    L.h3_rng_normal.restype = C.c_float
    L.h3_rng_normal.argtypes = [C.POINTER(Rng)]
    L.h3_video_latent_t.argtypes = [C.c_int]
    L.h3_align_frame_count.argtypes = [C.c_int]

    out = {"source": "reference h3_host.c compiled by oracle/Makefile ref"}
    out["temporal"] = []
    for req in [1, 5, 6, 17, 22, 23, 39, 56, 57, 124, 241, 361, 362, 500]:
        t = L.h3_temporal(req)
        out["temporal"].append([req, t.frame_count, t.video_t, t.audio_t])

    def grid(fn, n):
        s = Sigmas()
        ok = fn(n, C.byref(s))
        if not ok:
            return None
        return {"video": [fbits(s.video[i]) for i in range(n + 1)],
                "audio": [fbits(s.audio[i]) for i in range(n + 1)]}

    out["schedule"] = {str(n): grid(L.h3_schedule_build, n)
                       for n in [1, 2, 4, 7, 20, 29, 50, 100, 1000]}
    out["serving_schedule"] = {str(n): grid(L.h3_serving_schedule_build, n)
                               for n in [2, 3, 4, 11, 19, 20, 50, 1000]}

    out["layouts"] = {}
    for name, text, lt, lh, lw, at, frames, keys, refs in LAYOUTS:
        karr = (C.c_int * max(1, len(keys)))(*keys)
        rarr = (LayoutRef * max(1, len(refs)))(*[LayoutRef(*r) for r in refs])
        spec = LayoutSpec(text, lt, lh, lw, at, frames, karr, len(keys), rarr,
                          len(refs))
        lay = Layout()
        err = C.create_string_buffer(256)
        assert L.h3_layout_build(C.byref(spec), C.byref(lay), err, 256), \
            err.value
        n = lay.seq_len
        flat = []
        for i in range(n):
            p = lay.positions[i]
            flat += [p.t, p.h, p.w]
        raw = struct.pack("<%dd" % len(flat), *flat)
        entry = {
            "spec": [text, lt, lh, lw, at, frames, keys, refs],
            "seq_len": n,
            "segments": [[lay.segments[i].start, lay.segments[i].stop,
                          lay.segments[i].kind]
                         for i in range(lay.segment_count)],
            "rows": [lay.img_cond_rows, lay.img_target_rows,
                     lay.audio_cond_rows, lay.audio_target_rows],
            "positions_sha256": hashlib.sha256(raw).hexdigest(),
            # every 97th row in full, as exact double bits
            "sample": [[i, dbits(lay.positions[i].t), dbits(lay.positions[i].h),
                        dbits(lay.positions[i].w)] for i in range(0, n, 97)],
        }
        out["layouts"][name] = entry
        L.h3_layout_free(C.byref(lay))

    out["rng"] = {}
    for seed in [0, 1, 7, 42, 2**40 + 3]:
        r = Rng()
        L.h3_rng_seed(C.byref(r), seed)
        u = [L.h3_rng_u32(C.byref(r)) for _ in range(64)]
        r2 = Rng()
        L.h3_rng_seed(C.byref(r2), seed)
        nrm = [fbits(L.h3_rng_normal(C.byref(r2))) for _ in range(65)]
        out["rng"][str(seed)] = {"u32": u, "normal": nrm}

    path = os.path.join(HERE, "host_golden.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
