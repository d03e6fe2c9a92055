"""The reference engine's own model layer on this backend: h3_dit.c's
h3_dit_load_t2va + h3_dit_forward (reference h3_dit.c:1690-1872,
2574-2638), compiled unmodified from the reference sources into
oracle/_ref/engine_forward and linked to libh3_gpu_hip.so, runs one forward
on a synthetic checkpoint at the real H3 widths (hidden 5376, 56 heads,
SwiGLU 14336, 25 active blocks).  Its velocities must agree with this
repository's driver (h3hip_dit_forward_step) run on the same weights.

The checkpoint is written as safetensors shards in the format h3_weights.c
reads.  To keep it to ~6 GB of data, most big matrices are zero (file
holes): a block whose QKV / out / fc1 / fc2 are zero returns its input bit
for bit (zero branches under any gate), so the engine's 25 active blocks
reduce to the five that carry seeded weights, which the driver runs.  The
AdaLN projection weights are zero and their biases seeded, so every block's
modulation is its bias at every time row (the projection adds the bias to a
zero product exactly).  Norms, biases, the refiner, the patch projections
and the final heads are seeded.

The engine binary is built by `make -C oracle ref` (it needs the reference
tree at build time only); the test skips where it is absent.
"""
import ctypes as C
import json
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import h3hip
import oracle
from conftest import cosine_rel_l2

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE = os.path.join(ROOT, "oracle", "_ref", "engine_forward")
L = h3hip.lib()

H, HEADS, HD, FFN, TEXT_DIM, TIME_DIM = 5376, 56, 128, 14336, 5120, 2688
INNER = HEADS * HD
BLOCKS, ACTIVE = 50, 25


def uniform_active_blocks(active, blocks=BLOCKS):
    """configure_active_blocks (h3_dit.c:1312-1322): the skipped blocks are
    spread evenly, never the first or last."""
    keep = [True] * blocks
    skipped = blocks - active
    for i in range(skipped):
        b = ((2 * i + 1) * blocks) // (2 * skipped)
        b = max(b, 1)
        b = min(b, blocks - 2)
        keep[b] = False
    return [b for b in range(blocks) if keep[b]]


class Shard:
    """A safetensors file built tensor by tensor: 8-byte header length,
    JSON header, data (each tensor 4 KiB aligned; None payloads stay file
    holes, i.e. zeros)."""

    def __init__(self):
        self.entries = []
        self.size = 0

    def add(self, name, dtype, shape, payload=None):
        item = 2 if dtype == "BF16" else 4
        nbytes = int(np.prod(shape)) * item
        self.size = (self.size + 4095) & ~4095
        self.entries.append((name, dtype, list(shape), self.size, nbytes,
                             payload))
        self.size += nbytes

    def write(self, path):
        header = {n: {"dtype": d, "shape": s, "data_offsets": [o, o + b]}
                  for n, d, s, o, b, _ in self.entries}
        text = json.dumps(header).encode()
        pad = (-(8 + len(text))) % 4096
        text += b" " * pad
        base = 8 + len(text)
        with open(path, "wb") as f:
            f.write(len(text).to_bytes(8, "little"))
            f.write(text)
            for _, _, _, off, nbytes, payload in self.entries:
                if payload is None:
                    continue
                f.seek(base + off)
                data = payload() if callable(payload) else payload
                assert data.nbytes == nbytes
                f.write(memoryview(np.ascontiguousarray(data)).cast("B"))
            f.truncate(base + self.size)
        return base


def make_checkpoint(rng):
    """The synthetic checkpoint (a Shard to write) and the seeded values the
    driver needs."""
    pool = oracle.bf16((0.02 * rng.standard_normal(1 << 26)).astype(
        np.float32))

    def big(n):
        out = np.empty(n, np.uint16)
        at, src = 0, int(rng.integers(0, pool.size))
        while at < n:
            take = min(n - at, pool.size - src)
            out[at:at + take] = pool[src:src + take]
            at, src = at + take, 0
        return out

    def vec(n, std, mean=0.0):
        return oracle.bf16((mean + std * rng.standard_normal(n)).astype(
            np.float32))

    def f32_bf16_exact(n, std):
        return oracle.f32(vec(n, std)).astype(np.float32)

    active = uniform_active_blocks(ACTIVE)
    assert len(active) == ACTIVE and active[0] == 0 and active[-1] == 49
    seeded = [active[i] for i in (0, 1, 12, 23, 24)]
    shard = Shard()
    weights = {}

    def block(prefix, key, dense):
        w = {"norm1": vec(H, 0.1, 1.0), "norm2": vec(H, 0.1, 1.0),
             "q_norm": vec(HD, 0.1, 1.0), "k_norm": vec(HD, 0.1, 1.0)}
        for name, shape in (("qkv", (3 * INNER, H)), ("out", (H, INNER)),
                            ("fc1", (2 * FFN, H)), ("fc2", (H, FFN))):
            w[name] = big(shape[0] * shape[1]) if dense else None
        names = {"norm1": "norm1.weight", "norm2": "norm2.weight",
                 "qkv": "attn.qkv_proj.weight", "q_norm": "attn.q_norm.weight",
                 "k_norm": "attn.k_norm.weight", "out": "attn.out_proj.weight",
                 "fc1": "mlp.fc1.weight", "fc2": "mlp.fc2.weight"}
        shapes = {"norm1": (H,), "norm2": (H,), "q_norm": (HD,),
                  "k_norm": (HD,), "qkv": (3 * INNER, H), "out": (H, INNER),
                  "fc1": (2 * FFN, H), "fc2": (H, FFN)}
        for k, n in names.items():
            shard.add(prefix + n, "BF16", shapes[k], w[k])
        if key is not None:
            weights[key] = w

    for b in active:
        block(f"blocks.{b}.", ("block", b) if b in seeded else None,
              b in seeded)
    mods = {}
    for b in range(BLOCKS):
        mods[b] = vec(3 * 6 * H, 0.1)
        shard.add(f"blocks.{b}.adaln_proj.linear.weight", "BF16",
                  (3 * 6 * H, TIME_DIM))
        shard.add(f"blocks.{b}.adaln_proj.linear.bias", "BF16", (3 * 6 * H,),
                  mods[b])
    for i in range(2):
        block(f"token_refiner.blocks.{i}.", ("refiner", i), True)
    cond_w, cond_b = big(H * TEXT_DIM), vec(H, 0.02)
    shard.add("condition_proj.weight", "BF16", (H, TEXT_DIM), cond_w)
    shard.add("condition_proj.bias", "BF16", (H,), cond_b)
    ref_final = vec(H, 0.1, 1.0)
    shard.add("token_refiner.final_norm.weight", "BF16", (H,), ref_final)
    shard.add("time_embedder.proj_in.weight", "F32", (H, 256))
    shard.add("time_embedder.proj_in.bias", "F32", (H,))
    shard.add("time_embedder.proj_out.weight", "F32", (TIME_DIM, H))
    shard.add("time_embedder.proj_out.bias", "F32", (TIME_DIM,))
    inv_freq = np.empty(16, np.float32)
    L.h3hip_default_inv_freq(h3hip.ptr(inv_freq))
    shard.add("rope.inv_freq", "F32", (16,), inv_freq)
    final_mod = vec(2 * H, 0.1)
    shard.add("final_layer.adaln_proj.linear.weight", "BF16",
              (2 * H, TIME_DIM))
    shard.add("final_layer.adaln_proj.linear.bias", "BF16", (2 * H,),
              final_mod)
    final_norm = vec(H, 0.1, 1.0)
    shard.add("final_layer.norm.weight", "BF16", (H,), final_norm)
    heads = {"final_video_w": f32_bf16_exact(96 * H, 0.02),
             "final_video_b": f32_bf16_exact(96, 0.02),
             "final_audio_w": f32_bf16_exact(32 * H, 0.02),
             "final_audio_b": f32_bf16_exact(32, 0.02)}
    shard.add("final_layer.video_out.weight", "F32", (96, H),
              heads["final_video_w"])
    shard.add("final_layer.video_out.bias", "F32", (96,),
              heads["final_video_b"])
    shard.add("final_layer.audio_out.weight", "F32", (32, H),
              heads["final_audio_w"])
    shard.add("final_layer.audio_out.bias", "F32", (32,),
              heads["final_audio_b"])
    patch = {"video_patch_w": (0.05 * rng.standard_normal(H * 96)).astype(
                 np.float32),
             "video_patch_b": (0.02 * rng.standard_normal(H)).astype(
                 np.float32),
             "audio_patch_w": (0.05 * rng.standard_normal(H * 32)).astype(
                 np.float32),
             "audio_patch_b": (0.02 * rng.standard_normal(H)).astype(
                 np.float32)}
    shard.add("video_patch_proj.weight", "F32", (H, 96),
              patch["video_patch_w"])
    shard.add("video_patch_proj.bias", "F32", (H,), patch["video_patch_b"])
    shard.add("audio_patch_proj.weight", "F32", (H, 32),
              patch["audio_patch_w"])
    shard.add("audio_patch_proj.bias", "F32", (H,), patch["audio_patch_b"])

    text = vec(TEXT_ROWS * TEXT_DIM, 1.0)
    return dict(shard=shard, weights=weights, mods=mods, cond_w=cond_w,
                cond_b=cond_b, ref_final=ref_final, final_mod=final_mod,
                final_norm=final_norm, heads=heads, patch=patch,
                seeded=seeded, text=text)


TEXT_ROWS = 256


def test_reference_engine_forward_matches_driver(gpu):
    if not os.path.exists(ENGINE):
        pytest.skip("oracle/_ref/engine_forward not built (make -C oracle ref)")
    ck = make_checkpoint(np.random.default_rng(2024))
    shard, weights, mods, seeded, text = (ck["shard"], ck["weights"],
                                          ck["mods"], ck["seeded"],
                                          ck["text"])
    cond_w, cond_b, ref_final = ck["cond_w"], ck["cond_b"], ck["ref_final"]
    final_mod, final_norm = ck["final_mod"], ck["final_norm"]
    heads, patch = ck["heads"], ck["patch"]
    text_rows, lt, lh, lw, at, frames, steps, step = (TEXT_ROWS, 2, 16, 16, 8,
                                                      5, 4, 1)
    # tmpfs when it has room (no disk write-back), else the repository's
    # own file system; removed at the end either way
    where = ROOT
    if os.path.isdir("/dev/shm"):
        st = os.statvfs("/dev/shm")
        if st.f_bavail * st.f_frsize > 12 << 30:
            where = "/dev/shm"
    work = tempfile.mkdtemp(prefix=".engine_ckpt_", dir=where)
    try:
        shard.write(os.path.join(work, "model-00001-of-00001.safetensors"))
        text_path = os.path.join(work, "text.bin")
        text.tofile(text_path)
        print("engine: checkpoint written", flush=True)
        run = subprocess.run(
            [ENGINE, work, text_path, str(text_rows), str(lt), str(lh),
             str(lw), str(at), str(frames), str(steps), str(step),
             str(ACTIVE), "7", work],
            capture_output=True, text=True, timeout=600)
        print(run.stdout, run.stderr[-2000:], flush=True)
        assert run.returncode == 0, run.stderr[-2000:]
        ref_v = np.fromfile(os.path.join(work, "video_velocity.f32"),
                            np.float32)
        ref_a = np.fromfile(os.path.join(work, "audio_velocity.f32"),
                            np.float32)
        video_rows = np.fromfile(os.path.join(work, "video_rows.f32"),
                                 np.float32)
        audio_rows = np.fromfile(os.path.join(work, "audio_rows.f32"),
                                 np.float32)
    finally:
        shutil.rmtree(work, ignore_errors=True)

    # ---- the same forward through this repository's driver ----
    lay = h3hip.Layout()
    err = C.create_string_buffer(256)
    assert L.h3hip_layout_build(text_rows, lt, lh, lw, at, frames, None, 0,
                                None, 0, C.byref(lay), err, 256), err.value
    try:
        v_sig = np.zeros(steps + 1, np.float32)
        a_sig = np.zeros(steps + 1, np.float32)
        assert L.h3hip_serving_schedule_build(steps, h3hip.ptr(v_sig),
                                              h3hip.ptr(a_sig))
        vr = np.zeros(steps, np.uint32)
        ar = np.zeros(steps, np.uint32)
        n_time = L.h3hip_time_rows(steps, h3hip.ptr(v_sig), h3hip.ptr(a_sig),
                                   0, 0, h3hip.ptr(vr), h3hip.ptr(ar), None,
                                   None, None)
        rows = lay.seq_len
        pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                         lay.positions[i].w] for i in range(rows)])
        cos, sin = h3hip.rope_tables(pos)
        cfg = h3hip.dit_config(h3hip.FAMILY_H3, H, HEADS, FFN, rows,
                               blocks=len(seeded), time_rows=n_time)
        dit = h3hip.Dit(gpu, cfg)
        refiner = h3hip.Refiner(gpu, H, HEADS, FFN, TEXT_DIM)
        try:
            for i, b in enumerate(seeded):
                w = weights[("block", b)]
                for name in ("norm1", "norm2", "qkv", "q_norm", "k_norm",
                             "out", "fc1", "fc2"):
                    dit.write(name, w[name], i)
                dit.write("modulation", np.tile(mods[b], n_time), i)
            dit.set_rope(cos, sin)
            dit.sampler_create(lay, v_sig, a_sig, reuse_interval=1)
            dit.write("final_norm", final_norm)
            dit.write("final_modulation", np.tile(final_mod, n_time))
            for name, values in heads.items():
                dit.write(name, oracle.bf16(values))
            for name, values in patch.items():
                t = dit.tensor(name)
                assert L.h3_gpu_tensor_write_f32(t, h3hip.ptr(values),
                                                 values.size)
            for name, t in (("condition_w", cond_w), ("condition_b", cond_b),
                            ("final_norm", ref_final)):
                assert L.h3_gpu_tensor_write_bf16(
                    refiner.tensor(name), h3hip.ptr(t), t.size)
            for i in range(2):
                w = weights[("refiner", i)]
                for name in ("norm1", "norm2", "qkv", "q_norm", "k_norm",
                             "out", "fc1", "fc2"):
                    assert L.h3_gpu_tensor_write_bf16(
                        refiner.tensor(name, i), h3hip.ptr(w[name]),
                        w[name].size)
            src = gpu.bf16(text)
            refiner.run(dit.tensor("refined_text"), src, text_rows)
            gpu.free(src)
            dit.write_latents(video_rows, audio_rows)
            dit.forward_step(step)
            vrows, arows, vt, atr = dit.sampler_rows()
            got_v = dit.read("video_velocity")[:vt * 96]
            got_a = dit.read("audio_velocity")[:atr * 32]
        finally:
            refiner.close()
            dit.close()
    finally:
        L.h3hip_layout_free(C.byref(lay))
    for got, want, what in ((got_v, ref_v, "video"), (got_a, ref_a, "audio")):
        want_bits = oracle.bf16(want)
        assert got.size == want_bits.size, what
        cos_sim, rel = cosine_rel_l2(got, want_bits)
        same = int((got == want_bits).sum())
        print(f"engine vs driver {what}: cosine {cos_sim:.7f} rel-L2 "
              f"{rel:.3e}, {same}/{got.size} identical", flush=True)
        assert np.isfinite(want).all()
        assert cos_sim >= 0.999 and rel <= 1e-2, (what, cos_sim, rel)
