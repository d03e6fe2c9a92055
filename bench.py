"""Benchmark of the MI355X HIP backend on the DiT denoiser forward.

Workload (BASELINE.json metric "DiT block TFLOP/s + MFMA util %; s per
50-block forward @512x512x22f"): the Wan-shaped BF16 DiT block of the
benchmark configs -- hidden 5120, 40 heads x 128, GELU-tanh FFN 13824,
self-attention over 6 x 32 x 32 = 6144 video tokens with 3D RoPE, cross
attention to 512 text tokens, LayerNorm adaLN -- with all 50 blocks'
weights (~35 GB bf16, seeded random init on the device) resident in HBM.
One step = one 50-block forward; `value` = algorithmic TFLOP/s over the
timed steps.  Also reported: ms per block, s per 50-block forward, the
H3-real-shape forward (5376 hidden, 56 heads, SwiGLU, N = 2378), per-kernel
device times from HIP events on the backend's stream, the roofline of the
dominant kernel (the GEMMs), and the CPU oracle timed on a bounded sample
of the same workload (one Wan block at BASELINE config 1, 1536 video +
256 text rows).

    python bench.py [--gpus 1] [--steps 5] [--warmup 2] [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "h3.c_amd"))

import h3hip  # noqa: E402

BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


wan_positions = h3hip.wan_positions
rope_tables = h3hip.rope_tables


def time_forward(gpu, dit, blocks, steps, warmup):
    for _ in range(warmup):
        dit.run_blocks(0, blocks)
    L = gpu.L
    gpu.begin()
    L.h3_hip_marker(gpu.h, 0)
    wall = time.perf_counter()
    for _ in range(steps):
        if not L.h3hip_dit_run_blocks(dit.h, 0, blocks):
            raise RuntimeError(dit.error())
    L.h3_hip_marker(gpu.h, 1)
    gpu.submit()
    wall = time.perf_counter() - wall
    ms = __import__("ctypes").c_double()
    L.h3_hip_marker_elapsed(gpu.h, 0, 1, __import__("ctypes").byref(ms))
    return ms.value / steps, wall * 1000.0 / steps


OPS_GEMM, OPS_ACT, OPS_ATTN, OPS_ROWS, OPS_CTX = 1, 2, 4, 8, 16


KERNEL_NAMES = {
    "gemm_plain": "hk_gemm_mfma<0, false> (QKV, out, cross q, cross out, FFN "
                  "down)",
    "gemm_gelu": "hk_gemm_mfma<2, false> + split tail hk_gemm_mfma<3> "
                 "(FFN up + GELU)",
    "context_kv": "grouped hk_gemm_mfma<0, true>: the text's cross K/V of "
                  "all blocks in one launch",
    "attention": "hk_flash_fwd<false, false, 8 | 4> (self + cross, Q "
                 "norm (+ RoPE) applied as Q is loaded)",
    "row_ops": "adaLN / gates / Q-K norm + RoPE / head norm / residual rows",
}


def class_replay(gpu, dit, blocks, mask, reps=2):
    """Device ms of one forward's launches of one op class: the driver
    re-issues exactly those launches (same shapes, same tensors) for all
    blocks, bracketed by two HIP events on the backend's stream."""
    import ctypes as C
    L = gpu.L
    gpu.begin()
    if not L.h3hip_dit_run_blocks_ops(dit.h, 0, blocks, mask):  # warm
        raise RuntimeError(dit.error())
    L.h3_hip_marker(gpu.h, 2)
    for _ in range(reps):
        if not L.h3hip_dit_run_blocks_ops(dit.h, 0, blocks, mask):
            raise RuntimeError(dit.error())
    L.h3_hip_marker(gpu.h, 3)
    gpu.submit()
    ms = C.c_double()
    L.h3_hip_marker_elapsed(gpu.h, 2, 3, C.byref(ms))
    return ms.value / reps


def profile_pass(gpu, dit, blocks):
    """Launch pattern for counter collection: warm-up forward, one forward,
    one replay of the plain GEMMs, two launches of the modulation
    precompute's skinny GEMM, then add_bf16 over 64 Mi elements (reads
    2 x 128 MiB, writes 128 MiB) whose FETCH_SIZE / WRITE_SIZE readings scale
    the other kernels' counters to bytes."""
    L = gpu.L
    sep = gpu.new_f32(1)

    def separator():
        # an F32 fill, launched nowhere else in this pass, marks the
        # measured forward's first and last dispatch for the summariser
        gpu.begin()
        L.h3_gpu_fill_normal_f32(gpu.h, sep, 0, 1, 9, 0.0, 1.0)
        gpu.submit()
    dit.run_blocks(0, blocks)
    separator()
    dit.run_blocks(0, blocks)
    separator()
    gpu.begin()
    if not L.h3hip_dit_run_blocks_ops(dit.h, 0, blocks, OPS_GEMM):
        raise RuntimeError(dit.error())
    gpu.submit()
    # the modulation precompute's skinny projection at its H3 shape (39 time
    # rows x 2688 -> 3 x 6 x 5376), twice
    m, k, nn = 39, 2688, 3 * 6 * 5376
    x, w, y = gpu.new_bf16(m * k), gpu.new_bf16(nn * k), gpu.new_bf16(m * nn)
    gpu.begin()
    L.h3_gpu_fill_normal_bf16(gpu.h, x, 0, m * k, 7, 0.0, 1.0)
    L.h3_gpu_fill_normal_bf16(gpu.h, w, 0, nn * k, 8, 0.0, 0.02)
    for _ in range(2):
        gpu.check(L.h3_gpu_linear_bf16(gpu.h, y, x, w, None, m, k, nn),
                  "skinny linear")
    gpu.submit()
    for t in (x, w, y):
        gpu.free(t)
    n = 64 << 20
    a, b, c = gpu.new_bf16(n), gpu.new_bf16(n), gpu.new_bf16(n)
    gpu.begin()
    L.h3_gpu_fill_normal_bf16(gpu.h, a, 0, n, 5, 0.0, 1.0)
    L.h3_gpu_fill_normal_bf16(gpu.h, b, 0, n, 6, 0.0, 1.0)
    gpu.check(L.h3_gpu_add_bf16(gpu.h, c, a, b, n), "calibration add")
    gpu.submit()
    log("profile pass done")


def measured_peak(gpu, iterations=100000, reps=3):
    """The bf16 MFMA rate this GPU sustains with MFMAs alone
    (h3_hip_mfma_loop: one workgroup of four waves per CU, the GEMM's
    occupancy, 16 independent 32x32x16 MFMAs per iteration from registers,
    no LDS or memory traffic), timed by HIP events; the fastest of `reps`
    launches of about 20 ms each."""
    import ctypes as C
    L = gpu.L
    sink = gpu.new_f32(1024 * 256)
    flops = C.c_double()
    best = None
    gpu.begin()
    gpu.check(L.h3_hip_mfma_loop(gpu.h, sink, 1000, C.byref(flops)), "warm")
    gpu.submit()
    for _ in range(reps):
        gpu.begin()
        L.h3_hip_marker(gpu.h, 4)
        gpu.check(L.h3_hip_mfma_loop(gpu.h, sink, iterations, C.byref(flops)),
                  "mfma loop")
        L.h3_hip_marker(gpu.h, 5)
        gpu.submit()
        ms = C.c_double()
        L.h3_hip_marker_elapsed(gpu.h, 4, 5, C.byref(ms))
        tf = flops.value / (ms.value / 1e3) / 1e12
        best = tf if best is None else max(best, tf)
    gpu.free(sink)
    return best


def hbm_roof(gpu, mib=1024, reps=10):
    """The HBM rates plain streaming reaches on this GPU, for the row
    kernels' bytes to be read against: a device-to-device copy
    (hipMemcpyAsync through h3_gpu_copy_bf16) and this library's add_bf16
    (two reads, one write, 16 bytes per lane), over `mib` MiB operands,
    HIP events around `reps` launches after two warm-ups."""
    import ctypes as C
    L = gpu.L
    n = mib * (1 << 20) // 2
    a, b, c = gpu.new_bf16(n), gpu.new_bf16(n), gpu.new_bf16(n)
    gpu.begin()
    L.h3_gpu_fill_normal_bf16(gpu.h, a, 0, n, 5, 0.0, 1.0)
    L.h3_gpu_fill_normal_bf16(gpu.h, b, 0, n, 6, 0.0, 1.0)
    gpu.submit()
    out = {"operand_mib": mib}
    for key, launch, moved in (
            ("copy_gb_s", lambda: L.h3_gpu_copy_bf16(gpu.h, c, 0, a, 0, n),
             4 * n),
            ("add_bf16_gb_s", lambda: L.h3_gpu_add_bf16(gpu.h, c, a, b, n),
             6 * n)):
        gpu.begin()
        for _ in range(2):
            gpu.check(launch(), key)
        L.h3_hip_marker(gpu.h, 8)
        for _ in range(reps):
            gpu.check(launch(), key)
        L.h3_hip_marker(gpu.h, 9)
        gpu.submit()
        ms = C.c_double()
        L.h3_hip_marker_elapsed(gpu.h, 8, 9, C.byref(ms))
        out[key] = round(moved / (ms.value / reps / 1e3) / 1e9, 1)
    for t in (a, b, c):
        gpu.free(t)
    return out


def h3_measure(gpu, blocks, reps, latent_h=32, latent_w=32, full=True):
    """The H3 block at a real shape (512 text + 74 audio + video rows of a
    22-frame latent_h x latent_w latent: 2378 rows at 512x512, 3421 at
    864x480): one 50-block forward and, with full=True, the documented
    sparse window and BASELINE config 5, the 20-step serving-schedule Euler
    denoise with velocity reuse 2 (11 fresh forwards, extrapolated skipped
    steps), end to end on the GPU: patch projection, packing, blocks, final
    adaLN heads, Euler updates."""
    import ctypes as C
    L = h3hip.lib()
    lay = h3hip.Layout()
    err = C.create_string_buffer(256)
    if not L.h3hip_layout_build(512, 7, latent_h, latent_w, 37, 22, None, 0,
                                None, 0, C.byref(lay), err, 256):
        raise RuntimeError(err.value.decode())
    n = lay.seq_len
    pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                     lay.positions[i].w] for i in range(n)])
    steps = 20
    v_sig = np.zeros(steps + 1, np.float32)
    a_sig = np.zeros(steps + 1, np.float32)
    L.h3hip_serving_schedule_build(steps, h3hip.ptr(v_sig), h3hip.ptr(a_sig))
    vr = np.zeros(steps, np.uint32)
    ar = np.zeros(steps, np.uint32)
    time_rows = L.h3hip_time_rows(steps, h3hip.ptr(v_sig), h3hip.ptr(a_sig),
                                  0, 0, h3hip.ptr(vr), h3hip.ptr(ar), None,
                                  None, None)
    hcfg = h3hip.dit_config(h3hip.FAMILY_H3, 5376, 56, 14336, n,
                            blocks=blocks, time_rows=time_rows)
    hdit = h3hip.Dit(gpu, hcfg)
    try:
        hdit.init_random(seed=1, weight_std=0.02, mod_std=0.1)
        hc, hs = rope_tables(pos)
        hdit.set_rope(hc, hs)
        hdit.sampler_create(lay, v_sig, a_sig, reuse_interval=2)
        hdit.sampler_init_random(seed=2, weight_std=0.02, mod_std=0.1)
        # modulation of all 39 time rows from the random-init time MLP and
        # adaLN projections (reference h3_dit_schedule.c:78-337)
        # device time of the precompute's own ops (schedule_precompute_
        # device_s); the random-init fills of its (synthetic) projection
        # weights are timed apart; schedule_precompute_wall_s is the whole
        # call's wall clock, fills, uploads, syncs and timing events included
        L.h3_hip_op_timing_enable(gpu.h, 1)
        L.h3_hip_op_timing_reset(gpu.h)
        t0 = time.perf_counter()
        hdit.schedule_precompute(seed=3, weight_std=0.02)
        precompute_wall_s = time.perf_counter() - t0
        counts, all_ms, fill_ms = C.c_uint64(), C.c_double(), C.c_double()
        L.h3_hip_op_timing_read(gpu.h, b"", C.byref(counts), C.byref(all_ms))
        L.h3_hip_op_timing_read(gpu.h, b"fill_normal", C.byref(counts),
                                C.byref(fill_ms))
        L.h3_hip_op_timing_enable(gpu.h, 0)
        precompute_s = (all_ms.value - fill_ms.value) / 1e3
        precompute_fill_s = fill_ms.value / 1e3
        # forward alone, on the step-0 modulation rows
        hdit.gpu.begin()
        if not L.h3hip_dit_forward_step(hdit.h, 0):
            raise RuntimeError(hdit.error())
        hdit.gpu.submit()
        hms, _ = time_forward(gpu, hdit, blocks, reps, 1)
        hflops = hdit.block_flops()
        real = {"rows": int(n), "s_per_forward": round(hms / 1e3, 4),
                "ms_per_block": round(hms / blocks, 3),
                "tflops": round(blocks * hflops / (hms / 1e3) / 1e12, 1),
                "frac_of_peak": round(blocks * hflops / (hms / 1e3) / 1e12 /
                                      BF16_PEAK_TFLOPS, 4)}
        # per-class replays at this shape, as for the Wan forward
        cref = C.byref(hcfg)
        kern = {}
        for cname, mask, what in (
                ("gemm_plain", OPS_GEMM, "QKV + out-projection "
                 "(hk_gemm_mfma<0>, split tails)"),
                ("mlp_swiglu", OPS_ACT, "fc1 with SwiGLU epilogue "
                 "(hk_gemm_mfma<1>) + fc2 (hk_gemm_mfma<0>)"),
                ("attention", OPS_ATTN, "hk_flash_fwd (joint self-"
                 "attention, key-split last round)"),
                ("row_ops", OPS_ROWS, "adaLN / gate+adaLN / grouped Q-K "
                 "norm + RoPE rows")):
            cms = class_replay(gpu, hdit, blocks, mask)
            fl = L.h3hip_dit_block_class_flops(cref, mask)
            kern[cname] = {"kernel": what, "ms_per_forward": round(cms, 3)}
            if fl:
                tf = blocks * fl / (cms / 1e3) / 1e12
                kern[cname].update(tflops=round(tf, 1),
                                   frac_of_peak=round(tf / BF16_PEAK_TFLOPS,
                                                      4))
        real["kernels"] = kern
        gfl = (L.h3hip_dit_block_class_flops(cref, OPS_GEMM) +
               L.h3hip_dit_block_class_flops(cref, OPS_ACT))
        gms = kern["gemm_plain"]["ms_per_forward"] + \
            kern["mlp_swiglu"]["ms_per_forward"]
        gtf = blocks * gfl / (gms / 1e3) / 1e12
        real["roofline"] = {
            "kernel": "the block's GEMMs (QKV, out, fc1 SwiGLU, fc2)",
            "bound": "mfma", "achieved": round(gtf, 1),
            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(gtf / BF16_PEAK_TFLOPS, 4),
            "flops_per_block": gfl}
        if not full:
            return real, None
        # the reference's documented block-sparse window (README H3_SPARSE_ATTN
        # =16:8:14:8): forward time with the mask, then back to dense
        kept = L.h3hip_dit_set_sparse_window(hdit.h, C.byref(lay), 16, 8, 14,
                                             8, 0)
        if kept < 0:
            raise RuntimeError(hdit.error())
        sms, _ = time_forward(gpu, hdit, blocks, reps, 1)
        L.h3hip_dit_set_sparse_window(hdit.h, None, 0, 0, 0, 0, 1)
        qb, kt = (n + 127) // 128, (n + 63) // 64
        real["sparse_16_8_14_8"] = {
            "tiles_kept_frac": round(kept / (qb * kt), 4),
            "s_per_forward": round(sms / 1e3, 4)}
        t0 = time.perf_counter()
        evaluations = hdit.denoise()
        seconds = time.perf_counter() - t0
        v_out, a_out = hdit.read_latents()
        if not (np.isfinite(v_out).all() and np.isfinite(a_out).all()):
            raise RuntimeError("denoise produced non-finite latents")
        den = {"config": "BASELINE config 5: 20-step serving-schedule Euler "
                         "denoise, velocity reuse 2, H3 512x512x22f "
                         "(2378 rows), 50 blocks",
               "steps": steps, "fresh_forwards": int(evaluations),
               "seconds": round(seconds, 3),
               "s_per_fresh_forward": round(seconds / evaluations, 4),
               "schedule_precompute_device_s": round(precompute_s, 4),
               "schedule_precompute_wall_s": round(precompute_wall_s, 4),
               "schedule_weight_fill_s": round(precompute_fill_s, 4),
               "time_rows": int(time_rows)}
    finally:
        hdit.close()
        L.h3hip_layout_free(C.byref(lay))
    return real, den


def attention_sweep(gpu):
    """flash attention alone, bf16, 40 heads x 128, Q/K/V
    ~ N(0, 1).  Self-attention at 6144 rows (6 x 32 x 32) and 9720 rows
    (6 x 30 x 54) with the 3D RoPE of those grids applied by the call
    (h3_hip_sdpa_rope_bf16: Q rotated in the attention kernel as it is
    loaded, K once per key row by a pre-pass; the time covers both), and the
    same attention on pre-rotated Q/K without it
    (h3_gpu_sdpa_bf16, the kernel the blocks use after their Q/K norm +
    RoPE pass); cross-attention of those queries against 512 keys.  HIP
    events around 10 launches each, in two alternating passes, the faster
    kept."""
    import ctypes as C
    L = gpu.L
    out = {}
    scale = C.c_float(128 ** -0.5)
    heads = 40
    cases = (("self_6144", 6144, 6144, (6, 32, 32)),
             ("self_9720", 9720, 9720, (6, 30, 54)),
             ("cross_6144x512", 6144, 512, None),
             ("cross_9720x512", 9720, 512, None))
    for name, q_rows, kv_rows, grid in cases:
        tq = gpu.new_bf16(q_rows * heads * 128)
        tk = gpu.new_bf16(kv_rows * heads * 128)
        tv = gpu.new_bf16(kv_rows * heads * 128)
        to = gpu.new_bf16(q_rows * heads * 128)
        gpu.begin()
        for i, t in enumerate((tq, tk, tv)):
            L.h3_gpu_fill_normal_bf16(gpu.h, t, 0,
                                      L.h3_gpu_tensor_elements(t), 40 + i,
                                      0.0, 1.0)
        gpu.submit()
        tc = ts = None
        if grid:
            cos, sin = rope_tables(wan_positions(*grid))
            tc, ts = gpu.bf16(cos), gpu.bf16(sin)
        variants = ((name, "rope"), (name + "_no_rope", "plain")) if grid \
            else ((name, "cross"),)
        best = {}
        # two alternating passes, the faster of each kept: the first launches
        # after the fills run slow whichever variant comes first
        for label, mode in variants * 2:
            def launch():
                if mode == "rope":
                    return L.h3_hip_sdpa_rope_bf16(gpu.h, to, tq, tk, tv, tc,
                                                   ts, q_rows, heads, 128, 48,
                                                   scale)
                if mode == "plain":
                    return L.h3_gpu_sdpa_bf16(gpu.h, to, tq, tk, tv, q_rows,
                                              heads, 128, scale)
                return L.h3_gpu_sdpa_cross_bf16(gpu.h, to, tq, tk, tv, q_rows,
                                                kv_rows, heads, 128, scale)
            gpu.begin()
            for _ in range(2):
                launch()
            L.h3_hip_marker(gpu.h, 6)
            reps = 10
            for _ in range(reps):
                if not launch():
                    raise RuntimeError(gpu.error())
            L.h3_hip_marker(gpu.h, 7)
            gpu.submit()
            ms = C.c_double()
            L.h3_hip_marker_elapsed(gpu.h, 6, 7, C.byref(ms))
            t = ms.value / reps
            if label in best and best[label] <= t:
                continue
            best[label] = t
            tf = 4.0 * q_rows * kv_rows * heads * 128 / (t / 1e3) / 1e12
            out[label] = {"us": round(t * 1e3, 1), "tflops": round(tf, 1),
                          "frac_of_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
            if mode == "rope":
                out[label]["rope"] = ("3D RoPE: Q in the attention kernel, "
                                      "K by a pre-pass; both timed")
        for t_ in (tq, tk, tv, to, tc, ts):
            if t_ is not None:
                gpu.free(t_)
    return out


def wan_864x480(gpu, blocks, reps):
    """the Wan-shaped 50-block forward at 864x480x22f
    (6 x 30 x 54 = 9720 video rows, 512 text rows), weights resident."""
    rows, text = 6 * 30 * 54, 512
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, 5120, 40, 13824, rows,
                           blocks=blocks, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=4, weight_std=0.02, mod_std=0.1)
        cos, sin = rope_tables(wan_positions(6, 30, 54))
        dit.set_rope(cos, sin)
        ms, _ = time_forward(gpu, dit, blocks, reps, 1)
        flops = dit.block_flops()
        return {"rows": rows, "text_rows": text,
                "s_per_forward": round(ms / 1e3, 4),
                "ms_per_block": round(ms / blocks, 3),
                "tflops": round(blocks * flops / (ms / 1e3) / 1e12, 1),
                "tflop_per_block": round(flops / 1e12, 3)}
    finally:
        dit.close()


def weight_load(size_gib=2.0):
    """File -> HBM throughput of h3_gpu_tensor_load_bf16 (the pipelined
    loader), O_DIRECT and buffered, against read-everything-then-upload
    (np.fromfile, then h3_gpu_tensor_from_bf16: the reference's load
    order), each with the file's pages evicted from the page cache first
    ("cold": fsync, then posix_fadvise(DONTNEED) before every repetition, so
    the bytes come from the disk) and, for the buffered legs, with the file
    read once just before ("hot": page-cache resident).  Best of 3 per leg.
    O_DIRECT bypasses the page cache, so it has one leg."""
    import shutil
    import tempfile
    n = int(size_gib * (1 << 30)) // 2
    d = tempfile.mkdtemp(prefix=".bench_load_", dir=ROOT)
    out = {"bytes": 2 * n, "file": "random bytes behind a 4 KiB header"}
    try:
        path = os.path.join(d, "weights.bin")
        with open(path, "wb") as f:
            f.write(b"\0" * 4096)
            np.random.default_rng(0).integers(
                0, 1 << 16, n, dtype=np.uint16).tofile(f)
            f.flush()
            os.fsync(f.fileno())

        def evict():
            fd = os.open(path, os.O_RDONLY)
            try:
                os.fsync(fd)
                os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
            finally:
                os.close(fd)

        def warm():
            with open(path, "rb") as f:
                while f.read(64 << 20):
                    pass

        gpu = h3hip.Gpu()
        try:
            def loader():
                t = gpu.load(path, 4096, n)
                gpu.free(t)

            def read_upload():
                a = np.fromfile(path, dtype=np.uint16, offset=4096)
                t = gpu.bf16(a)
                gpu.free(t)

            legs = (("direct_gb_s", "1", loader, evict),
                    ("buffered_cold_gb_s", "0", loader, evict),
                    ("buffered_hot_gb_s", "0", loader, warm),
                    ("read_then_upload_cold_gb_s", None, read_upload, evict),
                    ("read_then_upload_hot_gb_s", None, read_upload, warm))
            for key, env, fn, prep in legs:
                if env is None:
                    os.environ.pop("H3_HIP_DIRECT_IO", None)
                else:
                    os.environ["H3_HIP_DIRECT_IO"] = env
                best = None
                for _ in range(3):
                    prep()
                    t0 = time.perf_counter()
                    fn()
                    dt = time.perf_counter() - t0
                    best = dt if best is None else min(best, dt)
                out[key] = round(2 * n / best / 1e9, 2)
            os.environ.pop("H3_HIP_DIRECT_IO", None)
            out["cache_state"] = (
                "cold: fsync + posix_fadvise(DONTNEED) before each "
                "repetition (bytes from the disk); hot: the file read once "
                "just before (page-cache resident); O_DIRECT bypasses the "
                "page cache")
        finally:
            gpu.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return out


def load_traffic(name):
    """HBM bytes per launch of the dominant kernel, measured offline with two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) and calibrated on a copy
    kernel; see profiles/.  None when no measurement is on file."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def load_counter(key):
    """A per-forward counter figure from profiles/mfma_util_wan512.json
    (written from the rocprofv3 --pmc runs of bench.py --profile-pass), or
    None when no measurement is on file."""
    path = os.path.join(ROOT, "profiles", "mfma_util_wan512.json")
    try:
        with open(path) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(seconds_budget=30.0):
    """The CPU oracle on one Wan block at BASELINE config 1 (1536 video rows,
    256 text rows, hidden 5120); returns TFLOP/s and the sample used."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    hidden, heads, ffn, rows, text = 5120, 40, 13824, 1536, 256
    rng = np.random.default_rng(0)

    def w(n, std=0.02, mean=0.0):
        return oracle.bf16((mean + std * rng.standard_normal(n,
                                                             np.float32)))
    inner = heads * 128
    wt = {"qkv": w(3 * inner * hidden), "qkv_bias": w(3 * inner),
          "q_norm": w(128, 0.02, 1.0), "k_norm": w(128, 0.02, 1.0),
          "out": w(hidden * inner), "out_bias": w(hidden),
          "norm3": w(hidden, 0.02, 1.0), "norm3_bias": w(hidden),
          "cq": w(inner * hidden), "cq_bias": w(inner),
          "ck": w(inner * hidden), "ck_bias": w(inner),
          "cv": w(inner * hidden), "cv_bias": w(inner),
          "cq_norm": w(128, 0.02, 1.0), "ck_norm": w(128, 0.02, 1.0),
          "co": w(hidden * inner), "co_bias": w(hidden),
          "fc1": w(ffn * hidden), "fc1_bias": w(ffn),
          "fc2": w(hidden * ffn), "fc2_bias": w(hidden),
          "modulation": w(6 * hidden, 0.1)}
    x = w(rows * hidden, 1.0)
    ctx = w(text * hidden, 1.0)
    cos, sin = rope_tables(wan_positions(6, 16, 16))
    t0 = time.perf_counter()
    oracle.wan_block(x, ctx, wt, np.zeros(rows, np.uint32), oracle.bf16(cos),
                     oracle.bf16(sin), rows, text, hidden, heads, ffn)
    dt = time.perf_counter() - t0
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, hidden, heads, ffn, rows,
                           text_rows=text)
    flops = h3hip.block_flops(cfg)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    return {"value": round(flops / dt / 1e12, 4), "unit": "TFLOP/s",
            "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "host_cpus": os.cpu_count(),
            "sample": (f"one Wan DiT block at BASELINE config 1 (1536 video "
                       f"+ 256 text rows, hidden 5120): {dt:.2f} s, "
                       f"{flops / 1e12:.3f} TFLOP; 50-block forward "
                       f"extrapolated {50 * dt:.0f} s")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--blocks", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-h3", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the Wan 512x512 forward and its per-class "
                         "replays (no attention sweep, 864x480 forward, H3 "
                         "shape or weight loading): the run whose rocprof "
                         "kernel averages match the line's own")
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 runs: one forward, one replay of the "
                         "plain GEMMs, one 64 Mi-element copy-like kernel of "
                         "known traffic (add_bf16) as the counter "
                         "calibration; no timing line")
    ap.add_argument("--h3-only", action="store_true",
                    help="for rocprofv3 runs: only the H3 block at its real "
                         "shape (2378 rows, 50 blocks): the forward, its "
                         "per-class replays, then add_bf16 over 64 Mi "
                         "elements as the counter calibration; prints that "
                         "section's JSON, not the bench line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend runs on one GPU; the "
                          "multi-GPU layout is a design note only "
                          "(--gpus must be 1)"}))
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py runs one process on one GPU")

    gpu = h3hip.Gpu()
    blocks = args.blocks
    if args.h3_only:
        real, _ = h3_measure(gpu, blocks, max(2, args.steps // 2), full=False)
        n = 64 << 20
        a, b, c = gpu.new_bf16(n), gpu.new_bf16(n), gpu.new_bf16(n)
        gpu.begin()
        gpu.L.h3_gpu_fill_normal_bf16(gpu.h, a, 0, n, 5, 0.0, 1.0)
        gpu.L.h3_gpu_fill_normal_bf16(gpu.h, b, 0, n, 6, 0.0, 1.0)
        gpu.check(gpu.L.h3_gpu_add_bf16(gpu.h, c, a, b, n), "calibration")
        gpu.submit()
        gpu.close()
        print(json.dumps({"h3_real_shape": real}), flush=True)
        return
    # ---- BASELINE shape: Wan block, 512x512x22f -> 6 x 32 x 32 tokens
    rows, text = 6 * 32 * 32, 512
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, 5120, 40, 13824, rows,
                           blocks=blocks, text_rows=text)
    log(f"allocating {blocks} Wan blocks ...")
    dit = h3hip.Dit(gpu, cfg)
    dit.init_random(seed=0, weight_std=0.02, mod_std=0.1)
    cos, sin = rope_tables(wan_positions(6, 32, 32))
    dit.set_rope(cos, sin)
    block_flops = dit.block_flops()
    gemm_flops = gpu.L.h3hip_dit_block_gemm_flops(
        __import__("ctypes").byref(cfg))
    attn_flops = gpu.L.h3hip_dit_block_attention_flops(
        __import__("ctypes").byref(cfg))
    if args.profile_pass:
        profile_pass(gpu, dit, blocks)
        dit.close()
        gpu.close()
        return
    log("timing ...")
    ms_step, wall_ms = time_forward(gpu, dit, blocks, args.steps, args.warmup)
    total_tflops = blocks * block_flops / (ms_step / 1e3) / 1e12
    log("per-class replays ...")
    L = gpu.L
    cref = __import__("ctypes").byref(cfg)
    plain_flops = L.h3hip_dit_block_plain_gemm_flops(cref)
    plain_launches = L.h3hip_dit_block_plain_gemm_launches(cref)
    cls = {}
    for name, mask in (("gemm_plain", OPS_GEMM), ("gemm_gelu", OPS_ACT),
                       ("context_kv", OPS_CTX),
                       ("attention", OPS_ATTN), ("row_ops", OPS_ROWS)):
        ms = class_replay(gpu, dit, blocks, mask)
        flops = L.h3hip_dit_block_class_flops(cref, mask)
        cls[name] = (ms, flops)
    gemm_ms = cls["gemm_plain"][0]
    gemm_tflops = blocks * plain_flops / (gemm_ms / 1e3) / 1e12
    per_launch_flops = plain_flops / plain_launches
    per_launch_ms = gemm_ms / (blocks * plain_launches)
    dit.close()
    log("measured MFMA peak and HBM streaming rates ...")
    peak_meas = measured_peak(gpu)
    hbm = hbm_roof(gpu)

    sweep = wan_big = loading = None
    if not args.no_extras:
        log("attention sweep and the 864x480 forward ...")
        sweep = attention_sweep(gpu)
        wan_big = wan_864x480(gpu, blocks, max(2, args.steps // 2))

    h3_real = h3_big = None
    denoise = None
    if not args.no_h3 and not args.no_extras:
        log("H3 real shape: forward + 20-step Euler denoise ...")
        h3_real, denoise = h3_measure(gpu, blocks, max(2, args.steps // 2))
        log("H3 864x480 forward ...")
        h3_big, _ = h3_measure(gpu, blocks, max(2, args.steps // 2),
                               latent_h=30, latent_w=54, full=False)

    if not args.no_extras:
        log("weight file loading ...")
        loading = weight_load()

    base = None
    if not args.no_cpu_baseline:
        log("CPU baseline ...")
        base = cpu_baseline()

    line = {
        "metric": "DiT block TFLOP/s + MFMA util %; s per 50-block forward "
                  "@512x512x22f",
        "value": round(total_tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded device-side N(0,1) latents/text, "
                "0.02 N(0,1) random-init weights)",
        "config": {"workload": "Wan-shaped DiT, 512x512x22f: 6144 video + "
                               "512 text tokens, hidden 5120, 40x128 heads, "
                               "GELU FFN 13824",
                   "blocks": blocks, "global_batch": 1, "seq_len": rows,
                   "parallelism": "single GPU"},
        "ms_per_block": round(ms_step / blocks, 3),
        "s_per_forward": round(ms_step / 1e3, 4),
        # MFMA utilisation by counter (SQ_VALU_MFMA_BUSY_CYCLES over the
        # forward, profiles/counters_wan512_profile_pass.md), and the rate
        # against the 2.5 PFLOP/s peak derived from this run's timing
        "mfma_util_pct": load_counter("forward_mfma_busy_pct"),
        "mfma_util_pct_source": "rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES / "
                                "GRBM_GUI_ACTIVE over one forward "
                                "(profiles/mfma_util_wan512.json)",
        "mfma_rate_pct_derived": round(100 * total_tflops /
                                       BF16_PEAK_TFLOPS, 1),
        "wall_ms_per_step": round(wall_ms, 3),
        "kernels": {
            name: dict(
                {"kernel": KERNEL_NAMES[name],
                 "ms_per_forward": round(ms, 3)},
                **({"tflops": round(blocks * fl / (ms / 1e3) / 1e12, 1),
                    "frac_of_peak": round(blocks * fl / (ms / 1e3) / 1e12 /
                                          BF16_PEAK_TFLOPS, 4)}
                   if fl else {}))
            for name, (ms, fl) in cls.items()},
        "roofline": {"kernel": "hk_gemm_mfma<0, false> (plain-epilogue GEMMs of "
                               "the forward)",
                     "bound": "mfma",
                     "achieved": round(per_launch_flops / (per_launch_ms /
                                                           1e3) / 1e12, 1),
                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(per_launch_flops / (per_launch_ms / 1e3) /
                                   1e12 / BF16_PEAK_TFLOPS, 4),
                     "peak_measured": round(peak_meas, 1),
                     "frac_of_measured": round(
                         per_launch_flops / (per_launch_ms / 1e3) / 1e12 /
                         peak_meas, 4),
                     "peak_measured_how": "h3_hip_mfma_loop: 4 waves per "
                                          "CU, 16 independent 32x32x16 bf16 "
                                          "MFMAs per iteration from "
                                          "registers, no LDS or memory; "
                                          "fastest of 3 x ~20 ms, HIP events",
                     "flops_per_launch": per_launch_flops,
                     "avg_launch_us": round(per_launch_ms * 1e3, 1),
                     "traffic": load_traffic("gemm_plain_wan512_traffic.json")},
        "hbm_streaming": dict(hbm, note="practical HBM rates on this GPU "
                                         "(vendor peak 8000 GB/s), for the "
                                         "row kernels' GB/s in profiles/"),
        "h3_real_shape": h3_real,
        "h3_864x480": h3_big,
        "denoise": denoise,
        "attention_sweep": sweep,
        "wan_864x480": wan_big,
        "weight_load": loading,
        "cpu_baseline": base,
    }
    gpu.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
