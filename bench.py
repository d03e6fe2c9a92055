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


def wan_positions(t, h, w):
    """(t, h, w) integer grid of the video tokens, row-major."""
    tt, hh, ww = np.meshgrid(np.arange(t), np.arange(h), np.arange(w),
                             indexing="ij")
    pos = np.stack([tt.ravel(), hh.ravel(), ww.ravel()], axis=1)
    return pos.astype(np.float64)


def rope_tables(positions):
    L = h3hip.lib()
    rows = positions.shape[0]
    inv = np.empty(16, np.float32)
    L.h3hip_default_inv_freq(h3hip.ptr(inv))
    pos = np.ascontiguousarray(positions, dtype=np.float64)
    cos = np.empty(rows * 48, np.float32)
    sin = np.empty(rows * 48, np.float32)
    L.h3hip_rope_tables(h3hip.ptr(pos), rows, h3hip.ptr(inv), 1.0,
                        h3hip.ptr(cos), h3hip.ptr(sin))
    return cos, sin


def h3_layout_rows(text_len, latent_t, latent_h, latent_w, audio_t):
    """Packed H3 sequence (text, audio, video) with its positions and the
    step-0 row map of the serving schedule."""
    L = h3hip.lib()
    lay = h3hip.Layout()
    err = __import__("ctypes").create_string_buffer(256)
    ok = L.h3hip_layout_build(text_len, latent_t, latent_h, latent_w, audio_t,
                              22, None, 0, None, 0,
                              __import__("ctypes").byref(lay), err, 256)
    if not ok:
        raise RuntimeError(err.value.decode())
    n = lay.seq_len
    pos = np.array([[lay.positions[i].t, lay.positions[i].h,
                     lay.positions[i].w] for i in range(n)])
    segs = [(lay.segments[i].start, lay.segments[i].stop,
             lay.segments[i].kind) for i in range(lay.segment_count)]
    L.h3hip_layout_free(__import__("ctypes").byref(lay))
    row_map = np.zeros(n, np.uint32)
    for start, stop, kind in segs:       # video row 0 / audio row 1 at step 0
        row_map[start:stop] = {0: 1, 4: 1 * 3 + 2, 5: 0}.get(kind, 0)
    return n, pos, row_map


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


def op_profile(gpu, dit, blocks):
    """One forward with per-op HIP-event timing; {op: (count, ms)}."""
    import ctypes as C
    L = gpu.L
    L.h3_hip_op_timing_enable(gpu.h, 1)
    L.h3_hip_op_timing_reset(gpu.h)
    dit.run_blocks(0, blocks)
    names = C.create_string_buffer(4096)
    L.h3_hip_op_timing_names(gpu.h, names, 4096)
    out = {}
    for name in names.value.decode().split():
        n, ms = C.c_uint64(), C.c_double()
        L.h3_hip_op_timing_read(gpu.h, name.encode(), C.byref(n), C.byref(ms))
        out[name] = (n.value, ms.value)
    L.h3_hip_op_timing_enable(gpu.h, 0)
    L.h3_hip_op_timing_reset(gpu.h)
    return out


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
            "cores": threads, "kind": "port",
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
    log("timing ...")
    ms_step, wall_ms = time_forward(gpu, dit, blocks, args.steps, args.warmup)
    prof = op_profile(gpu, dit, blocks)
    total_tflops = blocks * block_flops / (ms_step / 1e3) / 1e12
    gemm_n = sum(v[0] for k, v in prof.items() if k.startswith("gemm"))
    gemm_ms = sum(v[1] for k, v in prof.items() if k.startswith("gemm"))
    attn_ms = sum(v[1] for k, v in prof.items() if k.startswith("attention"))
    attn_n = sum(v[0] for k, v in prof.items() if k.startswith("attention"))
    gemm_tflops = blocks * gemm_flops / (gemm_ms / 1e3) / 1e12
    attn_tflops = blocks * attn_flops / (attn_ms / 1e3) / 1e12
    dit.close()

    h3_real = None
    if not args.no_h3:
        n, pos, row_map = h3_layout_rows(512, 7, 32, 32, 37)
        hcfg = h3hip.dit_config(h3hip.FAMILY_H3, 5376, 56, 14336, n,
                                blocks=blocks, time_rows=2)
        hdit = h3hip.Dit(gpu, hcfg)
        hdit.init_random(seed=1, weight_std=0.02, mod_std=0.1)
        hc, hs = rope_tables(pos)
        hdit.set_rope(hc, hs)
        hdit.set_row_map(row_map)
        hms, _ = time_forward(gpu, hdit, blocks, max(2, args.steps // 2), 1)
        hflops = hdit.block_flops()
        h3_real = {"rows": int(n), "s_per_forward": round(hms / 1e3, 4),
                   "ms_per_block": round(hms / blocks, 3),
                   "tflops": round(blocks * hflops / (hms / 1e3) / 1e12, 1)}
        hdit.close()

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
        "mfma_util_pct": round(100 * total_tflops / BF16_PEAK_TFLOPS, 1),
        "wall_ms_per_step": round(wall_ms, 3),
        "kernels": {
            "gemm": {"tflops": round(gemm_tflops, 1),
                     "frac_of_peak": round(gemm_tflops / BF16_PEAK_TFLOPS, 4),
                     "launches": gemm_n, "ms": round(gemm_ms, 3)},
            "attention": {"tflops": round(attn_tflops, 1),
                          "frac_of_peak": round(attn_tflops /
                                                BF16_PEAK_TFLOPS, 4),
                          "launches": attn_n, "ms": round(attn_ms, 3)},
            "ops_ms": {k: round(v[1], 3) for k, v in sorted(prof.items())},
        },
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 1),
                     "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
        "h3_real_shape": h3_real,
        "cpu_baseline": base,
    }
    gpu.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
