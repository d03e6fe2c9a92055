"""Where the MFMA GEMM's time goes, tile by tile.

Runs one launch of hk_gemm_mfma<0> per shape on the phase-trace build
(`make -C h3.c_amd trace` -> lib/libh3_gpu_hip_trace.so, the same kernels
with per-tile timestamps; see HK_GEMM_TRACE in csrc/hk_gemm.hip) and prints,
per round of tiles, the average time of each phase of a tile over the
workgroups:

  prologue   tile start -> first K stage landed in LDS (the wait also
             covers the previous tile's stores still in flight)
  main       the K loop
  bias       bias loads + barrier before staging
  stage      accumulators -> bf16 -> LDS, barrier
  store      LDS -> global stores issued
  drain      last LDS reads + barrier

and the shader clock over the tile (shader-clock ticks / real-time ticks).
The launch's own duration, from HIP events around an untraced launch of the
product library in a separate process, is printed by bench.py; here the
traced launch is timed the same way for reference.

    python3 h3.c_amd/gemm_phase_trace.py [--shapes qkv,out,down] [--cold]
"""
import argparse
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import h3hip  # noqa: E402

SHAPES = {  # name: (M, K, N); the Wan block at 512x512x22f
    "qkv": (6144, 5120, 15360),
    "out": (6144, 5120, 5120),
    "down": (6144, 13824, 5120),
    "up": (6144, 5120, 13824),
    # the H3 block at its real shape (2378 rows, hidden 5376, SwiGLU 14336)
    "h3out": (2378, 5376, 5376),
    "h3fc2": (2378, 14336, 5376),
}
WG, ITERS, SLOTS = 1024, 16, 12
PHASES = (("prologue", 0, 1), ("main", 1, 2), ("bias", 2, 3),
          ("stage", 3, 4), ("store", 4, 5), ("drain", 5, 6))


def trace_shape(gpu, L, name, m, k, n, out_dir=None, cold=False):
    # cold: X and W in enough copies to pass 700 MB, more than the 256 MB
    # Infinity Cache holds, and the traced launch reads the copy used
    # longest ago, as the forward reads every block's own weights
    copies = max(2, int(700e6 // ((m * k + n * k) * 2)) + 1) if cold else 1
    xs = [gpu.new_bf16(m * k) for _ in range(copies)]
    ws = [gpu.new_bf16(n * k) for _ in range(copies)]
    o, b = gpu.new_bf16(m * n), gpu.new_bf16(n)
    gpu.begin()
    for i in range(copies):
        L.h3_gpu_fill_normal_bf16(gpu.h, xs[i], 0, m * k, 1 + 10 * i, 0.0,
                                  1.0)
        L.h3_gpu_fill_normal_bf16(gpu.h, ws[i], 0, n * k, 2 + 10 * i, 0.0,
                                  0.02)
    L.h3_gpu_fill_normal_bf16(gpu.h, b, 0, n, 3, 0.0, 0.02)
    gpu.submit()
    sel = [0]

    def launch():
        i = sel[0] % copies
        sel[0] += 1
        gpu.check(L.h3_gpu_linear_bf16(gpu.h, o, xs[i], ws[i], b, m, k, n),
                  name)

    gpu.begin()
    for _ in range(3 * copies):
        launch()
    gpu.submit()
    if not L.h3_hip_gemm_trace_clear():
        raise RuntimeError("trace clear failed")
    gpu.begin()
    L.h3_hip_marker(gpu.h, 0)
    launch()
    L.h3_hip_marker(gpu.h, 1)
    gpu.submit()
    ms = C.c_double()
    L.h3_hip_marker_elapsed(gpu.h, 0, 1, C.byref(ms))
    tr = np.zeros(WG * ITERS * SLOTS, np.uint64)
    if not L.h3_hip_gemm_trace_read(tr.ctypes.data_as(C.c_void_p), tr.size):
        raise RuntimeError("trace read failed")
    for t in xs + ws + [o, b]:
        gpu.free(t)
    tr = tr.reshape(WG, ITERS, SLOTS).astype(np.int64)
    live = tr[:, :, 6] != 0
    t0 = tr[:, :, 0][live].min()
    tiles = ((m + 255) // 256) * ((n + 255) // 256)
    print(f"\n{name}{' (cold operands, %d copies)' % copies if cold else ''}: "
          f"M={m} K={k} N={n}, {tiles} tiles, "
          f"{int(live[:, 0].sum())} workgroups; traced launch "
          f"{ms.value * 1e3:.1f} us (event), first tile start to last tile "
          f"end {(tr[:, :, 6][live].max() - t0) / 100.0:.1f} us")
    print("round  tiles  start(min..max us)  " +
          "  ".join(f"{p:>8}" for p, _, _ in PHASES) +
          "    tile_us  clock_GHz  end(max us)")
    totals = {p: 0.0 for p, _, _ in PHASES}
    for r in range(ITERS):
        sel = live[:, r]
        if not sel.any():
            break
        row = tr[sel, r, :]
        start = (row[:, 0] - t0) / 100.0
        cells = []
        for p, a, bb in PHASES:
            d = (row[:, bb] - row[:, a]).mean() / 100.0
            totals[p] += d
            cells.append(f"{d:8.2f}")
        tile = (row[:, 6] - row[:, 0]).mean() / 100.0
        clk = ((row[:, 9] - row[:, 8]) /
               np.maximum(row[:, 6] - row[:, 0], 1)).mean() * 0.1
        end = (row[:, 6].max() - t0) / 100.0
        print(f"{r:5d}  {int(sel.sum()):5d}  {start.min():7.1f}..{start.max():7.1f}"
              f"       " + "  ".join(cells) +
              f"    {tile:7.2f}  {clk:9.3f}  {end:10.1f}")
    kst = k // 64
    main_cyc = ((tr[:, :, 2] - tr[:, :, 1]) *
                (tr[:, :, 9] - tr[:, :, 8]) /
                np.maximum(tr[:, :, 6] - tr[:, :, 0], 1))[live]
    stalls = tr[:, :, 10][live].any()
    print(f"K loop, wave 0, per 64-deep stage: "
          f"{main_cyc.mean() / kst:.0f} shader cycles (2048 = its MFMAs "
          f"alone)" + (f", of which {tr[:, :, 10][live].mean() / kst:.0f} "
                       f"waiting at the stage's loads + barrier and "
                       f"{tr[:, :, 11][live].mean() / kst:.0f} for "
                       f"fragment reads" if stalls else ""))
    tot = sum(totals.values())
    print("share of tile time: " + ", ".join(
        f"{p} {100 * v / tot:.1f}%" for p, v in totals.items()))
    # workgroups are dealt round-robin to the 8 XCDs (blockIdx % 8)
    wg = np.nonzero(live[:, 0])[0]
    fin = np.array([(tr[i, :, 6][live[i]].max() - t0) / 100.0 for i in wg])
    busy = np.array([((tr[i, :, 6] - tr[i, :, 0])[live[i]]).sum() / 100.0
                     for i in wg])
    clk = np.array([(((tr[i, :, 9] - tr[i, :, 8]) /
                      np.maximum(tr[i, :, 6] - tr[i, :, 0], 1))[live[i]])
                    .mean() * 0.1 for i in wg])
    print("xcd  workgroups  finish_us(mean/max)  busy_us(mean)  clock_GHz")
    for x in range(8):
        sel = (wg % 8) == x
        if sel.any():
            print(f"{x:3d}  {int(sel.sum()):10d}  {fin[sel].mean():9.1f}/"
                  f"{fin[sel].max():7.1f}  {busy[sel].mean():13.1f}  "
                  f"{clk[sel].mean():9.3f}")
    if out_dir:
        np.save(os.path.join(out_dir, f"gemm_trace_{name}.npy"), tr)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default="qkv,out,down")
    ap.add_argument("--cold", action="store_true",
                    help="rotate X and W over copies larger than the "
                         "Infinity Cache (the forward's case)")
    ap.add_argument("--save", default=None,
                    help="directory for the raw traces (.npy)")
    args = ap.parse_args()
    h3hip.LIB_PATH = os.path.join(HERE, "lib", "libh3_gpu_hip_trace.so")
    L = h3hip.lib()
    gpu = h3hip.Gpu()
    try:
        for name in args.shapes.split(","):
            trace_shape(gpu, L, name, *SHAPES[name], out_dir=args.save,
                        cold=args.cold)
    finally:
        gpu.close()


if __name__ == "__main__":
    main()
