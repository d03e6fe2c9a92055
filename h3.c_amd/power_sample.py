"""Package power and per-XCD shader clocks while one kernel runs back to
back for a few seconds: the MFMA-only loop (h3_hip_mfma_loop), the Wan QKV
GEMM (6144 x 5120 -> 15360, bias) and 6144-row self-attention (40 heads x
128).  `amd-smi metric -p -c` is sampled every 0.3 s from a second thread;
the first two and the last sample of each kernel are dropped (ramp).
With --cold the GEMM cycles through copies of X and W larger than the
256 MB Infinity Cache, as the forward reads every block's own weights.

    python3 h3.c_amd/power_sample.py [--cold]
"""
import csv
import ctypes as C
import io
import os
import subprocess
import sys
import threading
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import h3hip  # noqa: E402


def amd_smi():
    return subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0",
                           "--csv"], capture_output=True, text=True,
                          timeout=10).stdout


def run_for(gpu, label, launch, flops, seconds=4.0, batch=20):
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            samples.append(amd_smi())
            time.sleep(0.3)
    th = threading.Thread(target=sampler)
    th.start()
    t0, n = time.time(), 0
    while time.time() - t0 < seconds:
        gpu.begin()
        for _ in range(batch):
            gpu.check(launch(), label)
        gpu.submit()
        n += batch
    stop.set()
    th.join()
    dt = time.time() - t0
    print(f"== {label}: {n} launches in {dt:.2f} s, {dt / n * 1e6:.1f} us "
          f"each, {flops * n / dt / 1e12:.0f} TFLOP/s", flush=True)
    watts = []
    for out in samples[2:-1]:
        r = next(csv.DictReader(io.StringIO(out)), {})
        clk = [r.get(f"gfx_{i}_clk") for i in range(8)]
        print(f"  socket power {r.get('socket_power')} W, XCD clocks (MHz) "
              f"{' '.join(str(c) for c in clk)}", flush=True)
        try:
            watts.append(float(r.get("socket_power")))
        except (TypeError, ValueError):
            pass
    if watts:
        w = sum(watts) / len(watts)
        print(f"  mean {w:.0f} W: {w * dt / n:.3f} J per launch, "
              f"{w / (flops * n / dt) * 1e12:.2f} pJ per flop", flush=True)


def main():
    cold = "--cold" in sys.argv[1:]
    gpu = h3hip.Gpu()
    L = gpu.L
    try:
        m, k, n = 6144, 5120, 15360
        copies = 4 if cold else 1   # 4 x 220 MB of X and W
        xs = [gpu.new_bf16(m * k) for _ in range(copies)]
        ws = [gpu.new_bf16(n * k) for _ in range(copies)]
        o, b = gpu.new_bf16(m * n), gpu.new_bf16(n)
        rows, heads = 6144, 40
        q, kk, v, oo = (gpu.new_bf16(rows * heads * 128) for _ in range(4))
        gpu.begin()
        for i in range(copies):
            L.h3_gpu_fill_normal_bf16(gpu.h, xs[i], 0, m * k, 1 + 10 * i,
                                      0.0, 1.0)
            L.h3_gpu_fill_normal_bf16(gpu.h, ws[i], 0, n * k, 2 + 10 * i,
                                      0.0, 0.02)
        L.h3_gpu_fill_normal_bf16(gpu.h, b, 0, n, 3, 0.0, 0.02)
        for t, seed in ((q, 5), (kk, 6), (v, 7)):
            L.h3_gpu_fill_normal_bf16(gpu.h, t, 0, rows * heads * 128, seed,
                                      0.0, 1.0)
        gpu.submit()
        sink = gpu.new_f32(1024 * 256)
        fl = C.c_double()
        print(f"  idle socket power: "
              f"{next(csv.DictReader(io.StringIO(amd_smi())), {}).get('socket_power')} W",
              flush=True)
        gpu.run("h3_hip_mfma_loop", sink, 1, C.byref(fl))  # flops of one
        per_iteration = fl.value
        run_for(gpu, "MFMA-only loop (h3_hip_mfma_loop)",
                lambda: L.h3_hip_mfma_loop(gpu.h, sink, 20000, C.byref(fl)),
                per_iteration * 20000)
        turn = [0]

        def gemm():
            i = turn[0] % copies
            turn[0] += 1
            return L.h3_gpu_linear_bf16(gpu.h, o, xs[i], ws[i], b, m, k, n)
        run_for(gpu, "QKV GEMM 6144x5120->15360 (hk_gemm_mfma<0>)"
                + (f", X and W cycling over {copies} copies" if cold else ""),
                gemm, 2.0 * m * n * k)
        run_for(gpu, "self-attention 6144 rows, 40 heads (hk_flash_fwd)",
                lambda: L.h3_gpu_sdpa_bf16(gpu.h, oo, q, kk, v, rows, heads,
                                           128, C.c_float(128 ** -0.5)),
                4.0 * rows * rows * heads * 128)
    finally:
        gpu.close()


if __name__ == "__main__":
    main()
