"""Per-op parity of the HIP backend against the CPU oracle, through the C ABI.

Mirrors the reference's synthetic op tests (tests/test_cuda_dit.c,
tests/test_cuda_attention.c, tests/test_cuda_core.c): seeded inputs, an
independent CPU statement of each op, and the reference's tolerances --
bit-exact or one bf16 ulp for the row/elementwise ops, 1e-3 abs + 1e-2 rel
for GEMM and flash attention.
"""
import ctypes as C
import math

import numpy as np
import pytest

from conftest import (adaln_terms, assert_close, assert_row_close,
                      sdpa_p_rounding_bound,
                      assert_ulp, bf16_ulp_distance, rand_bf16, to_f32)

pytestmark = pytest.mark.gpu

import oracle  # noqa: E402


def _mod_setup(rng, rows, width, slots=6, mod_rows=4):
    mod = rand_bf16(rng, mod_rows * slots * width, 0.5)
    row_map = rng.integers(0, mod_rows, rows).astype(np.uint32)
    return mod, row_map


# ------------------------------------------------------------------ GEMM

@pytest.mark.parametrize("m,k,n,bias,mlp", [
    (4096, 1024, 8192, True, False),   # 512 tiles: two full rounds
    (2378, 1024, 5376, False, False),  # H3 rows: 210 tiles, bands of 8 + 2
    (2378, 512, 4608, False, True),    # MLP: fc1 with the SwiGLU epilogue
])
def test_linear_repeats_bit_exactly(gpu, m, k, n, bias, mlp):
    """The K loop keeps its two L2 prefetch loads in flight across the
    stage wait (vmcnt(2)), relying on loads retiring in issue order.  A
    stage read before its loads landed would show as results that change
    from run to run: the first run matches the oracle, and four more, each
    after an unrelated GEMM over other buffers, match it bit for bit.  For
    the MLP, n is the FFN width (fc1 has 2 n rows, fc2 brings it back to
    k)."""
    rng = np.random.default_rng(m + k + n)
    x = rand_bf16(rng, m * k)
    w = rand_bf16(rng, (2 * n if mlp else n) * k, 0.05)
    w2 = rand_bf16(rng, k * n, 0.05) if mlp else None
    b = rand_bf16(rng, n, 0.1) if bias else None
    tx, tw = gpu.bf16(x), gpu.bf16(w)
    tw2 = gpu.bf16(w2) if mlp else None
    tb = gpu.bf16(b) if bias else None
    to = gpu.new_bf16(m * (k if mlp else n))
    om, ok_, on = 2048, 2048, 8192
    ox = gpu.bf16(rand_bf16(rng, om * ok_))
    ow = gpu.bf16(rand_bf16(rng, on * ok_, 0.05))
    oo = gpu.new_bf16(om * on)

    def run():
        if mlp:
            gpu.run("h3_gpu_mlp_bf16", to, tx, tw, tw2, m, k, n, k)
        else:
            gpu.run("h3_gpu_linear_bf16", to, tx, tw, tb, m, k, n)
        return gpu.read_bf16(to)

    first = run()
    if mlp:
        want = oracle.mlp(x, w, w2, m, k, n)
        assert_close(first, want, what=f"MLP {m}x{k}x{n}", chained=1)
    else:
        want = oracle.linear(x, w, b, m, k, n)
        assert_close(first, want, what=f"linear {m}x{k}x{n}")
    for rep in range(4):
        gpu.run("h3_gpu_linear_bf16", oo, ox, ow, None, om, ok_, on)
        again = run()
        assert np.array_equal(again, first), f"repeat {rep + 1} differs"


@pytest.mark.parametrize("m,k,n,bias", [
    (32, 256, 256, False),      # reference test_cuda_core.c linear shape
    (100, 512, 768, True),      # ragged M
    (1, 256, 512, False),       # single row
    (300, 5376, 1024, False),   # real K (hidden); split-K (8 tiles)
    (257, 1024, 1280, True),    # M just past a tile; split-K in 2
    (64, 96, 256, True),        # K % 64 != 0 -> sequential fallback kernel
    (39, 2688, 4100, True),     # skinny path: time rows x modulation width
    (64, 128, 68, False),       # skinny path: full 64-row tile, ragged N
    (1, 64, 300, True),         # skinny, one row, one K step
    (32, 384, 132, False),      # skinny, 32 rows, 6 K steps (ring of 4)
    (17, 320, 1000, True),      # skinny, 5 K steps, ragged N
    (33, 64, 4, True),          # skinny, one row in the second half, N = 4
    (64, 2688, 96, False),      # skinny, all 64 rows, real K, one wave of N
    (65, 192, 256, False),      # one row past the skinny limit
    (512, 5120, 5120, True),    # split-K: Wan cross K/V projection (40 tiles)
    (260, 2048, 516, True),     # split-K, ragged M and N, 4 splits
    (600, 1088, 256, False),    # split-K with a short last split (17 steps)
    (4096, 512, 4352, True),    # 272 tiles: one full round + a split tail
    (4100, 256, 4200, True),    # 289 tiles, full round with ragged M and N
    (300, 64, 520, True),       # one K stage: loads and prefetch clamp to it
    (2378, 128, 1000, False),   # two K stages, H3 rows, ragged N
])
def test_linear_bf16(gpu, m, k, n, bias):
    rng = np.random.default_rng(m * 7 + k + n)
    x = rand_bf16(rng, m * k)
    w = rand_bf16(rng, n * k, 0.05)
    b = rand_bf16(rng, n, 0.1) if bias else None
    want = oracle.linear(x, w, b, m, k, n)
    tx, tw, to = gpu.bf16(x), gpu.bf16(w), gpu.new_bf16(m * n)
    tb = gpu.bf16(b) if bias else None
    gpu.run("h3_gpu_linear_bf16", to, tx, tw, tb, m, k, n)
    got = gpu.read_bf16(to)
    assert_close(got, want, what=f"linear {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n,bias", [
    (512, 5120, 5120, True),    # the Wan cross K/V shape: one paired launch
    (77, 512, 640, False),      # 3 + 3 tiles, 8 K steps, ragged M and N
    (600, 1088, 256, True),     # ragged M, a short last split
    (4096, 512, 4352, True),    # too many tiles to pair: two linears
])
def test_linear_pair(gpu, m, k, n, bias):
    """h3_hip_linear_pair_bf16: each output as h3_gpu_linear_bf16 would give
    it, against the oracle, whether the two share one split-K launch or
    not."""
    rng = np.random.default_rng(m + 3 * k + n)
    x = rand_bf16(rng, m * k)
    w0, w1 = rand_bf16(rng, n * k, 0.05), rand_bf16(rng, n * k, 0.05)
    b0 = rand_bf16(rng, n, 0.1) if bias else None
    b1 = rand_bf16(rng, n, 0.1) if bias else None
    o0, o1 = gpu.new_bf16(m * n), gpu.new_bf16(m * n)
    gpu.run("h3_hip_linear_pair_bf16", o0, o1, gpu.bf16(x), gpu.bf16(w0),
            gpu.bf16(b0) if bias else None, gpu.bf16(w1),
            gpu.bf16(b1) if bias else None, m, k, n)
    assert_close(gpu.read_bf16(o0), oracle.linear(x, w0, b0, m, k, n),
                 what=f"pair[0] {m}x{k}x{n}")
    assert_close(gpu.read_bf16(o1), oracle.linear(x, w1, b1, m, k, n),
                 what=f"pair[1] {m}x{k}x{n}")
    with pytest.raises(RuntimeError, match="distinct"):
        gpu.run("h3_hip_linear_pair_bf16", o0, o0, gpu.bf16(x), gpu.bf16(w0),
                None, gpu.bf16(w1), None, m, k, n)


@pytest.mark.parametrize("m,k,n,count,first,exact", [
    (300, 256, 512, 5, 0, True),     # 4 K steps: the single linear is
                                     # data-parallel too, so bit for bit
    (512, 5120, 1024, 6, 2, False),  # the Wan text shape (narrower), from
                                     # problem 2 of the table
    (77, 512, 640, 3, 1, False),     # ragged M and N
])
def test_linear_group(gpu, m, k, n, count, first, exact):
    """h3_hip_linear_group_bf16 runs problems [first, first + count) of a
    table in one launch: each output against the oracle, and where
    h3_gpu_linear_bf16 is also data-parallel, equal to it bit for bit;
    problems outside the range are left alone."""
    rng = np.random.default_rng(m + k + n + count)
    total = first + count
    x = rand_bf16(rng, m * k)
    ws = [rand_bf16(rng, n * k, 0.05) for _ in range(total)]
    bs = [rand_bf16(rng, n, 0.1) if p % 2 == 0 else None for p in range(total)]
    tx = gpu.bf16(x)
    tws = [gpu.bf16(w) for w in ws]
    tbs = [gpu.bf16(b) if b is not None else None for b in bs]
    tos = [gpu.new_bf16(m * n) for _ in range(total)]
    for t in tos:
        gpu.run("h3_gpu_fill_normal_bf16", t, 0, m * n, 9, 0.0, 1.0)
    before = [gpu.read_bf16(t).view(np.uint16).copy() for t in tos]
    P = C.c_void_p
    outs = (P * total)(*[t for t in tos])
    wts = (P * total)(*[t for t in tws])
    bis = (P * total)(*[t for t in tbs])
    table = gpu.L.h3_hip_linear_group_table(gpu.h, outs, wts, bis, total, m,
                                            k, n)
    assert table, gpu.error()
    try:
        gpu.run("h3_hip_linear_group_bf16", table, first, count, tx, m, k, n)
        for p in range(total):
            got = gpu.read_bf16(tos[p])
            if p < first:
                assert np.array_equal(got.view(np.uint16), before[p])
                continue
            assert_close(got, oracle.linear(x, ws[p], bs[p], m, k, n),
                         what=f"group[{p}] {m}x{k}x{n}")
            if exact:
                one = gpu.new_bf16(m * n)
                gpu.run("h3_gpu_linear_bf16", one, tx, tws[p], tbs[p], m, k,
                        n)
                assert np.array_equal(gpu.read_bf16(one).view(np.uint16),
                                      got.view(np.uint16))
    finally:
        gpu.L.h3_gpu_tensor_free(table)


def test_linear_group_rejects_another_shape(gpu):
    """The table's addresses were validated for the shape it was built with:
    a launch with more rows, another width, problems past the table's count
    or a tensor that is not a table fails before any kernel runs, and the
    outputs are left alone."""
    m, k, n = 128, 256, 256
    rng = np.random.default_rng(31)
    tx = gpu.bf16(rand_bf16(rng, 2 * m * 2 * k))
    tws = [gpu.bf16(rand_bf16(rng, n * k, 0.05)) for _ in range(2)]
    tos = [gpu.new_bf16(m * n) for _ in range(2)]
    for t in tos:
        gpu.run("h3_gpu_fill_normal_bf16", t, 0, m * n, 3, 0.0, 1.0)
    before = [gpu.read_bf16(t).view(np.uint16).copy() for t in tos]
    P = C.c_void_p
    table = gpu.L.h3_hip_linear_group_table(
        gpu.h, (P * 2)(*tos), (P * 2)(*tws), None, 2, m, k, n)
    assert table, gpu.error()
    plain = gpu.L.h3_gpu_tensor_from_u32(
        gpu.h, np.zeros(12, np.uint32).ctypes.data_as(P), 12)
    assert plain, gpu.error()
    try:
        for args, what in (((0, 2, tx, 2 * m, k, n), "differs"),
                           ((0, 2, tx, m, 2 * k, n), "differs"),
                           ((0, 2, tx, m, k, 2 * n), "differs"),
                           ((1, 2, tx, m, k, n), "past the"),
                           ((0, 2, tx, m, k, n), "not built")):
            tab = plain if what == "not built" else table
            with pytest.raises(RuntimeError, match=what):
                gpu.run("h3_hip_linear_group_bf16", tab, *args)
        for t, old in zip(tos, before):
            assert np.array_equal(gpu.read_bf16(t).view(np.uint16), old)
        gpu.run("h3_hip_linear_group_bf16", table, 0, 2, tx, m, k, n)
    finally:
        gpu.L.h3_gpu_tensor_free(table)
        gpu.L.h3_gpu_tensor_free(plain)


def test_head_norm_group_matches_per_tensor(gpu):
    """h3_hip_head_rms_norm_group_bf16 normalises problems [first, first +
    count) of a table in one launch, each bit-identical to
    h3_gpu_head_rms_norm_bf16 on that tensor with its own weight and
    against the oracle; problems outside the range are left alone; another
    shape or a range past the table fails."""
    rows, heads, hd, total, first, count = 77, 5, 128, 5, 1, 3
    rng = np.random.default_rng(91)
    xs = [rand_bf16(rng, rows * heads * hd) for _ in range(total)]
    ws = [rand_bf16(rng, hd, 0.3) for _ in range(total)]
    tg = [gpu.bf16(x) for x in xs]
    tr = [gpu.bf16(x) for x in xs]
    tw = [gpu.bf16(w) for w in ws]
    P = C.c_void_p
    table = gpu.L.h3_hip_head_norm_group_table(
        gpu.h, (P * total)(*tg), (P * total)(*tw), total, rows, heads, hd)
    assert table, gpu.error()
    try:
        gpu.run("h3_hip_head_rms_norm_group_bf16", table, first, count, rows,
                heads, hd, 1e-6)
        for p in range(total):
            got = gpu.read_bf16(tg[p]).view(np.uint16)
            if not first <= p < first + count:
                assert np.array_equal(got, xs[p].view(np.uint16))
                continue
            gpu.run("h3_gpu_head_rms_norm_bf16", tr[p], tw[p], rows, heads,
                    hd, 1e-6)
            assert np.array_equal(got,
                                  gpu.read_bf16(tr[p]).view(np.uint16))
            want = oracle.head_rms_norm(xs[p], ws[p], rows, heads, hd, 1e-6)
            assert_close(gpu.read_bf16(tg[p]), want, what=f"group norm {p}")
        for args, what in (((0, 2, rows + 1, heads, hd), "differs"),
                           ((0, 2, rows, heads + 1, hd), "differs"),
                           ((4, 2, rows, heads, hd), "past the")):
            with pytest.raises(RuntimeError, match=what):
                gpu.run("h3_hip_head_rms_norm_group_bf16", table, *args,
                        1e-6)
    finally:
        gpu.L.h3_gpu_tensor_free(table)


def test_mfma_loop_measures_a_plausible_rate(gpu):
    """h3_hip_mfma_loop (the bench's measured MFMA ceiling): the sums are
    exact small multiples of 2^-14, so two iterations give exactly twice
    one iteration's sums; the FLOP count it reports over the event time is
    a rate between 20% and 120% of the 2.5 PFLOP/s bf16 peak."""
    # room for up to 1024 CUs; entries of CUs the GPU lacks stay 0
    sink = gpu.f32(np.zeros(1024 * 256, np.float32))
    flops = C.c_double()
    got = []
    for it in (1, 2):
        gpu.run("h3_hip_mfma_loop", sink, it, C.byref(flops))
        got.append(gpu.read_f32(sink))
    assert np.isfinite(got[0]).all() and (got[0] >= 0).all()
    assert got[0].max() > 0
    np.testing.assert_array_equal(got[1], 2 * got[0])
    gpu.begin()
    gpu.L.h3_hip_marker(gpu.h, 0)
    assert gpu.L.h3_hip_mfma_loop(gpu.h, sink, 20000, C.byref(flops))
    gpu.L.h3_hip_marker(gpu.h, 1)
    gpu.submit()
    ms = C.c_double()
    assert gpu.L.h3_hip_marker_elapsed(gpu.h, 0, 1, C.byref(ms))
    tflops = flops.value / (ms.value * 1e-3) / 1e12
    assert 500 < tflops < 3000, tflops


def test_linear_stats_kind(gpu):
    """Routing-shape rule of the stats counters (reference
    h3_cuda_core.cu:838-841): rows >= 32, in >= 256, out >= 256 -> kind 1."""
    rng = np.random.default_rng(1)
    before = gpu.stats().mps_linear_dispatches
    x, w = gpu.bf16(rand_bf16(rng, 32 * 256)), gpu.bf16(rand_bf16(rng, 256 * 256))
    gpu.run("h3_gpu_linear_bf16", gpu.new_bf16(32 * 256), x, w, None, 32, 256,
            256)
    assert gpu.stats().mps_linear_dispatches == before + 1


@pytest.mark.parametrize("rows,d,ffn", [
    (64, 256, 512),       # 4 SwiGLU tiles, too few K steps to split
    (300, 1024, 1536),    # 24 tiles, cut along K (SwiGLU split-K reduce)
    (130, 5376, 512),     # 4 tiles at the real hidden size, 21 splits
    (300, 512, 4608),     # 72 tiles, 2 splits
    (300, 512, 17408),    # 272 tiles: one full round + a 16-tile split tail
])
def test_mlp_swiglu(gpu, rows, d, ffn):
    rng = np.random.default_rng(rows + d + ffn)
    x = rand_bf16(rng, rows * d)
    fc1 = rand_bf16(rng, 2 * ffn * d, 0.04)
    fc2 = rand_bf16(rng, d * ffn, 0.04)
    want = oracle.mlp(x, fc1, fc2, rows, d, ffn)
    out = gpu.new_bf16(rows * d)
    gpu.run("h3_gpu_mlp_bf16", out, gpu.bf16(x), gpu.bf16(fc1), gpu.bf16(fc2),
            rows, d, ffn, d)
    assert_close(gpu.read_bf16(out), want, what="SwiGLU MLP", chained=1)


def test_linear_gelu_full_round_and_split_tail(gpu):
    """272 tiles on 256 CUs: the first 256 run whole, the last 16 are cut
    along K and reduced with the bias and GELU."""
    m, k, n = 4096, 640, 4352
    rng = np.random.default_rng(17)
    x = rand_bf16(rng, m * k)
    w = rand_bf16(rng, n * k, 0.05)
    b = rand_bf16(rng, n, 0.1)
    want = oracle.gelu(oracle.linear(x, w, b, m, k, n))
    out = gpu.new_bf16(m * n)
    gpu.run("h3_gpu_linear_gelu_bf16", out, gpu.bf16(x), gpu.bf16(w),
            gpu.bf16(b), m, k, n)
    assert_close(gpu.read_bf16(out), want, what="linear+GELU", chained=1)


@pytest.mark.parametrize("k", [64, 512])
def test_linear_gelu_activation_exact(gpu, k):
    """The GEMM's GELU epilogue on its own: an identity weight makes the
    linear output exactly x, so the result must be oracle.gelu(x) over
    -12..12, the +-10 saturation of u included.  K = 64 runs the full-tile
    epilogue; K = 512 cuts the 16 tiles along K, so the split-K reduction
    applies the activation.

    Bound: one bf16 ulp, or an absolute |x| 2^-21.  For u below about -8.7
    the reference's own f32 value 0.5 x (1 + tanhf(u)) is a multiple of
    0.5 |x| 2^-24 (tanhf rounds next to -1), so there it is exact only to
    that absolute error, and ulps of a value that small mean nothing."""
    m, n = 4096, 64
    rng = np.random.default_rng(k)
    vals = oracle.bf16(np.concatenate([
        rng.uniform(-12, 12, m * n - 8),
        [0.0, -0.0, 1e-30, -1e-30, 5.6, -5.6, 11.0, -11.0]]).astype(
            np.float32))
    x = np.zeros((m, k), np.uint16)
    x[:, :n] = vals.reshape(m, n)
    w = np.zeros((n, k), np.uint16)
    w[np.arange(n), np.arange(n)] = 0x3F80            # 1.0
    out = gpu.new_bf16(m * n)
    gpu.run("h3_gpu_linear_gelu_bf16", out, gpu.bf16(x.ravel()),
            gpu.bf16(w.ravel()), None, m, k, n)
    got, want = gpu.read_bf16(out), oracle.gelu(vals)
    far = bf16_ulp_distance(got, want) > 1
    diff = np.abs(to_f32(got) - to_f32(want))
    limit = np.abs(to_f32(vals)) * 2.0 ** -21
    bad = far & (diff > limit)
    assert not bad.any(), (
        f"{bad.sum()} GELU values off, e.g. x={to_f32(vals)[bad][:4]}"
        f" got {to_f32(got)[bad][:4]}"
        f" want {to_f32(want)[bad][:4]}")
    # the absolute bound is needed only where 1 + tanhf(u) has lost bf16
    # precision: e^(2u) < 2^-17, i.e. u < -5.9, x < -4.2
    assert (to_f32(vals)[far] < -4.0).all(), to_f32(vals)[far].max()


def test_ffn_gelu(gpu):
    rows, d, ffn = 200, 512, 768
    rng = np.random.default_rng(5)
    x = rand_bf16(rng, rows * d)
    fc1, b1 = rand_bf16(rng, ffn * d, 0.05), rand_bf16(rng, ffn, 0.1)
    fc2, b2 = rand_bf16(rng, d * ffn, 0.05), rand_bf16(rng, d, 0.1)
    want = oracle.ffn_gelu(x, fc1, b1, fc2, b2, rows, d, ffn)
    out = gpu.new_bf16(rows * d)
    gpu.run("h3_gpu_ffn_gelu_bf16", out, None, gpu.bf16(x), gpu.bf16(fc1),
            gpu.bf16(b1), gpu.bf16(fc2), gpu.bf16(b2), rows, d, ffn, d)
    assert_close(gpu.read_bf16(out), want, what="GELU FFN", chained=1)


# ------------------------------------------------------------- row ops

WIDTHS = [8, 100, 5120, 5376]


@pytest.mark.parametrize("width", WIDTHS)
def test_adaln(gpu, width):
    rows = 37
    rng = np.random.default_rng(width)
    x = rand_bf16(rng, rows * width, 2.0)
    w = rand_bf16(rng, width, 0.1, 1.0)
    mod, rm = _mod_setup(rng, rows, width)
    want = oracle.adaln(x, w, mod, rm, rows, width, 6, 0, 1, 1e-5)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_adaln_bf16", out, gpu.bf16(x), gpu.bf16(w), gpu.bf16(mod),
            gpu.u32(rm), rows, width, 6, 0, 1, C.c_float(1e-5))
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(x, w, mod, rm, rows, width, 6, 0, 1, 1e-5),
                     "adaLN")


def test_adaln_offset(gpu):
    rows, width, off_rows = 5, 5376, 3
    rng = np.random.default_rng(9)
    x = rand_bf16(rng, (rows + off_rows) * width)
    w = rand_bf16(rng, width, 0.1, 1.0)
    mod, rm = _mod_setup(rng, rows, width)
    want = oracle.adaln(x[off_rows * width:], w, mod, rm, rows, width, 6, 3, 4,
                        1e-5)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_adaln_bf16_offset", out, gpu.bf16(x), off_rows * width,
            gpu.bf16(w), gpu.bf16(mod), gpu.u32(rm), rows, width, 6, 3, 4,
            C.c_float(1e-5))
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(x[off_rows * width:], w, mod, rm, rows,
                                 width, 6, 3, 4, 1e-5), "adaLN offset")


@pytest.mark.parametrize("width", WIDTHS)
def test_gate(gpu, width):
    rows = 29
    rng = np.random.default_rng(width + 1)
    res, br = rand_bf16(rng, rows * width), rand_bf16(rng, rows * width)
    mod, rm = _mod_setup(rng, rows, width)
    want = oracle.gate(res, br, mod, rm, rows, width, 6, 2)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_gate_bf16", out, gpu.bf16(res), gpu.bf16(br),
            gpu.bf16(mod), gpu.u32(rm), rows, width, 6, 2)
    assert_ulp(gpu.read_bf16(out), want, 0, "gate (bit-exact)")


@pytest.mark.parametrize("width", WIDTHS)
def test_gate_adaln(gpu, width):
    rows = 31
    rng = np.random.default_rng(width + 2)
    res, br = rand_bf16(rng, rows * width), rand_bf16(rng, rows * width)
    w = rand_bf16(rng, width, 0.1, 1.0)
    gmod, rm = _mod_setup(rng, rows, width)
    nmod = rand_bf16(rng, gmod.size, 0.5)
    gated_want, want = oracle.gate_adaln(res, br, w, gmod, nmod, rm, rows,
                                         width, 6, 5, 0, 1, 1e-5)
    gated, out = gpu.new_bf16(rows * width), gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_gate_adaln_bf16", gated, out, gpu.bf16(res), gpu.bf16(br),
            gpu.bf16(w), gpu.bf16(gmod), gpu.bf16(nmod), gpu.u32(rm), rows,
            width, 6, 5, 0, 1, C.c_float(1e-5))
    assert_ulp(gpu.read_bf16(gated), gated_want, 0, "gated residual")
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(gated_want, w, nmod, rm, rows, width, 6, 0,
                                 1, 1e-5), "gate+adaLN")


def test_gate_adaln_in_place(gpu):
    """The driver passes hidden as both residual and gated output."""
    rows, width = 17, 5376
    rng = np.random.default_rng(77)
    res, br = rand_bf16(rng, rows * width), rand_bf16(rng, rows * width)
    w = rand_bf16(rng, width, 0.1, 1.0)
    mod, rm = _mod_setup(rng, rows, width)
    gated_want, want = oracle.gate_adaln(res, br, w, mod, mod, rm, rows,
                                         width, 6, 2, 3, 4, 1e-5)
    hidden, out = gpu.bf16(res), gpu.new_bf16(rows * width)
    tmod = gpu.bf16(mod)
    gpu.run("h3_gpu_gate_adaln_bf16", hidden, out, hidden, gpu.bf16(br),
            gpu.bf16(w), tmod, tmod, gpu.u32(rm), rows, width, 6, 2, 3, 4,
            C.c_float(1e-5))
    assert_ulp(gpu.read_bf16(hidden), gated_want, 0, "in-place gated")
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(gated_want, w, mod, rm, rows, width, 6, 3, 4,
                                 1e-5), "in-place gate+adaLN")


@pytest.mark.parametrize("width", [8, 100, 5120])
@pytest.mark.parametrize("affine,modulated", [(False, True), (True, False),
                                              (True, True)])
def test_layer_adaln(gpu, width, affine, modulated):
    rows = 23
    rng = np.random.default_rng(width * 3 + affine + 2 * modulated)
    x = rand_bf16(rng, rows * width, 3.0, 0.5)
    w = rand_bf16(rng, width, 0.1, 1.0) if affine else None
    b = rand_bf16(rng, width, 0.1) if affine else None
    mod, rm = _mod_setup(rng, rows, width) if modulated else (None, None)
    want = oracle.layer_adaln(x, w, b, mod, rm, rows, width, 6, 0, 1, 1e-6)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_layer_adaln_bf16", out, gpu.bf16(x),
            gpu.bf16(w) if affine else None, gpu.bf16(b) if affine else None,
            gpu.bf16(mod) if modulated else None,
            gpu.u32(rm) if modulated else None, rows, width, 6, 0, 1,
            C.c_float(1e-6))
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(x, w, mod, rm, rows, width, 6, 0, 1, 1e-6,
                                 layer=True, bias=b), "LayerNorm adaLN")


@pytest.mark.parametrize("width", [100, 5120])
@pytest.mark.parametrize("gated", [True, False])
@pytest.mark.parametrize("affine,modulated", [(False, True), (True, False),
                                              (False, False), (True, True)])
def test_gate_layer_adaln_matches_the_two_ops(gpu, width, gated, affine,
                                              modulated):
    """The fused residual update + LayerNorm adaLN is bit-identical to
    h3_gpu_gate_bf16 (or h3_gpu_add_bf16) followed by h3_gpu_layer_adaln_bf16,
    in place on the residual as the Wan block calls it; the gated residual
    also matches the oracle's gate / add exactly."""
    rows = 19
    rng = np.random.default_rng(width + 4 * gated + 2 * affine + modulated)
    res, br = rand_bf16(rng, rows * width, 2.0), rand_bf16(rng, rows * width)
    mod, rm = _mod_setup(rng, rows, width)
    w = gpu.bf16(rand_bf16(rng, width, 0.1, 1.0)) if affine else None
    b = gpu.bf16(rand_bf16(rng, width, 0.1)) if affine else None
    tmod, trm, tbr = gpu.bf16(mod), gpu.u32(rm), gpu.bf16(br)
    # two ops
    h1, out1 = gpu.bf16(res), gpu.new_bf16(rows * width)
    if gated:
        gpu.run("h3_gpu_gate_bf16", h1, h1, tbr, tmod, trm, rows, width, 6, 2)
        want_gated = oracle.gate(res, br, mod, rm, rows, width, 6, 2)
    else:
        gpu.run("h3_gpu_add_bf16", h1, h1, tbr, rows * width)
        want_gated = oracle.add(res, br)
    gpu.run("h3_gpu_layer_adaln_bf16", out1, h1, w, b,
            tmod if modulated else None, trm if modulated else None, rows,
            width, 6, 3, 4, C.c_float(1e-6))
    # fused
    h2, out2 = gpu.bf16(res), gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_gate_layer_adaln_bf16", h2, out2, h2, tbr,
            tmod if gated else None, w, b, tmod if modulated else None,
            trm if (gated or modulated) else None, rows, width, 6, 2, 3, 4,
            C.c_float(1e-6))
    assert_ulp(gpu.read_bf16(h2), want_gated, 0, "gated residual")
    assert np.array_equal(gpu.read_bf16(h2), gpu.read_bf16(h1))
    assert np.array_equal(gpu.read_bf16(out2), gpu.read_bf16(out1))


@pytest.mark.parametrize("width", [8, 5376])
def test_rms_norm(gpu, width):
    rows = 9
    rng = np.random.default_rng(width + 3)
    x, w = rand_bf16(rng, rows * width), rand_bf16(rng, width, 0.1, 1.0)
    want = oracle.rms_norm(x, w, rows, width, 1e-5)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_rms_norm_bf16", out, gpu.bf16(x), gpu.bf16(w), rows, width,
            C.c_float(1e-5))
    assert_row_close(gpu.read_bf16(out), want,
                     adaln_terms(x, w, None, None, rows, width, 6, 0, 0,
                                 1e-5), "RMS norm")


@pytest.mark.parametrize("hd", [128, 64])
def test_head_rms_norm(gpu, hd):
    rows, heads = 33, 5
    rng = np.random.default_rng(11)
    x, w = rand_bf16(rng, rows * heads * hd), rand_bf16(rng, hd, 0.1, 1.0)
    want = oracle.head_rms_norm(x, w, rows, heads, hd, 1e-6)
    t = gpu.bf16(x)
    gpu.run("h3_gpu_head_rms_norm_bf16", t, gpu.bf16(w), rows, heads, hd,
            C.c_float(1e-6))
    assert_ulp(gpu.read_bf16(t), want, 1, "head RMS norm")


@pytest.mark.parametrize("grouped", [True, False])
@pytest.mark.parametrize("hd,rope_half", [(128, 48), (128, 64), (128, 52),
                                          (128, 46), (64, 16)])
def test_qkv_rope(gpu, grouped, hd, rope_half):
    seq, heads = 45, 3
    rng = np.random.default_rng(hd + rope_half + grouped)
    qkv = rand_bf16(rng, seq * 3 * heads * hd)
    qw, kw = rand_bf16(rng, hd, 0.1, 1.0), rand_bf16(rng, hd, 0.1, 1.0)
    ang = rng.uniform(-30, 30, seq * rope_half).astype(np.float32)
    cos, sin = oracle.bf16(np.cos(ang)), oracle.bf16(np.sin(ang))
    q, k, v = oracle.qkv_rope(qkv, qw, kw, cos, sin, seq, heads, hd,
                              rope_half, grouped, 1e-5)
    n = seq * heads * hd
    tq, tk, tv = gpu.new_bf16(n), gpu.new_bf16(n), gpu.new_bf16(n)
    name = ("h3_gpu_grouped_qkv_rope_bf16" if grouped
            else "h3_gpu_qkv_rope_bf16")
    gpu.run(name, tq, tk, tv, gpu.bf16(qkv), gpu.bf16(qw), gpu.bf16(kw),
            gpu.bf16(cos), gpu.bf16(sin), seq, heads, hd, rope_half,
            C.c_float(1e-5))
    assert_ulp(gpu.read_bf16(tq), q, 1, "query")
    assert_ulp(gpu.read_bf16(tk), k, 1, "key")
    assert_ulp(gpu.read_bf16(tv), v, 0, "value copy")


@pytest.mark.parametrize("seq,heads", [(45, 3), (300, 2), (2378, 4)])
def test_qkv_in_place_and_fused_attention(gpu, seq, heads):
    """The in-place Q/K norm + RoPE leaves, in the fused rows, exactly what
    h3_gpu_qkv_rope_bf16 writes to separate tensors (V untouched), and
    attention on the fused rows equals attention on those tensors, bit for
    bit."""
    hd, rope_half = 128, 48
    rng = np.random.default_rng(seq + heads)
    qkv = rand_bf16(rng, seq * 3 * heads * hd)
    qw, kw = rand_bf16(rng, hd, 0.1, 1.0), rand_bf16(rng, hd, 0.1, 1.0)
    ang = rng.uniform(-30, 30, seq * rope_half).astype(np.float32)
    cos, sin = oracle.bf16(np.cos(ang)), oracle.bf16(np.sin(ang))
    n = seq * heads * hd
    tq, tk, tv = gpu.new_bf16(n), gpu.new_bf16(n), gpu.new_bf16(n)
    tqw, tkw, tc, ts = gpu.bf16(qw), gpu.bf16(kw), gpu.bf16(cos), gpu.bf16(sin)
    gpu.run("h3_gpu_qkv_rope_bf16", tq, tk, tv, gpu.bf16(qkv), tqw, tkw, tc,
            ts, seq, heads, hd, rope_half, C.c_float(1e-5))
    fused = gpu.bf16(qkv)
    gpu.run("h3_hip_qk_norm_rope_inplace_bf16", fused, tqw, tkw, tc, ts, seq,
            heads, hd, rope_half, C.c_float(1e-5), 0)
    rows = gpu.read_bf16(fused).view(np.uint16).reshape(seq, 3, heads * hd)
    q = gpu.read_bf16(tq).view(np.uint16).reshape(seq, heads * hd)
    k = gpu.read_bf16(tk).view(np.uint16).reshape(seq, heads * hd)
    v = qkv.view(np.uint16).reshape(seq, 3, heads * hd)[:, 2]
    assert np.array_equal(rows[:, 0], q)
    assert np.array_equal(rows[:, 1], k)
    assert np.array_equal(rows[:, 2], v)
    scale = C.c_float(1.0 / math.sqrt(hd))
    split, joint = gpu.new_bf16(n), gpu.new_bf16(n)
    gpu.run("h3_gpu_sdpa_bf16", split, tq, tk, tv, seq, heads, hd, scale)
    gpu.run("h3_hip_sdpa_qkv_bf16", joint, fused, seq, heads, hd, scale)
    assert np.array_equal(gpu.read_bf16(split).view(np.uint16),
                          gpu.read_bf16(joint).view(np.uint16))


@pytest.mark.parametrize("seq,heads", [(45, 3), (300, 2), (2378, 4)])
def test_q_norm_rope_in_attention(gpu, seq, heads):
    """h3_hip_sdpa_qkv_norm_rope_bf16 on rows whose K alone was normalised
    and rotated in place equals normalising and rotating Q and K in place
    first and calling h3_hip_sdpa_qkv_bf16, bit for bit: the attention
    kernel repeats the row kernel's sums, rounding and RoPE exactly."""
    hd, rope_half = 128, 48
    rng = np.random.default_rng(7 * seq + heads)
    qkv = rand_bf16(rng, seq * 3 * heads * hd, 2.0)
    qw, kw = rand_bf16(rng, hd, 0.1, 1.0), rand_bf16(rng, hd, 0.1, 1.0)
    ang = rng.uniform(-30, 30, seq * rope_half).astype(np.float32)
    cos, sin = oracle.bf16(np.cos(ang)), oracle.bf16(np.sin(ang))
    tqw, tkw, tc, ts = gpu.bf16(qw), gpu.bf16(kw), gpu.bf16(cos), gpu.bf16(sin)
    eps, scale = C.c_float(1e-6), C.c_float(1.0 / math.sqrt(hd))
    both, keys = gpu.bf16(qkv), gpu.bf16(qkv)
    gpu.run("h3_hip_qk_norm_rope_inplace_bf16", both, tqw, tkw, tc, ts, seq,
            heads, hd, rope_half, eps, 0)
    gpu.run("h3_hip_qk_norm_rope_inplace_bf16", keys, tqw, tkw, tc, ts, seq,
            heads, hd, rope_half, eps, 1)
    rows_b = gpu.read_bf16(both).view(np.uint16).reshape(seq, 3, -1)
    rows_k = gpu.read_bf16(keys).view(np.uint16).reshape(seq, 3, -1)
    assert np.array_equal(rows_b[:, 1:], rows_k[:, 1:])
    assert np.array_equal(rows_k[:, 0],
                          qkv.view(np.uint16).reshape(seq, 3, -1)[:, 0])
    n = seq * heads * hd
    want, got = gpu.new_bf16(n), gpu.new_bf16(n)
    gpu.run("h3_hip_sdpa_qkv_bf16", want, both, seq, heads, hd, scale)
    gpu.run("h3_hip_sdpa_qkv_norm_rope_bf16", got, keys, tqw, tc, ts, seq,
            heads, hd, rope_half, eps, scale)
    assert np.array_equal(gpu.read_bf16(want).view(np.uint16),
                          gpu.read_bf16(got).view(np.uint16))


@pytest.mark.parametrize("q_rows,kv_rows,heads", [(300, 77, 2), (1000, 512, 3),
                                                  (70, 513, 2)])
def test_cross_q_norm_in_attention(gpu, q_rows, kv_rows, heads):
    """h3_hip_sdpa_cross_norm_bf16 equals h3_gpu_head_rms_norm_bf16 on Q
    followed by h3_gpu_sdpa_cross_bf16, bit for bit."""
    hd = 128
    rng = np.random.default_rng(q_rows + kv_rows + heads)
    q = rand_bf16(rng, q_rows * heads * hd, 3.0)
    k = rand_bf16(rng, kv_rows * heads * hd)
    v = rand_bf16(rng, kv_rows * heads * hd)
    w = rand_bf16(rng, hd, 0.1, 1.0)
    tq, tk, tv, tw = gpu.bf16(q), gpu.bf16(k), gpu.bf16(v), gpu.bf16(w)
    eps, scale = C.c_float(1e-6), C.c_float(1.0 / math.sqrt(hd))
    n = q_rows * heads * hd
    want, got = gpu.new_bf16(n), gpu.new_bf16(n)
    normed = gpu.bf16(q)
    gpu.run("h3_gpu_head_rms_norm_bf16", normed, tw, q_rows, heads, hd, eps)
    gpu.run("h3_gpu_sdpa_cross_bf16", want, normed, tk, tv, q_rows, kv_rows,
            heads, hd, scale)
    gpu.run("h3_hip_sdpa_cross_norm_bf16", got, tq, tk, tv, tw, q_rows,
            kv_rows, heads, hd, eps, scale)
    assert np.array_equal(gpu.read_bf16(want).view(np.uint16),
                          gpu.read_bf16(got).view(np.uint16))


def test_qkv_in_place_rejects_other_shapes(gpu):
    seq, heads, hd = 8, 2, 64
    buf = gpu.new_bf16(seq * 3 * heads * hd)
    w = gpu.new_bf16(hd)
    tab = gpu.new_bf16(seq * 16)
    gpu.begin()
    ok = gpu.L.h3_hip_qk_norm_rope_inplace_bf16(gpu.h, buf, w, w, tab, tab,
                                                seq, heads, hd, 16,
                                                C.c_float(1e-5), 0)
    gpu.submit()
    assert not ok and "head_dim 128" in gpu.error()


# ------------------------------------------------------------ attention

@pytest.mark.parametrize("q_rows,kv_rows,heads", [
    (100, 100, 2),      # reference test_cuda_attention.c hd128 N=100
    (300, 300, 3),      # two 256-query blocks, ragged key tail, 2 pieces
    (64, 64, 1),        # exactly one key tile
    (1000, 1000, 2),    # 8 work items on 256 CUs: 8 key-range pieces each
    (2378, 2378, 4),    # H3 length: 40 items, 8 pieces of 5 key tiles
    (300, 77, 2),       # cross attention, short context
    (70, 513, 2),       # cross attention, more keys than queries
])
def test_sdpa(gpu, q_rows, kv_rows, heads):
    hd = 128
    rng = np.random.default_rng(q_rows * 3 + kv_rows)
    q = rand_bf16(rng, q_rows * heads * hd)
    k = rand_bf16(rng, kv_rows * heads * hd)
    v = rand_bf16(rng, kv_rows * heads * hd)
    scale = 1.0 / math.sqrt(hd)
    want = oracle.sdpa(q, k, v, q_rows, kv_rows, heads, hd, scale)
    out = gpu.new_bf16(q_rows * heads * hd)
    if q_rows == kv_rows:
        gpu.run("h3_gpu_sdpa_bf16", out, gpu.bf16(q), gpu.bf16(k), gpu.bf16(v),
                q_rows, heads, hd, C.c_float(scale))
    else:
        gpu.run("h3_gpu_sdpa_cross_bf16", out, gpu.bf16(q), gpu.bf16(k),
                gpu.bf16(v), q_rows, kv_rows, heads, hd, C.c_float(scale))
    assert_close(gpu.read_bf16(out), want, what=f"SDPA {q_rows}x{kv_rows}",
                 extra_abs=sdpa_p_rounding_bound(q, k, v, q_rows, kv_rows,
                                                 heads, hd, scale))


@pytest.mark.parametrize("rows,heads", [
    (100, 2),       # one query block, ragged single key tile
    (300, 3),       # two query blocks, ragged tail, key-split pieces
    (1000, 2),      # 8 key-range pieces per item
    (2378, 4),      # the H3 length
])
def test_sdpa_rope_in_kernel(gpu, rows, heads):
    """Attention with the RoPE rotation inside the kernel equals the
    oracle's rotation followed by the oracle's attention."""
    hd = 128
    rng = np.random.default_rng(rows * 7 + heads)
    q, k, v = (rand_bf16(rng, rows * heads * hd) for _ in range(3))
    ang = rng.uniform(-30, 30, rows * 48)
    cos, sin = oracle.bf16(np.cos(ang)), oracle.bf16(np.sin(ang))
    scale = 1.0 / math.sqrt(hd)
    qr = oracle.rope_rotate(q, cos, sin, rows, heads)
    kr = oracle.rope_rotate(k, cos, sin, rows, heads)
    want = oracle.sdpa(qr, kr, v, rows, rows, heads, hd, scale)
    out = gpu.new_bf16(rows * heads * hd)
    gpu.run("h3_hip_sdpa_rope_bf16", out, gpu.bf16(q), gpu.bf16(k),
            gpu.bf16(v), gpu.bf16(cos), gpu.bf16(sin), rows, heads, hd, 48,
            C.c_float(scale))
    got = gpu.read_bf16(out)
    assert_close(got, want, what=f"RoPE SDPA {rows}",
                 extra_abs=sdpa_p_rounding_bound(qr, kr, v, rows, rows,
                                                 heads, hd, scale))
    # and the two-step path through the ordinary kernel
    ref = gpu.new_bf16(rows * heads * hd)
    gpu.run("h3_gpu_sdpa_bf16", ref, gpu.bf16(qr), gpu.bf16(kr), gpu.bf16(v),
            rows, heads, hd, C.c_float(scale))
    np.testing.assert_array_equal(got, gpu.read_bf16(ref))


def test_sdpa_rope_rejects_other_tables(gpu):
    rows, heads, hd = 64, 1, 128
    t = gpu.new_bf16(rows * heads * hd)
    c = gpu.new_bf16(rows * 32)
    gpu.begin()
    ok = gpu.L.h3_hip_sdpa_rope_bf16(gpu.h, t, t, t, t, c, c, rows, heads,
                                     hd, 32, C.c_float(0.1))
    gpu.submit()
    assert not ok and "rope_half 48" in gpu.error()


@pytest.mark.parametrize("n", [150, 1000])   # 1000: key-split pieces
def test_sdpa_head_major(gpu, n):
    heads, hd = 2, 128
    rng = np.random.default_rng(21 + n)
    q, k, v = (rand_bf16(rng, n * heads * hd) for _ in range(3))
    scale = 1.0 / math.sqrt(hd)
    want = oracle.sdpa(q, k, v, n, n, heads, hd, scale, head_major=True)
    out = gpu.new_bf16(n * heads * hd)
    gpu.run("h3_gpu_sdpa_bf16_head_major_output", out, gpu.bf16(q),
            gpu.bf16(k), gpu.bf16(v), n, heads, hd, C.c_float(scale))
    assert_close(gpu.read_bf16(out), want, what="head-major SDPA",
                 extra_abs=sdpa_p_rounding_bound(q, k, v, n, n, heads, hd,
                                                 scale, head_major=True))


@pytest.mark.parametrize("q_rows,kv_rows,pattern", [
    (700, 700, "rising"),     # 11 key tiles, ragged tail
    (1000, 1000, "rising"),   # key-range pieces: each piece's own maximum
    (300, 513, "rising"),     # cross attention
    (700, 700, "spikes"),     # maximum in the first tile, then jumps
    (100, 100, "rising"),     # a single ragged key tile
])
def test_sdpa_running_max_moves(gpu, q_rows, kv_rows, pattern):
    """Keys along q's direction with growing length make later key tiles
    score far above the running maximum (by more than 32 in the exp2
    domain), so the kernel must move its maximum and rescale O and l
    mid-sequence, several times per row."""
    heads, hd = 2, 128
    rng = np.random.default_rng(kv_rows + (7 if pattern == "spikes" else 0))
    u = rng.choice([-1.0, 1.0], hd).astype(np.float32)
    if pattern == "rising":
        amp = np.linspace(-2.0, 12.0, kv_rows)
    else:
        amp = rng.uniform(-1.0, 1.0, kv_rows)
        amp[:8] = 4.0
        amp[kv_rows // 3] = 9.0
        amp[2 * kv_rows // 3] = 14.0
    kf = (amp[:, None, None] * u[None, None, :] +
          0.05 * rng.standard_normal((kv_rows, heads, hd)))
    qf = 0.5 * u[None, None, :] + 0.05 * rng.standard_normal(
        (q_rows, heads, hd))
    q = oracle.bf16(qf.astype(np.float32).ravel())
    k = oracle.bf16(kf.astype(np.float32).ravel())
    v = rand_bf16(rng, kv_rows * heads * hd)
    scale = 1.0 / math.sqrt(hd)
    want = oracle.sdpa(q, k, v, q_rows, kv_rows, heads, hd, scale)
    out = gpu.new_bf16(q_rows * heads * hd)
    if q_rows == kv_rows:
        gpu.run("h3_gpu_sdpa_bf16", out, gpu.bf16(q), gpu.bf16(k), gpu.bf16(v),
                q_rows, heads, hd, C.c_float(scale))
    else:
        gpu.run("h3_gpu_sdpa_cross_bf16", out, gpu.bf16(q), gpu.bf16(k),
                gpu.bf16(v), q_rows, kv_rows, heads, hd, C.c_float(scale))
    assert_close(gpu.read_bf16(out), want,
                 what=f"SDPA {q_rows}x{kv_rows} {pattern}",
                 extra_abs=sdpa_p_rounding_bound(q, k, v, q_rows, kv_rows,
                                                 heads, hd, scale))


def test_sdpa_constant_keys_give_mean_value(gpu):
    """Invariant: identical keys -> uniform softmax -> output = mean of V."""
    n, heads, hd = 200, 1, 128
    rng = np.random.default_rng(3)
    q = rand_bf16(rng, n * heads * hd)
    k = np.tile(rand_bf16(rng, hd), n)
    vf = rng.standard_normal((n, hd)).astype(np.float32)
    v = oracle.bf16(vf)
    out = gpu.new_bf16(n * hd)
    gpu.run("h3_gpu_sdpa_bf16", out, gpu.bf16(q), gpu.bf16(k), gpu.bf16(v), n,
            heads, hd, C.c_float(1.0 / math.sqrt(hd)))
    got = to_f32(gpu.read_bf16(out)).reshape(n, hd)
    mean = to_f32(v).reshape(n, hd).astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(got, np.broadcast_to(mean, got.shape),
                               atol=2e-2, rtol=2e-2)


# --------------------------------------------------------- elementwise

def test_swiglu_gelu_add_sub(gpu):
    rows, width = 13, 300
    rng = np.random.default_rng(4)
    fused = rand_bf16(rng, rows * 2 * width, 3.0)
    out = gpu.new_bf16(rows * width)
    gpu.run("h3_gpu_swiglu_bf16", out, gpu.bf16(fused), rows, width)
    assert_ulp(gpu.read_bf16(out), oracle.swiglu(fused, rows, width), 1,
               "SwiGLU")
    x = rand_bf16(rng, 5000, 4.0)
    out = gpu.new_bf16(x.size)
    gpu.run("h3_gpu_gelu_bf16", out, gpu.bf16(x), x.size, 1)
    assert_ulp(gpu.read_bf16(out), oracle.gelu(x), 1, "GELU tanh")
    y = rand_bf16(rng, 5000)
    gpu.run("h3_gpu_add_bf16", out, gpu.bf16(x), gpu.bf16(y), x.size)
    assert_ulp(gpu.read_bf16(out), oracle.add(x, y), 0, "add")
    # 8-wide body plus a 3-element tail, in place
    x, y = rand_bf16(rng, 5003, 4.0), rand_bf16(rng, 5003)
    t = gpu.bf16(x)
    gpu.run("h3_gpu_add_bf16", t, t, gpu.bf16(y), x.size)
    assert_ulp(gpu.read_bf16(t), oracle.add(x, y), 0, "add, ragged")


def test_euler_step(gpu):
    n = 4099
    rng = np.random.default_rng(8)
    sample = rng.standard_normal(n + 10).astype(np.float32)
    last, prev = rand_bf16(rng, n), rand_bf16(rng, n)
    delta, ratio = 0.0625, -0.5
    want = sample.copy()
    want[10:] = oracle.euler(sample[10:], last, prev, delta, ratio)
    t = gpu.f32(sample)
    gpu.run("h3_gpu_euler_bf16", t, 10, gpu.bf16(last), gpu.bf16(prev), n,
            C.c_float(delta), C.c_float(ratio))
    np.testing.assert_array_equal(gpu.read_f32(t), want)


def test_final_adaln_head(gpu):
    rows, width, n, slots = 20, 5376, 96, 2
    rng = np.random.default_rng(12)
    x = rand_bf16(rng, (rows + 4) * width)
    nw = rand_bf16(rng, width, 0.1, 1.0)
    mod, rm = _mod_setup(rng, rows, width, slots=slots, mod_rows=2)
    w, b = rand_bf16(rng, n * width, 0.02), rand_bf16(rng, n, 0.1)
    want, inv_want = oracle.adaln_linear(x[4 * width:], nw, mod, rm, w, b,
                                         rows, width, n, slots, 0, 1, 1e-5)
    out, inv = gpu.new_bf16(rows * n), gpu.new_f32(rows)
    gpu.run("h3_gpu_adaln_linear_bf16", out, inv, gpu.bf16(x), 4 * width,
            gpu.bf16(nw), gpu.bf16(mod), gpu.u32(rm), gpu.bf16(w), gpu.bf16(b),
            rows, width, n, slots, 0, 1, C.c_float(1e-5))
    np.testing.assert_allclose(gpu.read_f32(inv), inv_want, rtol=1e-5)
    assert_close(gpu.read_bf16(out), want, what="final head", chained=1)


def test_patch_linear_bit_exact(gpu):
    """F32 patch projection keeps the reference hand kernel's sequential
    order, so it matches the oracle bit for bit."""
    rows, k, n = 40, 96, 5376
    rng = np.random.default_rng(13)
    x = rng.standard_normal(rows * k).astype(np.float32)
    w = (0.05 * rng.standard_normal(n * k)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    out_rows = 50
    rm = rng.permutation(out_rows)[:rows].astype(np.uint32)
    want = oracle.patch_linear(x, w, b, rows, k, n, row_map=rm,
                               out_rows=out_rows)
    out = gpu.bf16(np.zeros(out_rows * n, np.uint16))
    gpu.run("h3_gpu_patch_linear_bf16_map", out, gpu.f32(x), gpu.f32(w),
            gpu.f32(b), gpu.u32(rm), out_rows, rows, k, n)
    assert_ulp(gpu.read_bf16(out), want, 0, "mapped patch projection")


def test_patch_linear_shapes(gpu):
    """The h3_gpu_ entries accept only the checkpoint shapes (5376 outputs
    from 32 or 96 inputs, h3_cuda_core.cu:929-930; the reference's own test
    tests/test_cuda_core.c:890-894); the h3_hip_ variant takes a reduced
    width, bit-exact against the oracle."""
    rows, k, n = 12, 96, 256
    rng = np.random.default_rng(14)
    x = rng.standard_normal(rows * k).astype(np.float32)
    w = (0.05 * rng.standard_normal(n * k)).astype(np.float32)
    out = gpu.new_bf16(rows * n)
    tx, tw = gpu.f32(x), gpu.f32(w)
    gpu.begin()
    assert not gpu.L.h3_gpu_patch_linear_bf16_offset(gpu.h, out, 0, tx, 0, tw,
                                                      None, rows, k, n)
    assert "unsupported fused patch projection shape" in gpu.error()
    gpu.submit()
    gpu.run("h3_hip_patch_linear_bf16_offset", out, 0, tx, 0, tw, None, rows,
            k, n)
    want = oracle.patch_linear(x, w, None, rows, k, n)
    assert_ulp(gpu.read_bf16(out), want, 0, "reduced-width patch projection")


# ------------------------------------------------------------ contract

def test_ops_require_an_open_batch(gpu):
    t = gpu.new_bf16(16)
    ok = gpu.L.h3_gpu_add_bf16(gpu.h, t, t, t, 16)
    assert ok == 0 and "no active command buffer" in gpu.error()


def test_validation_errors(gpu):
    rng = np.random.default_rng(0)
    x = gpu.bf16(rand_bf16(rng, 64))
    f = gpu.new_f32(64)
    gpu.begin()
    try:
        assert gpu.L.h3_gpu_add_bf16(gpu.h, f, x, x, 64) == 0
        assert "wrong dtype" in gpu.error()
        assert gpu.L.h3_gpu_add_bf16(gpu.h, x, x, x, 65) == 0
        assert "too small" in gpu.error()
        mod, rm = gpu.bf16(rand_bf16(rng, 6 * 8)), gpu.u32(np.zeros(8, np.uint32))
        assert gpu.L.h3_gpu_gate_bf16(gpu.h, x, x, x, mod, rm, 8, 8, 6,
                                      6) == 0
        assert "slot" in gpu.error()
        assert gpu.L.h3_gpu_gate_adaln_bf16(
            gpu.h, x, x, x, x, x, mod, mod, rm, 1, 6000, 6, 2, 3, 4,
            C.c_float(1e-5)) == 0
        assert "out of range" in gpu.error()
    finally:
        gpu.L.h3_gpu_submit(gpu.h)


def test_int8_paths_report_unavailable(gpu):
    assert gpu.L.h3_gpu_has_int8_mlp(gpu.h) == 0
    assert gpu.L.h3_gpu_prefers_gpu_sampler(gpu.h) == 1

