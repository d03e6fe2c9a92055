"""Pins for the CPU oracle (oracle/h3_oracle.c) before it is trusted as the
checker of the HIP backend.

The reference's GPU arithmetic cannot run here (CUDA/Metal only), so each
oracle function is pinned by checks chosen so that a plausible mistake -- a
dropped term, a wrong slot or index, a transposed operand, a missing
rounding -- fails one of them:
  * exact small cases whose f32 arithmetic has no rounding at all;
  * float64 restatements of the reference formulas (cited per test) with a
    bound of one bf16 rounding;
  * invariants: zero gate -> residual, scale = -1 & shift = 0 -> zero,
    RoPE at position 0 -> identity and norm preservation, constant keys ->
    mean of V, a dominant key -> its value row, SwiGLU of zero -> zero;
  * the reference's own tiny op tests' shapes (tests/test_cuda_dit.c:135-143
    ROW_MAP {2,0,3,1}, tests/test_cuda_core.c MLP 4x8x6x5).
"""
import math

import numpy as np
import pytest

import oracle
from conftest import bf16_ulp_distance, to_f32

rng = np.random.default_rng(1234)


def b(x):
    return oracle.bf16(np.asarray(x, np.float32))


def f64(bits):
    return to_f32(bits).astype(np.float64)


def within_one_rounding(got_bits, exact, extra=0.0):
    """|got - exact| <= half a bf16 ulp of |exact| (+ extra)."""
    g = f64(got_bits)
    ex = np.asarray(exact, np.float64)
    mag = np.maximum(np.abs(ex), 1e-30)
    half_ulp = np.ldexp(1.0, np.frexp(mag)[1] - 9)
    return np.all(np.abs(g - ex) <= half_ulp * 1.0001 + extra)


# ---------------------------------------------------------------- linear

def test_linear_exact_small_integers():
    """Integer inputs: every partial sum is exact in f32, so the oracle must
    equal the integer matrix product (checks operand order W[n,k] and the
    bias)."""
    m, k, n = 3, 5, 4
    x = rng.integers(-4, 5, (m, k)).astype(np.float32)
    w = rng.integers(-4, 5, (n, k)).astype(np.float32)
    bias = rng.integers(-3, 4, n).astype(np.float32)
    got = to_f32(oracle.linear(b(x), b(w), b(bias), m, k, n)).reshape(m, n)
    np.testing.assert_array_equal(got, x @ w.T + bias)


def test_linear_against_float64():
    m, k, n = 37, 300, 70
    x, w = b(rng.standard_normal(m * k)), b(0.1 * rng.standard_normal(n * k))
    exact = f64(x).reshape(m, k) @ f64(w).reshape(n, k).T
    got = oracle.linear(x, w, None, m, k, n)
    # f32 sequential accumulation error bound k * 2^-24 * sum|x||w|
    bound = k * 2.0 ** -24 * (np.abs(f64(x).reshape(m, k)) @
                              np.abs(f64(w).reshape(n, k)).T)
    assert within_one_rounding(got, exact.ravel(), bound.ravel())


def test_linear_f32_exact_and_against_float64():
    """F32 linear: integer inputs are exact (operand order and bias); random
    inputs stay within the sequential-accumulation bound of float64."""
    m, k, n = 4, 6, 5
    x = rng.integers(-4, 5, (m, k)).astype(np.float32)
    w = rng.integers(-4, 5, (n, k)).astype(np.float32)
    bias = rng.integers(-3, 4, n).astype(np.float32)
    got = oracle.linear_f32(x, w, bias, m, k, n).reshape(m, n)
    np.testing.assert_array_equal(got, x @ w.T + bias)
    m, k, n = 9, 256, 40
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (0.1 * rng.standard_normal((n, k))).astype(np.float32)
    got = oracle.linear_f32(x, w, None, m, k, n).astype(np.float64)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = k * 2.0 ** -24 * (np.abs(x).astype(np.float64) @
                              np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got.reshape(m, n) - exact) <= bound + 1e-30)


def test_time_embedding_composition():
    """The timestep MLP (h3_dit_schedule.c:163-234) against a float64
    restatement: linear, x * sigmoid(x), linear, then bf16 rounding and the
    bf16 SiLU; equal within one bf16 rounding of the result."""
    rows, inp, hid, dim = 3, 16, 12, 8
    feat = rng.standard_normal(rows * inp).astype(np.float32)
    w1 = (0.3 * rng.standard_normal(hid * inp)).astype(np.float32)
    b1 = (0.1 * rng.standard_normal(hid)).astype(np.float32)
    w2 = (0.3 * rng.standard_normal(dim * hid)).astype(np.float32)
    b2 = (0.1 * rng.standard_normal(dim)).astype(np.float32)
    got = f64(oracle.time_embedding(feat, w1, b1, w2, b2, rows, inp, hid,
                                    dim))
    h = feat.astype(np.float64).reshape(rows, inp) @ \
        w1.astype(np.float64).reshape(hid, inp).T + b1
    h = h / (1 + np.exp(-h))
    o = h @ w2.astype(np.float64).reshape(dim, hid).T + b2
    o = f64(b(o.astype(np.float32)))
    want = (o / (1 + np.exp(-o))).ravel()
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)


# ------------------------------------------------------------ row ops

def _adaln64(x, w, mod, rm, rows, width, slots, shift, scale, eps):
    x = f64(x).reshape(rows, width)
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    m = f64(mod).reshape(-1, slots, width)[np.asarray(rm)]
    return (x * inv * f64(w)[None] * (1 + m[:, scale]) + m[:, shift]).ravel()


def test_adaln_reference_shape_and_formula():
    """tests/test_cuda_dit.c:135-143 shape: 4 rows, width 8, 3 slots,
    ROW_MAP {2, 0, 3, 1}; h3_cuda_dit.cu:141-175 formula."""
    rows, width, slots = 4, 8, 3
    rm = np.array([2, 0, 3, 1], np.uint32)
    x = b(rng.standard_normal(rows * width))
    w = b(1 + 0.1 * rng.standard_normal(width))
    mod = b(0.5 * rng.standard_normal(4 * slots * width))
    got = oracle.adaln(x, w, mod, rm, rows, width, slots, 0, 1, 1e-5)
    exact = _adaln64(x, w, mod, rm, rows, width, slots, 0, 1, 1e-5)
    assert within_one_rounding(got, exact, 1e-6 * np.abs(exact) + 1e-7)
    # slot order matters: swapping shift and scale must change the result
    swapped = oracle.adaln(x, w, mod, rm, rows, width, slots, 1, 0, 1e-5)
    assert not np.array_equal(swapped, got)


def test_adaln_scale_minus_one_is_zero():
    rows, width = 3, 64
    x = b(rng.standard_normal(rows * width))
    mod = np.zeros(2 * width, np.float32)
    mod[width:] = -1.0                      # slot 1 = scale = -1, shift = 0
    got = oracle.adaln(x, b(np.ones(width)), b(mod), [0, 0, 0], rows, width,
                       2, 0, 1, 1e-5)
    assert np.all(f64(got) == 0.0)


def test_adaln_unit_rms():
    rows, width = 5, 512
    x = b(3 * rng.standard_normal(rows * width))
    got = f64(oracle.adaln(x, b(np.ones(width)), b(np.zeros(2 * width)),
                           [0] * rows, rows, width, 2, 0, 1, 0.0))
    rms = np.sqrt((got.reshape(rows, width) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms, 1.0, atol=3e-3)


def test_gate_bit_exact_and_zero_gate():
    """h3_cuda_dit.cu:261-276: bf16(res + br * g).  bf16 x bf16 products and
    their sum with a bf16 are exact in float64, so rounding the float64
    value to f32 and then to bf16 is the same single rounding."""
    rows, width, slots = 4, 16, 6
    res, br = b(rng.standard_normal(rows * width)), b(
        rng.standard_normal(rows * width))
    mod = b(rng.standard_normal(3 * slots * width))
    rm = np.array([2, 0, 1, 2], np.uint32)
    got = oracle.gate(res, br, mod, rm, rows, width, slots, 4)
    g = f64(mod).reshape(3, slots, width)[rm][:, 4]
    exact = (f64(res).reshape(rows, width) + f64(br).reshape(rows, width) * g)
    np.testing.assert_array_equal(got, b(exact.astype(np.float32).ravel()))
    zero = oracle.gate(res, br, b(np.zeros(3 * slots * width)), rm, rows,
                       width, slots, 4)
    np.testing.assert_array_equal(zero, res)


def test_gate_adaln_is_gate_then_adaln():
    rows, width, slots = 6, 40, 6
    res, br = b(rng.standard_normal(rows * width)), b(
        rng.standard_normal(rows * width))
    w = b(1 + 0.1 * rng.standard_normal(width))
    gmod, nmod = b(rng.standard_normal(2 * slots * width)), b(
        rng.standard_normal(2 * slots * width))
    rm = np.array([1, 0, 1, 1, 0, 0], np.uint32)
    gated, out = oracle.gate_adaln(res, br, w, gmod, nmod, rm, rows, width,
                                   slots, 5, 0, 1, 1e-5)
    np.testing.assert_array_equal(
        gated, oracle.gate(res, br, gmod, rm, rows, width, slots, 5))
    np.testing.assert_array_equal(
        out, oracle.adaln(gated, w, nmod, rm, rows, width, slots, 0, 1, 1e-5))


def test_layer_adaln_statistics_and_formula():
    rows, width = 4, 256
    x = b(2 + 3 * rng.standard_normal(rows * width))
    plain = f64(oracle.layer_adaln(x, None, None, None, None, rows, width, 6,
                                   0, 0, 0.0)).reshape(rows, width)
    np.testing.assert_allclose(plain.mean(axis=1), 0, atol=3e-3)
    np.testing.assert_allclose(plain.var(axis=1), 1, atol=6e-3)
    w, bias = b(1 + 0.2 * rng.standard_normal(width)), b(
        0.3 * rng.standard_normal(width))
    mod = b(0.5 * rng.standard_normal(6 * width))
    got = oracle.layer_adaln(x, w, bias, mod, [0] * rows, rows, width, 6, 3,
                             4, 1e-6)
    xf = f64(x).reshape(rows, width)
    n = (xf - xf.mean(1, keepdims=True)) / np.sqrt(xf.var(1, keepdims=True) +
                                                    1e-6)
    m = f64(mod).reshape(6, width)
    exact = ((n * f64(w) + f64(bias)) * (1 + m[4]) + m[3]).ravel()
    assert within_one_rounding(got, exact, 1e-5 * (np.abs(n) + 1).ravel())


def test_head_rms_norm():
    rows, heads, hd = 3, 2, 128
    t = b(rng.standard_normal(rows * heads * hd))
    w = b(1 + 0.1 * rng.standard_normal(hd))
    got = oracle.head_rms_norm(t, w, rows, heads, hd, 1e-6)
    x = f64(t).reshape(rows * heads, hd)
    exact = x / np.sqrt((x * x).mean(1, keepdims=True) + 1e-6) * f64(w)
    assert within_one_rounding(got, exact.ravel(), 1e-6 * np.abs(exact).ravel())


# ---------------------------------------------------------------- RoPE

def _qkv_rope64(qkv, qw, kw, cos, sin, seq, heads, hd, half, grouped, eps):
    x = f64(qkv).reshape(seq, -1)
    out = []
    for part, wt in ((0, qw), (1, kw)):
        o = np.zeros((seq, heads, hd))
        for h in range(heads):
            if grouped:
                v = x[:, h * 3 * hd + part * hd: h * 3 * hd + (part + 1) * hd]
            else:
                v = x[:, part * heads * hd + h * hd: part * heads * hd +
                      (h + 1) * hd]
            n = v / np.sqrt((v * v).mean(1, keepdims=True) + eps) * f64(wt)
            c = f64(cos).reshape(seq, half)
            s = f64(sin).reshape(seq, half)
            r = n.copy()
            r[:, :half] = n[:, :half] * c - n[:, half:2 * half] * s
            r[:, half:2 * half] = n[:, half:2 * half] * c + n[:, :half] * s
            o[:, h] = r
        out.append(o.ravel())
    return out


@pytest.mark.parametrize("grouped", [True, False])
def test_qkv_rope_formula(grouped):
    """h3_cuda_attention.cu:175-237: per-head RMS, weight, rotate-half RoPE
    on dims [0, 2*half); grouped rows [head][q,k,v][dim]."""
    seq, heads, hd, half = 5, 2, 128, 48
    qkv = b(rng.standard_normal(seq * 3 * heads * hd))
    qw, kw = b(1 + 0.1 * rng.standard_normal(hd)), b(
        1 + 0.1 * rng.standard_normal(hd))
    ang = rng.uniform(-9, 9, seq * half)
    cos, sin = b(np.cos(ang)), b(np.sin(ang))
    q, k, v = oracle.qkv_rope(qkv, qw, kw, cos, sin, seq, heads, hd, half,
                              grouped, 1e-5)
    eq, ek = _qkv_rope64(qkv, qw, kw, cos, sin, seq, heads, hd, half, grouped,
                         1e-5)
    assert within_one_rounding(q, eq, 1e-5 * (np.abs(eq) + 0.05))
    assert within_one_rounding(k, ek, 1e-5 * (np.abs(ek) + 0.05))
    x = qkv.reshape(seq, -1)
    vref = np.concatenate(
        [x[:, h * 3 * hd + 2 * hd: h * 3 * hd + 3 * hd] if grouped
         else x[:, 2 * heads * hd + h * hd: 2 * heads * hd + (h + 1) * hd]
         for h in range(heads)], axis=1)
    np.testing.assert_array_equal(v, vref.ravel())


def test_rope_identity_and_norm_preservation():
    seq, heads, hd, half = 4, 1, 128, 48
    qkv = b(rng.standard_normal(seq * 3 * hd))
    ones = b(np.ones(hd))
    q0, _, _ = oracle.qkv_rope(qkv, ones, ones, b(np.ones(seq * half)),
                               b(np.zeros(seq * half)), seq, heads, hd, half,
                               True, 0.0)
    qn, _, _ = oracle.qkv_rope(qkv, ones, ones, b(np.ones(seq * half)),
                               b(np.zeros(seq * half)), seq, heads, hd, 0,
                               True, 0.0)
    np.testing.assert_array_equal(q0, qn)       # angle 0 == no rotation
    ang = rng.uniform(-5, 5, seq * half)
    c, s = np.cos(ang), np.sin(ang)
    qr, _, _ = oracle.qkv_rope(qkv, ones, ones, b(c), b(s), seq, heads, hd,
                               half, True, 0.0)
    n0 = (f64(q0).reshape(seq, hd) ** 2).sum(1)
    n1 = (f64(qr).reshape(seq, hd) ** 2).sum(1)
    np.testing.assert_allclose(n1, n0, rtol=2e-2)   # rotation keeps norm


# ------------------------------------------------------------ attention

def _sdpa64(q, k, v, nq, nk, heads, hd, scale):
    qf = f64(q).reshape(nq, heads, hd)
    kf = f64(k).reshape(nk, heads, hd)
    vf = f64(v).reshape(nk, heads, hd)
    s = np.einsum("qhd,khd->hqk", qf, kf) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, vf).ravel()


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("round_p", [False, True])
def test_sdpa_against_float64(round_p, seed):
    """The oracle's SDPA against float64 softmax(QK^T s) V.  Rounding each
    P to bf16 (relative error at most 2^-9) moves an output by at most
    2^-9 sum_k p_k |v_k|; the output's own bf16 rounding adds 2^-9 |o|; f32
    accumulation stays far below both.  The bound is twice that, so a
    dropped scale, a transposed operand or a wrong max fails it."""
    r = np.random.default_rng(100 + seed)
    nq, nk, heads, hd = 9, 33, 2, 128
    q, k, v = (b(r.standard_normal(n * heads * hd)) for n in (nq, nk, nk))
    scale = 1 / math.sqrt(hd)
    got = f64(oracle.sdpa(q, k, v, nq, nk, heads, hd, scale,
                          round_p=round_p))
    exact = _sdpa64(q, k, v, nq, nk, heads, hd, scale)
    spread = _sdpa64(q, k, b(np.abs(f64(v))), nq, nk, heads, hd, scale)
    p_term = 2.0 ** -9 * spread if round_p else 0.0
    tol = 2.0 * (p_term + 2.0 ** -9 * np.abs(exact)) + 1e-6
    assert np.all(np.abs(got - exact) <= tol)
    # the bound has the power to see a 2% error in the scale
    wrong = _sdpa64(q, k, v, nq, nk, heads, hd, 1.02 * scale)
    assert np.any(np.abs(wrong - exact) > tol)


def test_sdpa_invariants():
    nq, nk, hd = 3, 50, 128
    q = b(rng.standard_normal(nq * hd))
    v = b(rng.standard_normal(nk * hd))
    k = np.tile(b(rng.standard_normal(hd)), nk)
    got = f64(oracle.sdpa(q, k, v, nq, nk, 1, hd, 0.1)).reshape(nq, hd)
    np.testing.assert_allclose(got, np.tile(f64(v).reshape(nk, hd).mean(0),
                                            (nq, 1)), atol=2e-2)
    # one key aligned with the query dominates: output = that value row
    kk = b(np.zeros(nk * hd)).reshape(nk, hd)
    kk[17] = b(np.full(hd, 4.0))
    qq = b(np.full(nq * hd, 4.0))
    got = oracle.sdpa(qq, kk.ravel(), v, nq, nk, 1, hd, 1.0).reshape(nq, hd)
    np.testing.assert_array_equal(got, np.tile(v.reshape(nk, hd)[17],
                                               (nq, 1)))
    hm = oracle.sdpa(q, k, v, nq, nk, 1, hd, 0.1, head_major=True)
    rm = oracle.sdpa(q, k, v, nq, nk, 1, hd, 0.1)
    np.testing.assert_array_equal(hm, rm)  # one head: both layouts coincide


# -------------------------------------------------- elementwise and MLP

def test_swiglu_gelu_silu_formulas():
    rows, width = 3, 100
    fused = b(3 * rng.standard_normal(rows * 2 * width))
    got = oracle.swiglu(fused, rows, width)
    fz = f64(fused).reshape(rows, 2 * width)
    g, u = fz[:, :width], fz[:, width:]
    exact = (g / (1 + np.exp(-g)) * u).ravel()
    assert within_one_rounding(got, exact, 1e-6 * np.abs(exact))
    assert np.all(f64(oracle.swiglu(b(np.zeros(2 * width)), 1, width)) == 0)
    x = b(np.linspace(-12, 12, 301))
    xf = f64(x)
    inner = 0.7978845608028654 * (xf + 0.044715 * xf ** 3)
    exact = np.where(inner <= -10, 0.0, np.where(inner >= 10, xf,
                     0.5 * xf * (1 + np.tanh(inner))))
    # the reference's f32 formula loses |x| * 2^-23 or so to the cancellation
    # in 1 + tanh(inner) for large negative x; allow that f32 error
    assert within_one_rounding(oracle.gelu(x), exact,
                               1e-6 * np.abs(exact) + np.abs(xf) * 2.0 ** -22)
    # a wrong cubic coefficient or the erf form would not pass:
    wrong = 0.5 * xf * (1 + np.tanh(0.7978845608028654 * (xf + 0.05 * xf ** 3)))
    assert not within_one_rounding(oracle.gelu(x), wrong,
                                   np.abs(xf) * 2.0 ** -22)
    assert within_one_rounding(oracle.silu(x), xf / (1 + np.exp(-xf)),
                               1e-6 * np.abs(xf))


def test_mlp_reference_tiny_shape():
    """tests/test_cuda_core.c:1071-1110 shape (rows 4, in 8, hidden 6,
    out 5): fc1 rows [0, hidden) are the gate, [hidden, 2 hidden) the up
    projection."""
    rows, d, hid, out = 4, 8, 6, 5
    x, fc1, fc2 = (b(s * rng.standard_normal(n)) for s, n in
                   ((1.0, rows * d), (0.5, 2 * hid * d), (0.5, out * hid)))
    got = oracle.linear(oracle.swiglu(oracle.linear(x, fc1, None, rows, d,
                                                    2 * hid), rows, hid),
                        fc2, None, rows, hid, out)
    # float64 restatement with the two bf16 boundaries of the GEMM path
    fz = f64(x).reshape(rows, d) @ f64(fc1).reshape(2 * hid, d).T
    fz = f64(b(fz.astype(np.float32)))
    g, u = fz[:, :hid], fz[:, hid:]
    act = f64(b((g / (1 + np.exp(-g)) * u).astype(np.float32)))
    exact = act @ f64(fc2).reshape(out, hid).T
    # a one-ulp flip of an intermediate (g, u or the activation) may
    # propagate: allow 4 bf16 ulps of the activations through fc2
    bound = np.abs(act) @ np.abs(f64(fc2).reshape(out, hid)).T * 2.0 ** -6
    assert within_one_rounding(got, exact.ravel(), bound.ravel())
    # gate and up swapped must not pass
    swapped = (u / (1 + np.exp(-u)) * g) @ f64(fc2).reshape(out, hid).T
    assert not within_one_rounding(got, swapped.ravel(), bound.ravel())


def test_euler_closed_form():
    """h3_cuda_dit.cu:536-548: x + delta (v + r (v - v_prev))."""
    s = rng.standard_normal(64).astype(np.float32)
    last, prev = b(rng.standard_normal(64)), b(rng.standard_normal(64))
    got = oracle.euler(s, last, prev, 0.125, -0.5)
    exact = s + 0.125 * (f64(last) - 0.5 * (f64(last) - f64(prev)))
    np.testing.assert_allclose(got, exact, rtol=2e-7, atol=1e-7)
    np.testing.assert_array_equal(oracle.euler(s, last, prev, 0.0, 1.0), s)


def test_final_head_formula():
    rows, width, n = 3, 64, 5
    x = b(rng.standard_normal(rows * width))
    nw = b(1 + 0.1 * rng.standard_normal(width))
    mod = b(0.3 * rng.standard_normal(2 * 2 * width))
    w, bias = b(0.2 * rng.standard_normal(n * width)), b(rng.standard_normal(n))
    rm = np.array([1, 0, 1], np.uint32)
    got, inv = oracle.adaln_linear(x, nw, mod, rm, w, bias, rows, width, n, 2,
                                   0, 1, 1e-5)
    normed = oracle.adaln(x, nw, mod, rm, rows, width, 2, 0, 1, 1e-5)
    np.testing.assert_array_equal(got, oracle.linear(normed, w, bias, rows,
                                                     width, n))
    xf = f64(x).reshape(rows, width)
    np.testing.assert_allclose(inv, 1 / np.sqrt((xf * xf).mean(1) + 1e-5),
                               rtol=1e-6)


def test_patch_linear_exact_and_mapped():
    rows, k, n = 4, 6, 5
    x = rng.integers(-3, 4, (rows, k)).astype(np.float32)
    w = rng.integers(-3, 4, (n, k)).astype(np.float32)
    bias = rng.integers(-2, 3, n).astype(np.float32)
    rm = np.array([3, 0, 5, 1], np.uint32)
    got = to_f32(oracle.patch_linear(x, w, bias, rows, k, n, row_map=rm,
                                     out_rows=6)).reshape(6, n)
    want = np.zeros((6, n), np.float32)
    want[rm] = x @ w.T + bias
    np.testing.assert_array_equal(got, want)


# ---------------------------------------------------- block composition

def test_h3_blocks_zero_gates_leave_residual():
    """With gate slots 2 and 5 at zero both residual updates vanish, so any
    number of H3 blocks returns the input bit for bit (h3_dit.c:2100-2177
    order: attention gate, MLP gate, fused next-block adaLN)."""
    rows, d, heads, ffn = 20, 256, 2, 256
    hd = 128
    x = b(rng.standard_normal(rows * d))

    def block():
        mod = 0.3 * rng.standard_normal((1, 3, 6, d))
        mod[:, :, 2] = 0
        mod[:, :, 5] = 0
        return {"norm1": b(np.ones(d)), "norm2": b(np.ones(d)),
                "qkv": b(0.05 * rng.standard_normal(3 * heads * hd * d)),
                "q_norm": b(np.ones(hd)), "k_norm": b(np.ones(hd)),
                "out": b(0.05 * rng.standard_normal(d * heads * hd)),
                "fc1": b(0.05 * rng.standard_normal(2 * ffn * d)),
                "fc2": b(0.05 * rng.standard_normal(d * ffn)),
                "modulation": b(mod.ravel())}
    ang = rng.uniform(-3, 3, rows * 48)
    out = oracle.h3_blocks(x, [block(), block()], np.zeros(rows, np.uint32),
                           b(np.cos(ang)), b(np.sin(ang)), rows, d, heads,
                           ffn)
    np.testing.assert_array_equal(out, x)


def _wiring_block(d, heads, ffn, T, mode, mod_seed):
    """One H3 block whose weights make one branch a closed form of its adaLN
    input (hidden = heads * 128, ffn = hidden):
      mode "attn": q and k projections 0 (uniform softmax), v projection and
        out-projection the identity, so the attention branch returns the row
        mean of its adaLN output; attention gate 1, MLP gate 0;
      mode "mlp": attention gate 0, fc1 = [4 I ; I] (gate rows, up rows),
        fc2 = I, so the MLP branch is swiglu([4 a, a]) of its adaLN output a;
        MLP gate 1;
      mode "skip": both gates 0 (the block returns its input).
    norm1, norm2 and all modulation slots are distinct random values."""
    r = np.random.default_rng(mod_seed)
    hd = 128
    inner = heads * hd
    mod = 0.5 * r.standard_normal((T, 3, 6, d))
    mod[:, :, 2] = 1.0 if mode == "attn" else 0.0
    mod[:, :, 5] = 1.0 if mode == "mlp" else 0.0
    qkv = np.zeros((heads, 3, hd, d))
    for h in range(heads):
        qkv[h, 2, :, h * hd:(h + 1) * hd] = np.eye(hd)
    fc1 = np.concatenate([4.0 * np.eye(ffn, d), np.eye(ffn, d)])
    return {"norm1": b(1.0 + 0.5 * r.standard_normal(d)),
            "norm2": b(1.0 + 0.5 * r.standard_normal(d)),
            "qkv": b(qkv.ravel()), "q_norm": b(np.ones(hd)),
            "k_norm": b(np.ones(hd)), "out": b(np.eye(d, inner).ravel()),
            "fc1": b(fc1.ravel()), "fc2": b(np.eye(d, ffn).ravel()),
            "modulation": b(mod.ravel())}


def _wiring_setup(rows=24, d=256, heads=2, T=3):
    r = np.random.default_rng(77)
    x = b(r.standard_normal(rows * d))
    row_map = r.integers(0, 3 * T, rows).astype(np.uint32)
    ang = r.uniform(-3, 3, rows * 48)
    return x, row_map, b(np.cos(ang)), b(np.sin(ang))


def _attn_closed_form(x, w, row_map, rows, d, shift, scale, norm):
    """x + mean over rows of adaln(x; norm, slots shift/scale), the value the
    "attn" wiring block must produce, in float64."""
    a = oracle.adaln(x, w[norm], w["modulation"], row_map, rows, d, 6, shift,
                     scale, 1e-5)
    y = f64(a).reshape(rows, d).mean(axis=0)
    return f64(x).reshape(rows, d) + y[None, :], y


def _assert_attn_wiring(got, x, w, row_map, rows, d):
    want, y = _attn_closed_form(x, w, row_map, rows, d, 0, 1, "norm1")
    g = f64(got).reshape(rows, d)
    # bf16 rounding of the mean and of the residual sum
    tol = 2.0 ** -8 * (np.abs(y)[None, :] + np.abs(want)) + 1e-30
    assert (np.abs(g - want) <= tol).all(), float(np.abs(g - want).max())
    # the check has the power to see a swapped slot pair or norm weight
    for shift, scale, norm in ((1, 0, "norm1"), (0, 1, "norm2"),
                               (3, 4, "norm1")):
        wrong, _ = _attn_closed_form(x, w, row_map, rows, d, shift, scale,
                                     norm)
        assert (np.abs(g - wrong) > tol).any()


def test_h3_block_attention_branch_wiring():
    """The attention branch reads adaLN(x; norm1, shift slot 0, scale slot 1)
    of the block's own modulation row (row_map[r]) and is added through gate
    slot 2 (h3_dit.c:2030-2032 adaLN, :2100-2105 gate).  With q = k = 0 and
    identity v / out projections the branch is the row mean of that adaLN
    output, so the block output is x + mean(adaLN(x)) up to two bf16
    roundings; slots 1/0, norm2 or slots 3/4 in its place fail."""
    rows, d, heads = 24, 256, 2
    x, row_map, cos, sin = _wiring_setup(rows, d, heads)
    w = _wiring_block(d, heads, d, 3, "attn", 5)
    got = oracle.h3_blocks(x, [w], row_map, cos, sin, rows, d, heads, d)
    _assert_attn_wiring(got, x, w, row_map, rows, d)


def test_h3_block_mlp_branch_wiring():
    """The MLP branch reads adaLN(x; norm2, shift slot 3, scale slot 4) and
    is added through gate slot 5 (h3_dit.c:2100-2105 gate + adaLN,
    :2139-2177 MLP gate).  With the attention gate at 0 and fc1 = [4I ; I],
    fc2 = I the block output is gate(x, swiglu([4a, a]), slot 5) with
    a = adaLN(x) -- bit for bit, since every step in between is exact; slots
    4/3, norm1 or slots 0/1 in its place fail."""
    rows, d, heads = 24, 256, 2
    x, row_map, cos, sin = _wiring_setup(rows, d, heads)
    w = _wiring_block(d, heads, d, 3, "mlp", 6)
    got = oracle.h3_blocks(x, [w], row_map, cos, sin, rows, d, heads, d)

    def closed(shift, scale, norm):
        a = oracle.adaln(x, w[norm], w["modulation"], row_map, rows, d, 6,
                         shift, scale, 1e-5).reshape(rows, d)
        fused = np.concatenate([b(4.0 * f64(a)), a], axis=1)
        m = oracle.swiglu(fused.ravel(), rows, d)
        return oracle.gate(x, m, w["modulation"], row_map, rows, d, 6, 5)

    np.testing.assert_array_equal(got, closed(3, 4, "norm2"))
    for wrong in ((4, 3, "norm2"), (3, 4, "norm1"), (0, 1, "norm2")):
        assert not np.array_equal(got, closed(*wrong))


def test_h3_blocks_fused_adaln_takes_the_next_blocks_weights():
    """The MLP gate of block i is fused with block i+1's attention adaLN,
    which must use block i+1's norm1 and modulation (h3_dit.c:2139-2178).
    Block 0 is a pass-through (both gates 0, so its output is its input bit
    for bit) with its own distinct norm1 / modulation; block 1 is the
    attention-wiring block.  The two-block output must be the closed form of
    block 1 alone; block 0's weights in the fused adaLN fail it."""
    rows, d, heads = 24, 256, 2
    x, row_map, cos, sin = _wiring_setup(rows, d, heads)
    w0 = _wiring_block(d, heads, d, 3, "skip", 8)
    w1 = _wiring_block(d, heads, d, 3, "attn", 9)
    got = oracle.h3_blocks(x, [w0, w1], row_map, cos, sin, rows, d, heads, d)
    _assert_attn_wiring(got, x, w1, row_map, rows, d)
    wrong, y = _attn_closed_form(x, w0, row_map, rows, d, 0, 1, "norm1")
    tol = 2.0 ** -8 * (np.abs(y)[None, :] + np.abs(wrong))
    assert (np.abs(f64(got).reshape(rows, d) - wrong) > tol).any()


# ------------------------------------------------- Wan block composition
#
# The Wan-style block (BASELINE's benchmark block) has no counterpart in the
# reference; its specification is the Wan 2.x block order: self-attention on
# LayerNorm(x)(1 + slot 1) + slot 0 gated by slot 2, cross-attention on
# norm3(x) (a LayerNorm with its own affine) added without a gate, and the
# GELU-tanh FFN on LayerNorm(x)(1 + slot 4) + slot 3 gated by slot 5.  Its
# primitives are the reference's LayerNorm (h3_cuda_core.cu:250-295), gate
# (h3_cuda_dit.cu:261-276) and GELU-tanh (h3_cuda_core.cu:139-158), each
# pinned above.  The tests below build weights that reduce one branch of
# oracle.wan_block to a closed form of its input, with every modulation slot
# a distinct random value, so that a swapped slot, norm or branch fails.

WAN_EPS = 1e-6


def _wan_setup(rows=24, d=256, T=3, text_rows=8, seed=78):
    r = np.random.default_rng(seed)
    # a large per-row offset: LayerNorm removes it, a per-head RMS does not
    x = b(r.standard_normal((rows, d)) + 3.0 * r.standard_normal((rows, 1)))
    ctx = b(r.standard_normal(text_rows * d))
    row_map = r.integers(0, 3 * T, rows).astype(np.uint32)
    ang = r.uniform(-3, 3, rows * 48)
    return x.ravel(), ctx, row_map, b(np.cos(ang)), b(np.sin(ang))


def _wan_wiring_block(d, heads, ffn, T, seed, self_attn=False, cross=False,
                      ffn_on=False):
    """Weights of one Wan block (hidden = heads * 128) whose branches are
    closed forms of their inputs:
      self_attn: q = k = 0 (uniform softmax), v and out projections the
        identity, so the branch is the row mean of its adaLN output;
        otherwise out = 0, so the branch is exactly 0;
      cross: cq, ck, cv and co projections the identity (no bias), so the
        branch is SDPA(head_rms(norm3(x)), head_rms(ctx), ctx); otherwise
        co = 0;
      ffn_on: fc1 = fc2 = I (ffn = hidden), so the branch is gelu(a) of its
        adaLN output a; otherwise fc2 = 0.
    Modulation slots, norm3's weight and bias are distinct random values;
    every bias not named is 0."""
    r = np.random.default_rng(seed)
    hd = 128
    inner = heads * hd
    assert inner == d and ffn == d
    mod = 0.5 * r.standard_normal((T, 3, 6, d))
    eye = np.eye(d)
    zero = np.zeros((d, d))
    qkv = np.concatenate([zero, zero, eye if self_attn else zero])
    return {
        "modulation": b(mod.ravel()),
        "qkv": b(qkv.ravel()), "qkv_bias": b(np.zeros(3 * inner)),
        "q_norm": b(np.ones(hd)), "k_norm": b(np.ones(hd)),
        "out": b((eye if self_attn else zero).ravel()),
        "out_bias": b(np.zeros(d)),
        "norm3": b(1.0 + 0.5 * r.standard_normal(d)),
        "norm3_bias": b(0.5 * r.standard_normal(d)),
        "cq": b(eye.ravel()), "cq_bias": b(np.zeros(inner)),
        "cq_norm": b(np.ones(hd)),
        "ck": b(eye.ravel()), "ck_bias": b(np.zeros(inner)),
        # key rms 2: logits of order 1-2, so p varies over (0.1, 0.9)
        "ck_norm": b(2.0 * np.ones(hd)),
        "cv": b(eye.ravel()), "cv_bias": b(np.zeros(inner)),
        "co": b((eye if cross else zero).ravel()), "co_bias": b(np.zeros(d)),
        "fc1": b(eye.ravel()), "fc1_bias": b(np.zeros(ffn)),
        "fc2": b((eye if ffn_on else zero).ravel()),
        "fc2_bias": b(np.zeros(d)),
    }


def _run_wan(x, ctx, w, row_map, cos, sin, rows, text_rows, d, heads):
    return oracle.wan_block(x, ctx, w, row_map, cos, sin, rows, text_rows, d,
                            heads, d, eps=WAN_EPS)


def _mod_slot(w, row_map, d, slot):
    """[rows][d] float64 of modulation slot `slot` at each row's time row."""
    mod = f64(w["modulation"]).reshape(-1, 6, d)
    return mod[row_map.astype(np.int64), slot]


def test_wan_block_self_attention_branch_wiring():
    """Self-attention reads LayerNorm(x)(1 + slot 1) + slot 0 (no affine) of
    the row's own modulation row and is added through gate slot 2.  With
    q = k = 0 and identity v / out the branch is the row mean y of that
    adaLN output, so the block returns x + slot2 * y up to the bf16 rounding
    of y and of the sum; slots 1/0, 3/4, gate slot 5 or norm3's affine in
    their place fail."""
    rows, d, heads, T = 24, 256, 2, 3
    x, ctx, row_map, cos, sin = _wan_setup(rows, d, T)
    w = _wan_wiring_block(d, heads, d, T, 11, self_attn=True)
    got = f64(_run_wan(x, ctx, w, row_map, cos, sin, rows, 8, d, heads))
    got = got.reshape(rows, d)

    def closed(shift, scale, gate_slot, affine=False):
        a = oracle.layer_adaln(x, w["norm3"] if affine else None,
                               w["norm3_bias"] if affine else None,
                               w["modulation"], row_map, rows, d, 6, shift,
                               scale, WAN_EPS)
        y = f64(a).reshape(rows, d).mean(axis=0)[None, :]
        g = _mod_slot(w, row_map, d, gate_slot)
        return f64(x).reshape(rows, d) + g * y, np.abs(g * y)

    want, gy = closed(0, 1, 2)
    tol = 2.0 ** -8 * (gy + np.abs(want)) + 1e-30
    assert (np.abs(got - want) <= tol).all(), float(np.abs(got - want).max())
    for wrong in ((1, 0, 2), (3, 4, 2), (0, 1, 5), (0, 1, 2, True)):
        other, _ = closed(*wrong)
        assert (np.abs(got - other) > tol).any(), wrong


def test_wan_block_cross_attention_reads_norm3_and_is_ungated():
    """Cross-attention's Q projection reads norm3(x) = LayerNorm(x) * w3 + b3
    (no modulation) and its output is added to the residual without a gate.
    With identity projections and two text rows, the second all zero, each
    head's attention is p * v0 with p = sigmoid(scale * q_h . k0_h), q the
    per-head RMS of norm3(x) and k0 that of the first text row, so the block
    returns x + p * v0 in closed form (float64 after the pinned primitives,
    within the bf16 roundings of P, O and the sum).  Q read from x,
    LayerNorm without the affine, or adaLN slots 0/1, or the residual gated
    by slot 2 or 5, all fail."""
    rows, d, heads, T, text = 24, 256, 2, 3, 2
    hd = 128
    x, ctx, row_map, cos, sin = _wan_setup(rows, d, T, text_rows=text)
    ctx = ctx.reshape(text, d).copy()
    ctx[1] = 0
    ctx = ctx.ravel()
    w = _wan_wiring_block(d, heads, d, T, 12, cross=True)
    got = f64(_run_wan(x, ctx, w, row_map, cos, sin, rows, text, d, heads))
    got = got.reshape(rows, d)
    k0 = f64(oracle.head_rms_norm(ctx[:d], w["ck_norm"], 1, heads, hd,
                                  WAN_EPS)).reshape(heads, hd)
    v0 = f64(ctx[:d]).reshape(heads, hd)
    scale = 1.0 / math.sqrt(hd)

    def closed(qin, gate_slot=None):
        q = f64(oracle.head_rms_norm(qin, w["cq_norm"], rows, heads, hd,
                                     WAN_EPS)).reshape(rows, heads, hd)
        p = 1.0 / (1.0 + np.exp(-scale * np.einsum("rhd,hd->rh", q, k0)))
        o = (p[:, :, None] * v0[None]).reshape(rows, d)
        if gate_slot is not None:
            o = o * _mod_slot(w, row_map, d, gate_slot)
        return f64(x).reshape(rows, d) + o, np.abs(o)

    norm3 = oracle.layer_adaln(x, w["norm3"], w["norm3_bias"], None, None,
                               rows, d, 6, 0, 0, WAN_EPS)
    want, o = closed(norm3)
    tol = 2.0 ** -7 * o + 2.0 ** -8 * np.abs(want) + 1e-30
    assert (np.abs(got - want) <= tol).all(), float(np.abs(got - want).max())
    plain_ln = oracle.layer_adaln(x, None, None, None, None, rows, d, 6, 0, 0,
                                  WAN_EPS)
    modulated = oracle.layer_adaln(x, None, None, w["modulation"], row_map,
                                   rows, d, 6, 0, 1, WAN_EPS)
    for name, other in (("x", closed(x)), ("no affine", closed(plain_ln)),
                        ("slots 0/1", closed(modulated)),
                        ("gate 2", closed(norm3, 2)),
                        ("gate 5", closed(norm3, 5))):
        assert (np.abs(got - other[0]) > tol).any(), name


def test_wan_block_cross_attention_constant_keys_give_mean_of_values():
    """With the key projection 0 and a constant key bias every text key is
    the same, so the cross-attention of every row is the mean of the text
    values, added ungated through co = I: the block returns x + mean(ctx)
    up to the bf16 rounding of the mean and of the sum, whatever Q is."""
    rows, d, heads, T, text = 24, 256, 2, 3, 8
    x, ctx, row_map, cos, sin = _wan_setup(rows, d, T, text_rows=text)
    w = _wan_wiring_block(d, heads, d, T, 13, cross=True)
    w["ck"] = b(np.zeros(d * d))
    w["ck_bias"] = b(np.random.default_rng(5).standard_normal(d))
    got = f64(_run_wan(x, ctx, w, row_map, cos, sin, rows, text, d, heads))
    y = f64(ctx).reshape(text, d).mean(axis=0)[None, :]
    want = f64(x).reshape(rows, d) + y
    tol = 2.0 ** -8 * (np.abs(y) + np.abs(want))
    assert (np.abs(got.reshape(rows, d) - want) <= tol).all()


def test_wan_block_ffn_branch_wiring():
    """The FFN reads LayerNorm(x)(1 + slot 4) + slot 3 and is added through
    gate slot 5.  With the other two branches 0 (bit-exact pass-throughs)
    and fc1 = fc2 = I the block returns gate(x, gelu(a), slot 5) bit for
    bit; slots 4/3, 0/1, gate slot 2 or norm3's affine fail."""
    rows, d, heads, T = 24, 256, 2, 3
    x, ctx, row_map, cos, sin = _wan_setup(rows, d, T)
    w = _wan_wiring_block(d, heads, d, T, 14, ffn_on=True)
    got = _run_wan(x, ctx, w, row_map, cos, sin, rows, 8, d, heads)

    def closed(shift, scale, gate_slot, affine=False):
        a = oracle.layer_adaln(x, w["norm3"] if affine else None,
                               w["norm3_bias"] if affine else None,
                               w["modulation"], row_map, rows, d, 6, shift,
                               scale, WAN_EPS)
        return oracle.gate(x, oracle.gelu(a), w["modulation"], row_map, rows,
                           d, 6, gate_slot)

    np.testing.assert_array_equal(got, closed(3, 4, 5))
    for wrong in ((4, 3, 5), (0, 1, 5), (3, 4, 2), (3, 4, 5, True)):
        assert not np.array_equal(got, closed(*wrong)), wrong


def test_wan_block_all_branches_off_is_identity():
    """out = co = fc2 = 0 (zero biases): every branch adds an exact zero, so
    the block returns its input bit for bit."""
    rows, d, heads, T = 24, 256, 2, 3
    x, ctx, row_map, cos, sin = _wan_setup(rows, d, T)
    w = _wan_wiring_block(d, heads, d, T, 15)
    got = _run_wan(x, ctx, w, row_map, cos, sin, rows, 8, d, heads)
    np.testing.assert_array_equal(got, x)


def test_rope_rotate_pins():
    """RoPE rotation alone (h3_cuda_attention.cu:218-233): angle 0 is the
    identity, angle pi/2 maps (x, y) to (-y, x) exactly, dims from 96 on are
    copied, the pair norm is kept to bf16 rounding, and on rows whose
    per-head RMS is exactly 1 with unit norm weights it equals the rotation
    step of oracle.qkv_rope."""
    rows, heads, hd = 6, 2, 128
    x = b(rng.standard_normal(rows * heads * hd))
    one, zero = b(np.ones(rows * 48)), b(np.zeros(rows * 48))
    np.testing.assert_array_equal(
        oracle.rope_rotate(x, one, zero, rows, heads), x)
    r = f64(oracle.rope_rotate(x, zero, one, rows, heads)).reshape(
        rows, heads, hd)
    xf = f64(x).reshape(rows, heads, hd)
    np.testing.assert_array_equal(r[..., :48], -xf[..., 48:96])
    np.testing.assert_array_equal(r[..., 48:96], xf[..., :48])
    np.testing.assert_array_equal(r[..., 96:], xf[..., 96:])
    ang = rng.uniform(-7, 7, rows * 48)
    c, s = b(np.cos(ang)), b(np.sin(ang))
    r = f64(oracle.rope_rotate(x, c, s, rows, heads)).reshape(rows, heads, hd)
    n0 = xf[..., :48] ** 2 + xf[..., 48:96] ** 2
    n1 = r[..., :48] ** 2 + r[..., 48:96] ** 2
    cs = (f64(c) ** 2 + f64(s) ** 2).reshape(rows, 1, 48)
    assert np.allclose(n1, n0 * cs, rtol=2 ** -6, atol=1e-6)
    # rows of +-1 have RMS exactly 1, so qkv_rope's norm is the identity
    sign = b(np.where(rng.standard_normal(rows * heads * hd) < 0, -1.0, 1.0))
    qkv = np.concatenate([sign.reshape(rows, heads * hd)] * 3,
                         axis=1).ravel()
    qn, _, _ = oracle.qkv_rope(qkv, b(np.ones(hd)), b(np.ones(hd)), c, s,
                               rows, heads, hd, 48, False, 0.0)
    np.testing.assert_array_equal(
        oracle.rope_rotate(sign, c, s, rows, heads), qn)


def test_bf16_rounding_is_rne():
    """RNE ties: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> even (1);
    1 + 3 * 2^-8 -> 1 + 2^-6 (even mantissa)."""
    vals = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 1e-40,
                     65504.0], np.float32)
    got = to_f32(b(vals))
    assert got[0] == 1.0 and got[1] == 1 + 2 ** -6 and got[2] == -1.0
    assert bf16_ulp_distance(b(vals[3:4]), b(np.float32(1e-40))) == 0


def test_token_pool_expand_pins():
    """Token reduction oracle (h3_cuda_dit.cu:336-470): a singleton pair
    copies its row; a pair of small integers pools to their exact mean;
    expanding an unchanged stack (reduced == baseline, scale 1) restores the
    original grid bit for bit; scale 0 returns the original rows; exact
    prefix rows take the reduced row."""
    width, input_rows = 8, 5
    x = rng.integers(-8, 9, (input_rows, width)).astype(np.float32) * 2
    pairs = np.array([0, 3, 1, 1, 2, 4], np.uint32)        # rows 0..2
    bidx = np.array([0, 0xFFFFFFFF, 1], np.uint32)
    out, orig, base = oracle.token_pool(b(x), pairs, bidx, input_rows, 3, 2,
                                        width)
    o = f64(out).reshape(3, width)
    np.testing.assert_array_equal(o[0], (x[0] + x[3]) / 2)
    np.testing.assert_array_equal(o[1], x[1])
    np.testing.assert_array_equal(o[2], (x[2] + x[4]) / 2)
    np.testing.assert_array_equal(f64(orig).reshape(input_rows, width), x)
    np.testing.assert_array_equal(f64(base).reshape(2, width),
                                  o[[0, 2]])
    parents = np.array([0, 1, 2, 0, 2], np.uint32)
    same = oracle.token_expand(orig, out, base, bidx, parents, input_rows,
                               width, 0, 1.0)
    # rows with a baseline return the original; row 1 has none -> reduced
    want = f64(orig).reshape(input_rows, width).copy()
    want[1] = o[1]
    np.testing.assert_array_equal(f64(same).reshape(input_rows, width), want)
    moved = b(f64(out) + 1.0)
    zero = oracle.token_expand(orig, moved, base, bidx, parents, input_rows,
                               width, 2, 0.0)
    z = f64(zero).reshape(input_rows, width)
    np.testing.assert_array_equal(z[0], f64(moved).reshape(3, width)[0])
    np.testing.assert_array_equal(z[2:], want[2:] * 0 +
                                  f64(orig).reshape(input_rows, width)[2:])


# ------------------------------------------------------ sampler and refiner

def test_reuse_schedule_and_ratio_literals():
    """oracle.reuse_schedule against the reference's literals
    (tests/test_h3.c:128-147) and the ratio's clamp (h3_dit.c:2644-2655)."""
    sel = oracle.reuse_schedule(20, 3)
    assert [s for s in range(20) if sel[s]] == [0, 3, 6, 9, 12, 15, 18, 19]
    assert sum(oracle.reuse_schedule(20, 2)) == 11
    assert sum(oracle.reuse_schedule(50, 3)) == 18
    assert all(oracle.reuse_schedule(20, 1))
    r = oracle.extrapolation_ratio
    assert r(0.5, 0.6, 0.7, True) == pytest.approx(1.0)
    assert r(0.5, 0.6, 0.7, False) == 0.0
    assert r(0.5, 0.6, 0.6, True) == 0.0
    assert r(0.0, 0.6, 0.65, True) == 2.0 and r(1.0, 0.6, 0.65, True) == -2.0


def _denoise_with_velocity(monkeypatch, velocity, sigmas, reuse):
    """oracle.h3_denoise with the forward replaced by velocity(sigma)."""
    nv, na = 6, 4
    m = dict(video_patch=2, audio_channels=2, video_conditions=1,
             audio_conditions=0,
             video_input=np.linspace(-1, 1, 2 * (nv // 2 + 1)).astype(
                 np.float32),
             audio_input=np.linspace(2, 3, na).astype(np.float32))

    def forward(mm, step):
        v = velocity(sigmas[step])
        return b(np.full(nv, v)), b(np.full(na, -v))

    monkeypatch.setattr(oracle, "h3_forward_step", forward)
    return m, oracle.h3_denoise(m, sigmas, sigmas, reuse)


def test_denoise_loop_constant_velocity(monkeypatch):
    """Constant v: every step, fresh or extrapolated, moves x by
    (sigma_i - sigma_i+1) v, so x_N = x_0 + (sigma_0 - sigma_N) v; the
    condition rows ahead of the targets are untouched."""
    sig = np.linspace(1.0, 0.0, 11).astype(np.float32)
    for reuse in (1, 2, 3):
        m, (video, audio, n) = _denoise_with_velocity(
            monkeypatch, lambda s: 0.75, sig, reuse)
        assert n == sum(oracle.reuse_schedule(10, reuse))
        v0, a0 = m["video_input"], m["audio_input"]
        assert np.array_equal(video[:2], v0[:2])
        np.testing.assert_allclose(video[2:], v0[2:] + 0.75, atol=2e-6)
        np.testing.assert_allclose(audio, a0 - 0.75, atol=2e-6)


def test_denoise_extrapolation_is_exact_for_linear_velocity(monkeypatch):
    """v(sigma) = sigma: the reuse extrapolation v_last + r (v_last - v_prev)
    with r = (s - s_last) / (s_last - s_prev) reproduces v(s) on skipped
    steps, except the first skipped step, which has no previous evaluation
    and holds v(s_0) (ratio 0).  So reuse 2 lands where evaluating every
    step does plus that one step's (s_1 - s_2)(s_0 - s_1), to bf16 rounding
    of the velocities, and every-step evaluation follows
    sum (s_i - s_i+1) s_i.  A wrong sign of r, a stale v_prev or the wrong
    sigma pair fails this."""
    sig = np.linspace(1.0, 0.0, 9).astype(np.float32)
    _, (v_all, _, n1) = _denoise_with_velocity(monkeypatch, lambda s: s, sig,
                                                1)
    _, (v_re, _, n2) = _denoise_with_velocity(monkeypatch, lambda s: s, sig,
                                               2)
    assert (n1, n2) == (8, 5)
    exact = sum((sig[i] - sig[i + 1]) * sig[i] for i in range(8))
    x0 = np.linspace(-1, 1, 8).astype(np.float32)[2:]
    np.testing.assert_allclose(v_all[2:], x0 + exact, atol=4e-3)
    first_hold = (sig[1] - sig[2]) * (sig[0] - sig[1])
    np.testing.assert_allclose(v_re[2:], v_all[2:] + first_hold, atol=4e-3)
    # no reuse at all would drift: constant-hold of the last velocity
    held = sum((sig[i] - sig[i + 1]) * sig[i - (i % 2)] for i in range(8))
    assert abs(held - exact) > 0.02


def test_refiner_with_zero_branches_is_norm_of_projection():
    """Zero out-projection and fc2 weights make both residual branches add
    exact zeros, so refine_text reduces to the final RMSNorm of the biased
    condition projection (h3_dit.c:851-866), bit for bit; nonzero branches
    must change it."""
    rows, td, d, heads, ffn = 5, 64, 256, 2, 128
    r = np.random.default_rng(9)
    w = {"condition_w": b(r.standard_normal(d * td) * 0.1),
         "condition_b": b(r.standard_normal(d) * 0.1),
         "final_norm": b(1 + 0.05 * r.standard_normal(d))}
    blocks = []
    for _ in range(2):
        blocks.append({
            "norm1": b(1 + 0.05 * r.standard_normal(d)),
            "qkv": b(r.standard_normal(3 * 256 * d) * 0.05),
            "q_norm": b(np.ones(128)), "k_norm": b(np.ones(128)),
            "out": b(np.zeros(d * 256)),
            "norm2": b(1 + 0.05 * r.standard_normal(d)),
            "fc1": b(r.standard_normal(2 * ffn * d) * 0.05),
            "fc2": b(np.zeros(d * ffn))})
    w["blocks"] = blocks
    src = b(r.standard_normal(rows * td))
    got = oracle.refine_text(src, w, rows, td, d, heads, ffn)
    proj = oracle.linear(src, w["condition_w"], w["condition_b"], rows, td, d)
    assert np.array_equal(got, oracle.rms_norm(proj, w["final_norm"], rows,
                                               d, 1e-5))
    blocks[1]["fc2"] = b(r.standard_normal(d * ffn) * 0.05)
    assert not np.array_equal(
        oracle.refine_text(src, w, rows, td, d, heads, ffn), got)
