"""Shared test setup: import paths, the `gpu` marker, the GPU context and the
comparison helpers used by the parity tests."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "h3.c_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs the HIP backend)")


@pytest.fixture(scope="session")
def gpu():
    import h3hip
    g = h3hip.Gpu()
    yield g
    g.close()


def bf16_ulp_distance(a, b):
    """Distance in bf16 representable steps between two bf16 bit arrays."""
    a = np.asarray(a, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b, dtype=np.uint16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    ma = np.where(a & 0x8000, -(a & 0x7FFF), a & 0x7FFF)
    mb = np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(ma - mb)


def assert_ulp(got, want, max_ulp=1, what=""):
    d = bf16_ulp_distance(got, want)
    worst = int(d.max()) if d.size else 0
    bad = int((d > max_ulp).sum())
    assert bad == 0, f"{what}: {bad} values beyond {max_ulp} ulp (worst {worst})"


def to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32)
            << 16).view(np.float32)


def assert_close(got_bits, want_bits, atol=1e-3, rtol=1e-2, what="",
                 chained=0, extra_abs=None):
    """The reference's GEMM / flash tolerance: |g - r| <= atol + rtol |r|
    (tests/test_cuda_dit.c:73-91, tests/test_cuda_attention.c:79-114).

    chained = number of extra bf16 rounding boundaries inside the op (the
    SwiGLU/GELU activation between two GEMMs).  Where the two sides round an
    intermediate to neighbouring bf16 values, that one-ulp flip propagates
    through the following GEMM; the bound then grows by
    chained * 4 * 2^-8 * rms(reference)."""
    g = to_f32(got_bits).astype(np.float64)
    r = to_f32(want_bits).astype(np.float64)
    err = np.abs(g - r)
    extra = chained * 4 * 2.0 ** -8 * np.sqrt(np.mean(r * r)) if r.size else 0
    if extra_abs is not None:
        extra = extra + np.asarray(extra_abs, dtype=np.float64).reshape(-1)
    bad = err > atol + rtol * np.abs(r) + extra
    assert not np.isnan(g).any(), f"{what}: NaN in output"
    assert int(bad.sum()) == 0, (
        f"{what}: {int(bad.sum())}/{g.size} beyond tolerance, "
        f"max err {err.max():.3g}")


def sdpa_p_rounding_bound(q, k, v, q_rows, kv_rows, heads, hd, scale,
                          head_major=False):
    """Per-output bound on what rounding P to bf16 can move an attention
    output: flash kernels round P relative to their own running maximum
    (a tile's, or a stale one within 2^8), the oracle relative to the row's
    global maximum; the two roundings of one P differ by at most one bf16
    ulp, 2^-8 relative, so |O_a - O_b| <= 2^-8 sum_j p_j |v_j| / sum_j p_j.
    Computed in float64 from the bf16 inputs."""
    Q = to_f32(q).astype(np.float64).reshape(q_rows, heads, hd)
    K = to_f32(k).astype(np.float64).reshape(kv_rows, heads, hd)
    V = np.abs(to_f32(v).astype(np.float64).reshape(kv_rows, heads, hd))
    s = np.einsum("qhd,khd->hqk", Q, K) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    b = 2.0 ** -8 * np.einsum("hqk,khd->hqd", p, V)
    return b if head_major else b.transpose(1, 0, 2)


def cosine_rel_l2(got_bits, want_bits):
    g = to_f32(got_bits).astype(np.float64)
    r = to_f32(want_bits).astype(np.float64)
    cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-300))
    rel = float(np.linalg.norm(g - r) / (np.linalg.norm(r) + 1e-300))
    return cos, rel


def rand_bf16(rng, n, scale=1.0, mean=0.0):
    import oracle
    return oracle.bf16((mean + scale * rng.standard_normal(n)).astype(
        np.float32))


def assert_row_close(got, want, terms, what="", ulps=1, rel=2.0 ** -17):
    """Row-op check: |g - r| <= ulps bf16 ulps of max(|g|, |r|)
    + rel * terms, where `terms` is the magnitude of the f32 operands that
    are summed into each output (e.g. |n (1 + scale)| + |shift| for adaLN).
    The second term bounds the effect of the device's f32 reduction order on
    the row statistic: near-cancelling outputs make that effect many bf16
    ulps of a small result while staying tiny against the operands."""
    g = to_f32(got).astype(np.float64)
    r = to_f32(want).astype(np.float64)
    mag = np.maximum(np.abs(g), np.abs(r))
    ulp = np.ldexp(1.0, np.frexp(np.where(mag > 0, mag, 1e-38))[1] - 8)
    bound = ulps * ulp + rel * np.asarray(terms, dtype=np.float64)
    err = np.abs(g - r)
    bad = err > bound
    assert not np.isnan(g).any(), f"{what}: NaN"
    assert int(bad.sum()) == 0, (
        f"{what}: {int(bad.sum())}/{g.size} beyond bound; worst excess "
        f"{float((err - bound).max()):.3g}")


def adaln_terms(x, w, mod, row_map, rows, width, slots, shift_slot,
                scale_slot, eps, layer=False, bias=None):
    """|n (1 + scale)| + |b (1 + scale)| + |shift| per output, float64."""
    xf = to_f32(x).astype(np.float64).reshape(rows, width)
    if layer:
        mean = xf.mean(axis=1, keepdims=True)
        inv = 1.0 / np.sqrt(((xf - mean) ** 2).mean(axis=1, keepdims=True)
                            + eps)
        n = (np.abs(xf) + np.abs(mean)) * inv
    else:
        inv = 1.0 / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + eps)
        n = np.abs(xf) * inv
    if w is not None:
        n = n * np.abs(to_f32(w).astype(np.float64))[None, :]
    if bias is not None:
        n = n + np.abs(to_f32(bias).astype(np.float64))[None, :]
    if mod is None:
        return n.ravel()
    m = to_f32(mod).astype(np.float64).reshape(-1, slots, width)
    rm = np.asarray(row_map)
    sc = m[rm, scale_slot, :]
    sh = m[rm, shift_slot, :]
    return (n * np.abs(1.0 + sc) + np.abs(sh)).ravel()
