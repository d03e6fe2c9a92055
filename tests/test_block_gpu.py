"""Block-level parity: the DiT driver (h3hip_dit.c, run through the C ABI)
against the oracle's restatement of the reference block order, on identical
seeded weights and inputs.

Bar: per-block hidden state cosine >= 0.999 and
relative L2 <= 1e-2 against the CPU reference.
"""
import numpy as np
import pytest

from conftest import cosine_rel_l2

pytestmark = pytest.mark.gpu

import h3hip  # noqa: E402
import oracle  # noqa: E402

H3_NAMES = ["norm1", "norm2", "qkv", "q_norm", "k_norm", "out", "fc1", "fc2",
            "modulation"]
WAN_NAMES = ["norm3", "norm3_bias", "qkv", "qkv_bias", "q_norm", "k_norm",
             "out", "out_bias", "fc1", "fc1_bias", "fc2", "fc2_bias", "cq",
             "cq_bias", "ck", "ck_bias", "cv", "cv_bias", "cq_norm",
             "ck_norm", "co", "co_bias", "modulation"]


def _rope(rng, rows, half=48):
    ang = rng.uniform(-40, 40, rows * half).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _check(got, want, what):
    cos, rel = cosine_rel_l2(got, want)
    assert cos >= 0.999 and rel <= 1e-2, f"{what}: cos {cos:.6f} rel {rel:.3g}"
    return cos, rel


@pytest.mark.parametrize("hidden,heads,ffn,rows,blocks", [
    (512, 4, 1024, 300, 2),       # small, two blocks (fused cross-block adaLN)
    (1024, 8, 2048, 700, 3),      # three blocks, ragged rows
    (5376, 56, 14336, 200, 1),    # the real H3 block shape
])
def test_h3_blocks(gpu, hidden, heads, ffn, rows, blocks):
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, hidden, heads, ffn, rows,
                           blocks=blocks, time_rows=2)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=hidden + rows, weight_std=0.02, mod_std=0.1)
        rng = np.random.default_rng(rows)
        cos, sin = _rope(rng, rows)
        dit.set_rope(cos, sin)
        row_map = rng.integers(0, 2 * 3, rows).astype(np.uint32)
        dit.set_row_map(row_map)
        weights = [{n: dit.read(n, b) for n in H3_NAMES}
                   for b in range(blocks)]
        x0 = dit.read("hidden")
        dit.run_blocks(0, blocks)
        got = dit.read("hidden")
        want = oracle.h3_blocks(x0, weights, row_map, oracle.bf16(cos),
                                oracle.bf16(sin), rows, hidden, heads, ffn)
        _check(got, want, f"H3 {blocks} block(s) {hidden}/{rows}")
    finally:
        dit.close()


@pytest.mark.parametrize("hidden,heads,ffn,rows,text", [
    (512, 4, 1024, 300, 64),
    (5120, 40, 13824, 256, 77),   # the Wan block shape
])
def test_wan_block(gpu, hidden, heads, ffn, rows, text):
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, hidden, heads, ffn, rows,
                           blocks=1, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=7 + rows, weight_std=0.02, mod_std=0.1)
        rng = np.random.default_rng(text)
        cos, sin = _rope(rng, rows)
        dit.set_rope(cos, sin)
        w = {n: dit.read(n, 0) for n in WAN_NAMES}
        x0, ctx = dit.read("hidden"), dit.read("context")
        dit.run_blocks(0, 1)
        got = dit.read("hidden")
        want = oracle.wan_block(x0, ctx, w, np.zeros(rows, np.uint32),
                                oracle.bf16(cos), oracle.bf16(sin), rows, text,
                                hidden, heads, ffn)
        _check(got, want, f"Wan block {hidden}/{rows}")
    finally:
        dit.close()


def test_wan_blocks_fused_across_blocks(gpu):
    """Two Wan blocks in one call: the first block's FFN gate also produces
    the second block's self-attention adaLN.  Against the oracle block by
    block, and bit-identical to running the blocks in separate calls (which
    takes the unfused gate and adaLN)."""
    hidden, heads, ffn, rows, text = 512, 4, 1024, 200, 40
    cfg = h3hip.dit_config(h3hip.FAMILY_WAN, hidden, heads, ffn, rows,
                           blocks=2, text_rows=text)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=19, weight_std=0.02, mod_std=0.1)
        rng = np.random.default_rng(5)
        cos, sin = _rope(rng, rows)
        dit.set_rope(cos, sin)
        ws = [{n: dit.read(n, b) for n in WAN_NAMES} for b in range(2)]
        x0, ctx = dit.read("hidden"), dit.read("context")
        dit.run_blocks(0, 2)
        fused = dit.read("hidden")
        want = x0
        for b in range(2):
            want = oracle.wan_block(want, ctx, ws[b],
                                    np.zeros(rows, np.uint32),
                                    oracle.bf16(cos), oracle.bf16(sin), rows,
                                    text, hidden, heads, ffn)
        _check(fused, want, "Wan 2 blocks")
        dit.write("hidden", x0)
        dit.run_blocks(0, 1)
        dit.run_blocks(1, 1)
        assert np.array_equal(dit.read("hidden"), fused)
    finally:
        dit.close()


def test_h3_block_full_size_properties(gpu):
    """BASELINE config 2 shape at H3 real size (N = 2378 rows): no oracle run
    at this size; checks finiteness, determinism of a re-run and that a zero
    gate leaves the residual stream unchanged (gate slots 2 and 5 = 0 ->
    hidden_out == hidden_in, bit for bit)."""
    rows, hidden = 2378, 5376
    cfg = h3hip.dit_config(h3hip.FAMILY_H3, hidden, 56, 14336, rows,
                           blocks=1, time_rows=1)
    dit = h3hip.Dit(gpu, cfg)
    try:
        dit.init_random(seed=3, mod_std=0.1)
        x0 = dit.read("hidden")
        dit.run_blocks(0, 1)
        y1 = dit.read("hidden")
        assert np.isfinite(oracle.f32(y1)).all()
        dit.write("hidden", x0)
        dit.run_blocks(0, 1)
        assert np.array_equal(dit.read("hidden"), y1), "not deterministic"
        mod = dit.read("modulation").reshape(1, 3, 6, hidden).copy()
        mod[:, :, 2, :] = 0
        mod[:, :, 5, :] = 0
        dit.write("modulation", mod.ravel())
        dit.write("hidden", x0)
        dit.run_blocks(0, 1)
        assert np.array_equal(dit.read("hidden"), x0)
    finally:
        dit.close()
