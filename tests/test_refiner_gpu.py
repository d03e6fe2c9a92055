"""The text token refiner (reference refine_text, h3_dit.c:766-884) on the
GPU against the oracle's composition of the same ops, at small widths and
at the reference's real ones (text 5120 -> hidden 5376, 42 heads, FFN
14336) with a short prompt."""
import numpy as np
import pytest

import h3hip
import oracle
from conftest import cosine_rel_l2

pytestmark = pytest.mark.gpu

NAMES = ["norm1", "qkv", "q_norm", "k_norm", "out", "norm2", "fc1", "fc2"]


@pytest.mark.parametrize("rows,text_dim,hidden,heads,ffn", [
    (12, 384, 256, 2, 512),
    (77, 640, 512, 4, 768),
    (1, 256, 256, 2, 256),
    (40, 5120, 5376, 42, 14336),
])
def test_refiner_matches_oracle(gpu, rows, text_dim, hidden, heads, ffn):
    r = h3hip.Refiner(gpu, hidden, heads, ffn, text_dim)
    try:
        r.init_random(rows + hidden, weight_std=0.05 if hidden < 1024
                      else 0.02)
        rng = np.random.default_rng(rows)
        src_bits = h3hip.f32_to_bf16(
            rng.standard_normal(rows * text_dim).astype(np.float32))
        src = gpu.bf16(src_bits)
        out = gpu.new_bf16(rows * hidden)
        r.run(out, src, rows)
        got = gpu.read_bf16(out)
        w = {k: r.read(k) for k in ("condition_w", "condition_b",
                                    "final_norm")}
        w["blocks"] = [{k: r.read(k, b) for k in NAMES} for b in range(2)]
        want = oracle.refine_text(src_bits, w, rows, text_dim, hidden, heads,
                                  ffn)
        cos, rel = cosine_rel_l2(got, want)
        assert cos >= 0.999 and rel <= 1e-2, (cos, rel)
        gpu.free(src)
        gpu.free(out)
    finally:
        r.close()


def test_refiner_rejects_short_tensors(gpu):
    r = h3hip.Refiner(gpu, 256, 2, 256, 256)
    try:
        src = gpu.new_bf16(10 * 256)
        out = gpu.new_bf16(10 * 256)
        with pytest.raises(RuntimeError, match="invalid refiner run"):
            r.run(out, src, 11)
        gpu.free(src)
        gpu.free(out)
    finally:
        r.close()
