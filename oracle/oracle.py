"""CPU oracle of the DiT denoiser path -- TEST INFRASTRUCTURE ONLY.

Python side of oracle/h3_oracle.c: numpy wrappers of the restated reference
kernels and the block compositions in the reference's op order.  Only the
tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.

Every function cites the reference lines it restates.  Pins (golden vectors,
known answers, invariants) for each live in tests/test_oracle_pins.py and
tests/test_host_math.py.
"""
import ctypes as C
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libh3_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libh3ref.so")

_P = C.c_void_p
_SZ = C.c_size_t
_F = C.c_float
_I = C.c_int

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        sig = {
            "orc_linear_bf16": [_P, _P, _P, _P, _SZ, _SZ, _SZ],
            "orc_linear_f32": [_P, _P, _P, _P, _SZ, _SZ, _SZ],
            "orc_token_pool": [_P, _P, _P, _P, _P, _P, _SZ, _SZ],
            "orc_token_expand": [_P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _F],
            "orc_sdpa_sparse": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _F, C.c_int,
                                C.c_int, _P, _P],
            "orc_patch_linear": [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ],
            "orc_adaln": [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _F],
            "orc_gate": [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ],
            "orc_gate_adaln": [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ,
                               _SZ, _SZ, _SZ, _F],
            "orc_layer_adaln": [_P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ,
                                _SZ, _F],
            "orc_rms_norm": [_P, _P, _P, _SZ, _SZ, _F],
            "orc_head_rms_norm": [_P, _P, _SZ, _SZ, _SZ, _F],
            "orc_qkv_rope": [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ,
                             _SZ, _I, _F],
            "orc_sdpa": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, _F, _I, _I],
            "orc_rope_rotate": [_P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ],
            "orc_swiglu": [_P, _P, _SZ, _SZ],
            "orc_gelu": [_P, _P, _SZ],
            "orc_silu": [_P, _P, _SZ],
            "orc_add": [_P, _P, _P, _SZ],
            "orc_sub": [_P, _P, _P, _SZ],
            "orc_euler": [_P, _P, _P, _SZ, _F, _F],
            "orc_adaln_linear": [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ,
                                 _SZ, _SZ, _SZ, _SZ, _F],
            "orc_f32_to_bf16": [_P, _P, _SZ],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.restype = None
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def bf16(x):
    """float32 -> bf16 bits (RNE), via the oracle's own rounding."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16(_p(x), _p(out), x.size)
    return out


def f32(b):
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32)
            << 16).view(np.float32)


# ------------------------------------------------------------------- ops

def linear(x, w, bias, m, k, n):
    """h3_cuda_core.cu:358-371 (sequential-k fmaf from the bias)."""
    out = np.empty(m * n, dtype=np.uint16)
    lib().orc_linear_bf16(_p(_u16(x)), _p(_u16(w)),
                          _p(None if bias is None else _u16(bias)), _p(out),
                          m, k, n)
    return out


def linear_f32(x, w, bias, m, k, n):
    """h3_cuda_core.cu:343-356 (F32, sequential-k fmaf from the bias)."""
    out = np.empty(m * n, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().orc_linear_f32(_p(x), _p(w), _p(b), _p(out), m, k, n)
    return out


def time_embedding(features, in_w, in_b, out_w, out_b, rows, inp, hid, dim):
    """The timestep MLP of the schedule precompute (h3_dit_schedule.c:
    163-234): F32 linear inp -> hid, SiLU (x / (1 + e^-x), :15-20), F32
    linear hid -> dim, cast to bf16, bf16 SiLU (:23-29).  Returns bf16
    bits [rows][dim]."""
    h = linear_f32(features, in_w, in_b, rows, inp, hid)
    h = (h / (np.float32(1) + np.exp(-h))).astype(np.float32)
    o = linear_f32(h, out_w, out_b, rows, hid, dim)
    return silu(bf16(o))


def patch_linear(x, w, bias, m, k, n, row_map=None, out_rows=None):
    """h3_cuda_core.cu:374-403 (F32 in, bf16 rows out)."""
    rows = out_rows if out_rows is not None else m
    out = np.zeros(rows * n, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rm = None if row_map is None else np.ascontiguousarray(row_map, np.uint32)
    lib().orc_patch_linear(_p(x), _p(w), _p(b), _p(out), _p(rm), m, k, n)
    return out


def adaln(x, w, mod, row_map, rows, width, slots, shift, scale, eps):
    """h3_cuda_dit.cu:141-175."""
    out = np.empty(rows * width, dtype=np.uint16)
    rm = np.ascontiguousarray(row_map, dtype=np.uint32)
    lib().orc_adaln(_p(_u16(x)), _p(_u16(w)), _p(_u16(mod)), _p(rm), _p(out),
                    rows, width, slots, shift, scale, eps)
    return out


def gate(res, br, mod, row_map, rows, width, slots, gate_slot):
    """h3_cuda_dit.cu:261-276."""
    out = np.empty(rows * width, dtype=np.uint16)
    rm = np.ascontiguousarray(row_map, dtype=np.uint32)
    lib().orc_gate(_p(_u16(res)), _p(_u16(br)), _p(_u16(mod)), _p(rm),
                   _p(out), rows, width, slots, gate_slot)
    return out


def gate_adaln(res, br, w, gate_mod, norm_mod, row_map, rows, width, slots,
               gate_slot, shift, scale, eps):
    """h3_cuda_dit.cu:281-332; returns (gated, normalised)."""
    gated = np.empty(rows * width, dtype=np.uint16)
    out = np.empty(rows * width, dtype=np.uint16)
    rm = np.ascontiguousarray(row_map, dtype=np.uint32)
    lib().orc_gate_adaln(_p(_u16(res)), _p(_u16(br)), _p(_u16(w)),
                         _p(_u16(gate_mod)), _p(_u16(norm_mod)), _p(rm),
                         _p(gated), _p(out), rows, width, slots, gate_slot,
                         shift, scale, eps)
    return gated, out


def layer_adaln(x, w, b, mod, row_map, rows, width, slots, shift, scale,
                eps):
    """h3_cuda_core.cu:250-295 LayerNorm (+affine) with adaLN modulation."""
    out = np.empty(rows * width, dtype=np.uint16)
    rm = None if row_map is None else np.ascontiguousarray(row_map, np.uint32)
    lib().orc_layer_adaln(_p(_u16(x)), _p(None if w is None else _u16(w)),
                          _p(None if b is None else _u16(b)),
                          _p(None if mod is None else _u16(mod)), _p(rm),
                          _p(out), rows, width, slots, shift, scale, eps)
    return out


def rms_norm(x, w, rows, width, eps):
    """h3_cuda_core.cu:184-210."""
    out = np.empty(rows * width, dtype=np.uint16)
    lib().orc_rms_norm(_p(_u16(x)), _p(_u16(w)), _p(out), rows, width, eps)
    return out


def head_rms_norm(t, w, rows, heads, hd, eps):
    """h3_cuda_core.cu:322-341 (returns a new array)."""
    out = _u16(t).copy()
    lib().orc_head_rms_norm(_p(out), _p(_u16(w)), rows, heads, hd, eps)
    return out


def qkv_rope(qkv, qw, kw, cos, sin, seq, heads, hd, rope_half, grouped, eps):
    """h3_cuda_attention.cu:175-237; returns (q, k, v)."""
    n = seq * heads * hd
    q = np.empty(n, np.uint16)
    k = np.empty(n, np.uint16)
    v = np.empty(n, np.uint16)
    lib().orc_qkv_rope(_p(_u16(qkv)), _p(_u16(qw)), _p(_u16(kw)),
                       _p(_u16(cos)), _p(_u16(sin)), _p(q), _p(k), _p(v), seq,
                       heads, hd, rope_half, int(grouped), eps)
    return q, k, v


def rope_rotate(x, cos, sin, rows, heads, hd=128, half=48):
    """The RoPE pair rotation alone (h3_cuda_attention.cu:218-233 without
    the Q/K norm) on [rows][heads][hd] bf16 bits."""
    out = np.empty(rows * heads * hd, np.uint16)
    lib().orc_rope_rotate(_p(_u16(x)), _p(_u16(cos)), _p(_u16(sin)), _p(out),
                          rows, heads, hd, half)
    return out


def sdpa(q, k, v, q_rows, kv_rows, heads, hd, scale, head_major=False,
         round_p=True):
    """h3_cuda_attention.cu:488-549 with the flash kernels' bf16-P rule."""
    out = np.empty(q_rows * heads * hd, np.uint16)
    lib().orc_sdpa(_p(_u16(q)), _p(_u16(k)), _p(_u16(v)), _p(out), q_rows,
                   kv_rows, heads, hd, scale, int(head_major), int(round_p))
    return out


def sdpa_sparse(q, k, v, rows, heads, hd, scale, ptr, idx,
                head_major=False, round_p=True):
    """Block-sparse joint attention over a CSR of 64-row key tiles per
    128-row query block (h3_gpu.h:44-52; h3_cuda_attention.cu:1652-1673)."""
    out = np.empty(rows * heads * hd, np.uint16)
    p = np.ascontiguousarray(ptr, dtype=np.uint32)
    i = np.ascontiguousarray(idx, dtype=np.uint32)
    lib().orc_sdpa_sparse(_p(_u16(q)), _p(_u16(k)), _p(_u16(v)), _p(out),
                          rows, heads, hd, scale, int(head_major),
                          int(round_p), _p(p), _p(i))
    return out


def token_pool(inp, pairs, baseline_indices, input_rows, rows,
               baseline_rows, width):
    """h3_cuda_dit.cu:336-360; returns (output, original, baseline).
    original / baseline start as zeros where nothing is written."""
    out = np.zeros(rows * width, np.uint16)
    original = np.zeros(input_rows * width, np.uint16)
    baseline = np.zeros(max(baseline_rows, 1) * width, np.uint16)
    lib().orc_token_pool(_p(_u16(inp)),
                         _p(np.ascontiguousarray(pairs, np.uint32)), _p(out),
                         _p(baseline),
                         _p(np.ascontiguousarray(baseline_indices, np.uint32)),
                         _p(original), rows, width)
    return out, original, baseline


def token_expand(original, reduced, baseline, baseline_indices, parents,
                 rows, width, exact_prefix_rows, update_scale):
    """h3_cuda_dit.cu:441-470."""
    out = np.empty(rows * width, np.uint16)
    lib().orc_token_expand(_p(_u16(original)), _p(_u16(reduced)),
                           _p(_u16(baseline)),
                           _p(np.ascontiguousarray(baseline_indices,
                                                   np.uint32)),
                           _p(np.ascontiguousarray(parents, np.uint32)),
                           _p(out), rows, width, exact_prefix_rows,
                           update_scale)
    return out


def swiglu(fused, rows, width):
    """h3_cuda_core.cu:104-114."""
    out = np.empty(rows * width, np.uint16)
    lib().orc_swiglu(_p(_u16(fused)), _p(out), rows, width)
    return out


def gelu(x):
    """h3_cuda_core.cu:139-158 (tanh form)."""
    x = _u16(x)
    out = np.empty(x.size, np.uint16)
    lib().orc_gelu(_p(x), _p(out), x.size)
    return out


def silu(x):
    x = _u16(x)
    out = np.empty(x.size, np.uint16)
    lib().orc_silu(_p(x), _p(out), x.size)
    return out


def add(a, b):
    a = _u16(a)
    out = np.empty(a.size, np.uint16)
    lib().orc_add(_p(a), _p(_u16(b)), _p(out), a.size)
    return out


def euler(sample, last, prev, delta, ratio):
    """h3_cuda_dit.cu:536-548 (returns the updated copy)."""
    s = np.ascontiguousarray(sample, dtype=np.float32).copy()
    lib().orc_euler(_p(s), _p(_u16(last)), _p(_u16(prev)), s.size, delta,
                    ratio)
    return s


def adaln_linear(x, nw, mod, row_map, w, bias, rows, width, n, slots, shift,
                 scale, eps):
    """h3_cuda_dit.cu:179-234; returns (out, inverse)."""
    out = np.empty(rows * n, np.uint16)
    inv = np.empty(rows, np.float32)
    rm = np.ascontiguousarray(row_map, dtype=np.uint32)
    lib().orc_adaln_linear(_p(_u16(x)), _p(_u16(nw)), _p(_u16(mod)), _p(rm),
                           _p(_u16(w)), _p(None if bias is None else
                                           _u16(bias)),
                           _p(out), _p(inv), rows, width, n, slots, shift,
                           scale, eps)
    return out, inv


def mlp(x, fc1, fc2, rows, d, ffn):
    """h3_gpu_mlp_bf16 on the reference's GEMM path (h3_cuda_core.cu:
    1067-1104): fused fc1 rounded to bf16, SwiGLU to bf16, fc2."""
    fused = linear(x, fc1, None, rows, d, 2 * ffn)
    act = swiglu(fused, rows, ffn)
    return linear(act, fc2, None, rows, ffn, d)


def ffn_gelu(x, fc1, b1, fc2, b2, rows, d, ffn):
    """GELU-tanh FFN: fc2(gelu(bf16(fc1 x + b1))) + b2."""
    h = linear(x, fc1, b1, rows, d, ffn)
    return linear(gelu(h), fc2, b2, rows, ffn, d)


# ---------------------------------------------------------- block orders

def h3_blocks(hidden, blocks, row_map, cos, sin, rows, hidden_dim, heads, ffn,
              hd=128, rope_half=48, eps=1e-5, sparse=None):
    """Consecutive H3 blocks in the reference run order (h3_dit.c:2008-2180,
    BF16 path; fused gate+adaLN; the MLP gate of block i fused with block
    i+1's attention adaLN, :2139-2178).  blocks: list of dicts with norm1,
    norm2, qkv, q_norm, k_norm, out, fc1, fc2, modulation (bf16 bits).
    sparse: optional (ptr, idx) block-sparse mask of the joint attention.
    Returns the final hidden state."""
    S = 6
    inner = heads * hd
    x = _u16(hidden).copy()
    a = None
    for i, w in enumerate(blocks):
        mod = w["modulation"]
        if a is None:
            a = adaln(x, w["norm1"], mod, row_map, rows, hidden_dim, S, 0, 1,
                      eps)
        qkv = linear(a, w["qkv"], None, rows, hidden_dim, 3 * inner)
        q, k, v = qkv_rope(qkv, w["q_norm"], w["k_norm"], cos, sin, rows,
                           heads, hd, rope_half, True, eps)
        if sparse is None:
            o = sdpa(q, k, v, rows, rows, heads, hd, 1.0 / math.sqrt(hd))
        else:
            o = sdpa_sparse(q, k, v, rows, heads, hd, 1.0 / math.sqrt(hd),
                            sparse[0], sparse[1])
        y = linear(o, w["out"], None, rows, inner, hidden_dim)
        x, b = gate_adaln(x, y, w["norm2"], mod, mod, row_map, rows,
                          hidden_dim, S, 2, 3, 4, eps)
        m = mlp(b, w["fc1"], w["fc2"], rows, hidden_dim, ffn)
        if i + 1 < len(blocks):
            nxt = blocks[i + 1]
            x, a = gate_adaln(x, m, nxt["norm1"], mod, nxt["modulation"],
                              row_map, rows, hidden_dim, S, 5, 0, 1, eps)
        else:
            x = gate(x, m, mod, row_map, rows, hidden_dim, S, 5)
            a = None
    return x


def refine_text(source, w, rows, text_dim, hidden_dim, heads, ffn, hd=128,
                eps=1e-5):
    """Text token refiner in the reference op order (refine_text and
    run_refiner_block, h3_dit.c:766-884): biased condition projection, two
    pre-norm blocks of RMSNorm -> QKV -> per-head q/k RMS (no RoPE) -> SDPA
    -> out + residual, RMSNorm -> fc1 -> SwiGLU -> fc2 + residual, and a final
    RMSNorm.  w: condition_w, condition_b, final_norm, blocks[2] of dicts
    with norm1, qkv, q_norm, k_norm, out, norm2, fc1, fc2 (bf16 bits)."""
    inner = heads * hd
    x = linear(source, w["condition_w"], w["condition_b"], rows, text_dim,
               hidden_dim)
    for b in w["blocks"]:
        n = rms_norm(x, b["norm1"], rows, hidden_dim, eps)
        qkv = linear(n, b["qkv"], None, rows, hidden_dim, 3 * inner)
        q, k, v = qkv_rope(qkv, b["q_norm"], b["k_norm"], b["q_norm"],
                           b["q_norm"], rows, heads, hd, 0, True, eps)
        o = sdpa(q, k, v, rows, rows, heads, hd, 1.0 / math.sqrt(hd))
        x = add(x, linear(o, b["out"], None, rows, inner, hidden_dim))
        n = rms_norm(x, b["norm2"], rows, hidden_dim, eps)
        x = add(x, mlp(n, b["fc1"], b["fc2"], rows, hidden_dim, ffn))
    return rms_norm(x, w["final_norm"], rows, hidden_dim, eps)


def reuse_schedule(steps, interval):
    """Evaluated steps under velocity reuse (h3_dit.c:2672-2687)."""
    return [interval == 1 or s == 0 or s == steps - 1 or s % interval == 0
            for s in range(steps)]


def extrapolation_ratio(current, last, previous, have_previous):
    """Clamped linear velocity extrapolation ratio (h3_dit.c:2644-2655),
    evaluated in F32 like the reference."""
    if not have_previous:
        return np.float32(0.0)
    den = np.float32(last) - np.float32(previous)
    r = ((np.float32(current) - np.float32(last)) / den
         if den != 0 else np.float32(0.0))
    return np.float32(min(max(r, -2.0), 2.0))


def h3_forward_step(m, step):
    """One sampler forward (h3_dit.c:2182-2528, fused patch/pack and fused
    final-head path): pack text / patch-projected latent rows into the
    sequence in layout order, run the blocks with the step's row map, then
    the final adaLN + heads of the audio and video targets.  `m` is a dict
    holding the model (see tests/test_sampler_gpu.py); returns (video,
    audio) velocities as bf16 bits."""
    d, vp, ac = m["hidden"], m["video_patch"], m["audio_channels"]
    hidden = np.zeros(m["rows"] * d, np.uint16)
    vo = ao = to = 0
    for start, stop, kind in m["segments"]:
        n = stop - start
        if kind == 0:
            hidden[start * d:stop * d] = m["refined_text"][to * d:(to + n) * d]
            to += n
        elif kind in (1, 2, 5):
            hidden[start * d:stop * d] = patch_linear(
                m["video_input"][vo * vp:(vo + n) * vp], m["video_patch_w"],
                m["video_patch_b"], n, vp, d)
            vo += n
        else:
            hidden[start * d:stop * d] = patch_linear(
                m["audio_input"][ao * ac:(ao + n) * ac], m["audio_patch_w"],
                m["audio_patch_b"], n, ac, d)
            ao += n
    x = h3_blocks(hidden, m["blocks"], m["step_maps"][step], m["cos"],
                  m["sin"], m["rows"], d, m["heads"], m["ffn"],
                  eps=m["eps"])
    a0, na = m["audio_target_start"], m["audio_targets"]
    v0, nv = m["video_target_start"], m["video_targets"]
    audio, _ = adaln_linear(x[a0 * d:(a0 + na) * d], m["final_norm"],
                            m["final_modulation"],
                            m["final_audio_maps"][step], m["final_audio_w"],
                            m["final_audio_b"], na, d, ac, 2, 0, 1, m["eps"])
    video, _ = adaln_linear(x[v0 * d:(v0 + nv) * d], m["final_norm"],
                            m["final_modulation"],
                            m["final_video_maps"][step], m["final_video_w"],
                            m["final_video_b"], nv, d, vp, 2, 0, 1, m["eps"])
    return video, audio


def h3_denoise(m, video_sigmas, audio_sigmas, reuse_interval,
               forward=None):
    """The GPU Euler loop with velocity reuse (h3_dit.c:2745-2917): cache
    the previous velocity before each fresh evaluation, extrapolate on the
    skipped steps, x += (sigma_i - sigma_i+1) (v + r (v - v_prev)).
    `forward(m, step) -> (video, audio)` evaluates the velocities (default:
    h3_forward_step, the oracle's own forward; a test may pass the device's
    forward to check the loop alone at sizes the oracle forward cannot run).
    Returns the updated (video, audio) F32 latent rows and the number of
    evaluations."""
    if forward is None:
        forward = h3_forward_step
    steps = len(video_sigmas) - 1
    vp, ac = m["video_patch"], m["audio_channels"]
    video = np.array(m["video_input"], np.float32)
    audio = np.array(m["audio_input"], np.float32)
    voff = m["video_conditions"] * vp
    aoff = m["audio_conditions"] * ac
    sel = reuse_schedule(steps, reuse_interval)
    last = previous = -1
    vv = av = vprev = aprev = None
    evaluations = 0
    for step in range(steps):
        if sel[step]:
            if last >= 0 and reuse_interval > 1:
                vprev, aprev = vv.copy(), av.copy()
                previous = last
            mm = dict(m, video_input=video, audio_input=audio)
            vv, av = forward(mm, step)
            last = step
            evaluations += 1
        have = previous >= 0
        if sel[step]:
            vr = ar = np.float32(0.0)
        else:
            vr = extrapolation_ratio(video_sigmas[step], video_sigmas[last],
                                     video_sigmas[previous] if have else 0.0,
                                     have)
            ar = extrapolation_ratio(audio_sigmas[step], audio_sigmas[last],
                                     audio_sigmas[previous] if have else 0.0,
                                     have)
        vdt = np.float32(video_sigmas[step]) - np.float32(video_sigmas[step + 1])
        adt = np.float32(audio_sigmas[step]) - np.float32(audio_sigmas[step + 1])
        nv, na = vv.size, av.size
        video[voff:voff + nv] = euler(video[voff:voff + nv], vv,
                                      vprev if have else vv, vdt, vr)
        audio[aoff:aoff + na] = euler(audio[aoff:aoff + na], av,
                                      aprev if have else av, adt, ar)
    return video, audio, evaluations


def wan_block(hidden, context, w, row_map, cos, sin, rows, text_rows, d,
              heads, ffn, hd=128, rope_half=48, eps=1e-6):
    """One Wan-style block (the benchmark block; the reference has none).
    Specification, Wan 2.x order: x += slot2 * selfattn(LN(x)(1 + slot1)
    + slot0); x += crossattn(norm3(x), context) (LayerNorm with affine, no
    gate); x += slot5 * ffn(LN(x)(1 + slot4) + slot3).  Q/K norms are per
    head (128-wide weights), as the reference's grouped QK norm is
    (h3_cuda_attention.cu:175-237).  Primitives: LayerNorm
    h3_cuda_core.cu:250-295, gate h3_cuda_dit.cu:261-276, GELU-tanh
    h3_cuda_core.cu:139-158.  The wiring is pinned by the closed-form tests
    in tests/test_oracle_pins.py (test_wan_block_*)."""
    S = 6
    inner = heads * hd
    scale = 1.0 / math.sqrt(hd)
    x = _u16(hidden).copy()
    mod = w["modulation"]
    a = layer_adaln(x, None, None, mod, row_map, rows, d, S, 0, 1, eps)
    qkv = linear(a, w["qkv"], w["qkv_bias"], rows, d, 3 * inner)
    q, k, v = qkv_rope(qkv, w["q_norm"], w["k_norm"], cos, sin, rows, heads,
                       hd, rope_half, False, eps)
    o = sdpa(q, k, v, rows, rows, heads, hd, scale)
    y = linear(o, w["out"], w["out_bias"], rows, inner, d)
    x = gate(x, y, mod, row_map, rows, d, S, 2)
    c = layer_adaln(x, w["norm3"], w["norm3_bias"], None, None, rows, d, S, 0,
                    0, eps)
    cq = head_rms_norm(linear(c, w["cq"], w["cq_bias"], rows, d, inner),
                       w["cq_norm"], rows, heads, hd, eps)
    ck = head_rms_norm(linear(context, w["ck"], w["ck_bias"], text_rows, d,
                              inner), w["ck_norm"], text_rows, heads, hd, eps)
    cv = linear(context, w["cv"], w["cv_bias"], text_rows, d, inner)
    co = sdpa(cq, ck, cv, rows, text_rows, heads, hd, scale)
    x = add(x, linear(co, w["co"], w["co_bias"], rows, inner, d))
    a = layer_adaln(x, None, None, mod, row_map, rows, d, S, 3, 4, eps)
    f = ffn_gelu(a, w["fc1"], w["fc1_bias"], w["fc2"], w["fc2_bias"], rows,
                 d, ffn)
    return gate(x, f, mod, row_map, rows, d, S, 5)


# --------------------------------------------------- reference host build

_ref = None


def ref_lib():
    """The reference's own h3_host.c, compiled by `make -C oracle ref`
    (only where /root/reference exists).  Returns None when absent."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = C.CDLL(REF_PATH)
    return _ref
