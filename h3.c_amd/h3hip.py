"""ctypes binding of libh3_gpu_hip.so (the h3_gpu.h C ABI, the h3_hip.h
extras, the host math of h3hip_host.h and the DiT driver of h3hip_dit.h).

This is plumbing for tests and the benchmark: it allocates nothing on the
device itself and calls the C ABI exactly as the engine's C code would.
Loading fails loudly when the shared library has not been built.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libh3_gpu_hip.so")

F32, BF16, I8, U32 = 0, 1, 2, 3
FAMILY_H3, FAMILY_WAN = 0, 1

_P = C.c_void_p
_U32 = C.c_uint32
_SZ = C.c_size_t
_F = C.c_float
_I = C.c_int


class DitConfig(C.Structure):
    _fields_ = [("family", _I), ("hidden", _U32), ("heads", _U32),
                ("head_dim", _U32), ("ffn", _U32), ("blocks", _U32),
                ("rows", _U32), ("text_rows", _U32), ("time_rows", _U32),
                ("rope_half", _U32), ("epsilon", _F)]


class Position(C.Structure):
    _fields_ = [("t", C.c_double), ("h", C.c_double), ("w", C.c_double)]


class Segment(C.Structure):
    _fields_ = [("start", _SZ), ("stop", _SZ), ("kind", _I)]


class LayoutRef(C.Structure):
    _fields_ = [("kind", _I), ("latent_t", _I), ("latent_h", _I),
                ("latent_w", _I), ("audio_t", _I)]


class Layout(C.Structure):
    _fields_ = [("seq_len", _SZ), ("segments", C.POINTER(Segment)),
                ("segment_count", _SZ), ("positions", C.POINTER(Position)),
                ("img_cond_rows", _SZ), ("img_target_rows", _SZ),
                ("audio_cond_rows", _SZ), ("audio_target_rows", _SZ)]


class SamplerConfig(C.Structure):
    _fields_ = [("layout", C.POINTER(Layout)), ("steps", _I),
                ("video_sigmas", C.POINTER(_F)),
                ("audio_sigmas", C.POINTER(_F)), ("reuse_interval", _I),
                ("video_patch", _U32), ("audio_channels", _U32)]


class Rng(C.Structure):
    _fields_ = [("state", C.c_uint64), ("increment", C.c_uint64),
                ("spare", _F), ("has_spare", _I)]


class Stats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "allocated_bytes", "live_bytes", "peak_live_bytes",
        "tensor_allocations", "direct_dispatches", "mps_linear_dispatches",
        "mps_conv_dispatches", "mps_sdpa_dispatches", "blit_copies",
        "submissions")] + [("command_encode_seconds", C.c_double),
                           ("command_wait_seconds", C.c_double),
                           ("gpu_seconds", C.c_double)]


_lib = None


def lib():
    """Load the backend library once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with "
                           "`make -C h3.c_amd` (or __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    sig = {
        "h3_gpu_create": (_P, [C.c_char_p, C.c_char_p, _SZ]),
        "h3_gpu_free": (None, [_P]),
        "h3_gpu_error": (C.c_char_p, [_P]),
        "h3_gpu_begin": (_I, [_P]),
        "h3_gpu_continue": (_I, [_P]),
        "h3_gpu_submit": (_I, [_P]),
        "h3_gpu_get_stats": (_I, [_P, C.POINTER(Stats)]),
        "h3_gpu_prefers_gpu_sampler": (_I, [_P]),
        "h3_gpu_has_int8_mlp": (_I, [_P]),
        "h3_gpu_tensor_new_f32": (_P, [_P, _SZ]),
        "h3_gpu_tensor_new_bf16": (_P, [_P, _SZ]),
        "h3_gpu_tensor_from_f32": (_P, [_P, _P, _SZ]),
        "h3_gpu_tensor_from_bf16": (_P, [_P, _P, _SZ]),
        "h3_gpu_tensor_from_u32": (_P, [_P, _P, _SZ]),
        "h3_gpu_tensor_free": (None, [_P]),
        "h3_gpu_tensor_elements": (_SZ, [_P]),
        "h3_gpu_tensor_dtype": (_I, [_P]),
        "h3_gpu_tensor_read_f32": (_I, [_P, _P, _SZ]),
        "h3_gpu_tensor_read_f32_range": (_I, [_P, _SZ, _P, _SZ]),
        "h3_gpu_tensor_read_bf16": (_I, [_P, _P, _SZ]),
        "h3_gpu_tensor_write_f32": (_I, [_P, _P, _SZ]),
        "h3_gpu_tensor_write_f32_range": (_I, [_P, _SZ, _P, _SZ]),
        "h3_gpu_tensor_write_bf16": (_I, [_P, _P, _SZ]),
        "h3_gpu_linear_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32]),
        "h3_gpu_linear_gelu_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32,
                                         _U32]),
        "h3_gpu_linear_f32": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32]),
        "h3_gpu_mlp_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _U32]),
        "h3_gpu_ffn_gelu_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _U32,
                                      _U32, _U32, _U32]),
        "h3_gpu_adaln_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32,
                                   _U32, _U32, _F]),
        "h3_gpu_adaln_bf16_offset": (_I, [_P, _P, _P, _SZ, _P, _P, _P, _U32,
                                          _U32, _U32, _U32, _U32, _F]),
        "h3_gpu_gate_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U32, _U32, _U32,
                                  _U32]),
        "h3_gpu_gate_adaln_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P,
                                        _U32, _U32, _U32, _U32, _U32, _U32,
                                        _F]),
        "h3_hip_linear_pair_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P,
                                         _U32, _U32, _U32]),
        "h3_hip_linear_bf16_noalloc": (_I, [_P, _P, _P, _P, _P, _U32, _U32,
                                            _U32]),
        "h3_hip_device_allocations": (C.c_uint64, [_P]),
        "h3_hip_sdpa_rope_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32,
                                       _U32, _U32, _F]),
        "h3_hip_qk_norm_rope_inplace_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U32,
                                                  _U32, _U32, _U32, _F, _I]),
        "h3_hip_sdpa_qkv_norm_rope_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U32,
                                                _U32, _U32, _U32, _F, _F]),
        "h3_hip_sdpa_cross_norm_bf16": (_I, [_P, _P, _P, _P, _P, _P, _U32,
                                             _U32, _U32, _U32, _F, _F]),
        "h3_hip_sdpa_qkv_bf16": (_I, [_P, _P, _P, _U32, _U32, _U32, _F]),
        "h3_hip_linear_group_table": (_P, [_P, _P, _P, _P, _U32, _U32, _U32,
                                           _U32]),
        "h3_hip_head_norm_group_table": (_P, [_P, _P, _P, _U32, _U32, _U32,
                                              _U32]),
        "h3_hip_head_rms_norm_group_bf16": (_I, [_P, _P, _U32, _U32, _U32,
                                                 _U32, _U32, _F]),
        "h3_hip_linear_group_bf16": (_I, [_P, _P, _U32, _U32, _P, _U32, _U32,
                                          _U32]),
        "h3_gpu_layer_adaln_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _U32,
                                         _U32, _U32, _U32, _U32, _F]),
        "h3_gpu_gate_layer_adaln_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P,
                                              _P, _P, _P, _U32, _U32, _U32,
                                              _U32, _U32, _U32, _F]),
        "h3_gpu_rms_norm_bf16": (_I, [_P, _P, _P, _P, _U32, _U32, _F]),
        "h3_gpu_layer_norm_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _F]),
        "h3_gpu_head_rms_norm_bf16": (_I, [_P, _P, _P, _U32, _U32, _U32, _F]),
        "h3_gpu_qkv_rope_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P,
                                      _U32, _U32, _U32, _U32, _F]),
        "h3_gpu_grouped_qkv_rope_bf16": (_I, [_P, _P, _P, _P, _P, _P, _P, _P,
                                              _P, _U32, _U32, _U32, _U32,
                                              _F]),
        "h3_gpu_sdpa_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _F]),
        "h3_gpu_sdpa_bf16_head_major_output": (_I, [_P, _P, _P, _P, _P, _U32,
                                                    _U32, _U32, _F]),
        "h3_gpu_sdpa_cross_bf16": (_I, [_P, _P, _P, _P, _P, _U32, _U32, _U32,
                                        _U32, _F]),
        "h3_gpu_swiglu_bf16": (_I, [_P, _P, _P, _U32, _U32]),
        "h3_gpu_gelu_bf16": (_I, [_P, _P, _P, _U32, _I]),
        "h3_gpu_silu_bf16": (_I, [_P, _P, _P, _U32]),
        "h3_gpu_add_bf16": (_I, [_P, _P, _P, _P, _U32]),
        "h3_gpu_sub_bf16": (_I, [_P, _P, _P, _P, _U32]),
        "h3_gpu_cast_f32_to_bf16": (_I, [_P, _P, _P, _U32]),
        "h3_gpu_cast_bf16_to_f32": (_I, [_P, _P, _P, _U32]),
        "h3_gpu_copy_bf16": (_I, [_P, _P, _SZ, _P, _SZ, _SZ]),
        "h3_gpu_euler_bf16": (_I, [_P, _P, _SZ, _P, _P, _U32, _F, _F]),
        "h3_gpu_adaln_linear_bf16": (_I, [_P, _P, _P, _P, _SZ, _P, _P, _P,
                                          _P, _P, _U32, _U32, _U32, _U32,
                                          _U32, _U32, _F]),
        "h3_hip_patch_linear_bf16_offset": (_I, [_P, _P, _SZ, _P, _SZ, _P, _P,
                                                 _U32, _U32, _U32]),
        "h3_gpu_patch_linear_bf16_offset": (_I, [_P, _P, _SZ, _P, _SZ, _P, _P,
                                                 _U32, _U32, _U32]),
        "h3_gpu_patch_linear_bf16_map": (_I, [_P, _P, _P, _P, _P, _P, _U32,
                                              _U32, _U32, _U32]),
        "h3_gpu_fill_normal_bf16": (_I, [_P, _P, _SZ, _SZ, C.c_uint64, _F,
                                         _F]),
        "h3_gpu_fill_normal_f32": (_I, [_P, _P, _SZ, _SZ, C.c_uint64, _F,
                                        _F]),
        "h3_hip_op_timing_enable": (_I, [_P, _I]),
        "h3_hip_op_timing_reset": (_I, [_P]),
        "h3_hip_op_timing_read": (_I, [_P, C.c_char_p,
                                       C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_double)]),
        "h3_hip_op_timing_names": (_I, [_P, C.c_char_p, _SZ]),
        "h3_hip_marker": (_I, [_P, _I]),
        "h3_hip_mfma_loop": (_I, [_P, _P, _U32, C.POINTER(C.c_double)]),
        "h3_hip_marker_elapsed": (_I, [_P, _I, _I, C.POINTER(C.c_double)]),
        # DiT driver
        "h3hip_dit_create": (_P, [_P, C.POINTER(DitConfig), C.c_char_p, _SZ]),
        "h3hip_dit_free": (None, [_P]),
        "h3hip_dit_init_random": (_I, [_P, C.c_uint64, _F, _F]),
        "h3hip_dit_set_rope": (_I, [_P, _P, _P]),
        "h3hip_dit_set_row_map": (_I, [_P, _P]),
        "h3hip_dit_tensor": (_P, [_P, C.c_char_p, _U32]),
        "h3hip_dit_run_blocks": (_I, [_P, _U32, _U32]),
        "h3hip_dit_run_blocks_ops": (_I, [_P, _U32, _U32, C.c_uint]),
        "h3hip_dit_block_plain_gemm_flops": (C.c_double,
                                             [C.POINTER(DitConfig)]),
        "h3hip_dit_block_plain_gemm_launches": (_U32,
                                                [C.POINTER(DitConfig)]),
        "h3hip_dit_block_flops": (C.c_double, [C.POINTER(DitConfig)]),
        "h3hip_dit_block_class_flops": (C.c_double,
                                        [C.POINTER(DitConfig), C.c_uint]),
        "h3_gpu_grouped_qkv_linear_rope_bf16": (_I, [_P, _P, _P, _P, _P, _P,
                                                     _P, _P, _P, _P, _P,
                                                     _U32, _U32, _U32, _U32,
                                                     _U32, _F]),
        "h3hip_dit_block_gemm_flops": (C.c_double, [C.POINTER(DitConfig)]),
        "h3hip_dit_block_attention_flops": (C.c_double,
                                            [C.POINTER(DitConfig)]),
        "h3hip_dit_error": (C.c_char_p, [_P]),
        "h3hip_dit_sampler_create": (_I, [_P, C.POINTER(SamplerConfig)]),
        "h3hip_dit_sampler_init_random": (_I, [_P, C.c_uint64, _F, _F]),
        "h3hip_dit_sampler_write_latents": (_I, [_P, _P, _P]),
        "h3hip_dit_sampler_read_latents": (_I, [_P, _P, _P]),
        "h3hip_dit_forward_step": (_I, [_P, _I]),
        "h3hip_dit_denoise": (_I, [_P]),
        "h3hip_dit_schedule_precompute": (_I, [_P, C.c_uint64, _F]),
        "h3hip_dit_set_sparse_window": (C.c_long, [_P, C.POINTER(Layout),
                                                   C.c_uint, C.c_uint,
                                                   C.c_uint, C.c_uint, _I]),
        "h3hip_sparse_mask": (C.c_long, [C.POINTER(Layout), C.c_uint,
                                         C.c_uint, C.c_uint, C.c_uint, _P,
                                         _P, _SZ]),
        "h3_gpu_tensor_load_bf16": (_P, [_P, C.c_char_p, C.c_uint64, _SZ]),
        "h3_gpu_tensor_load_f32": (_P, [_P, C.c_char_p, C.c_uint64, _SZ]),
        "h3_gpu_tensor_read_file_bf16": (_I, [_P, C.c_char_p, C.c_uint64,
                                              _SZ, C.c_char_p, _SZ]),
        "h3_gpu_tensor_stream_file_bf16": (_I, [_P, C.c_char_p, C.c_uint64,
                                                _SZ, C.c_char_p, _SZ]),
        "h3_gpu_sdpa_set_sparse": (_I, [_P, _P, _SZ, _P, _SZ, _U32]),
        "h3_gpu_token_pool_bf16": (_I, [_P, _P, _P, _SZ, _P, _SZ, _P, _SZ,
                                        _P, _P, _U32, _U32, _U32, _U32]),
        "h3_gpu_token_pool_adaln_bf16": (_I, [_P, _P, _P, _P, _SZ, _P, _SZ,
                                              _P, _SZ, _P, _P, _P, _P, _P,
                                              _U32, _U32, _U32, _U32, _U32,
                                              _U32, _U32, _F]),
        "h3_gpu_token_expand_delta_bf16": (_I, [_P, _P, _P, _SZ, _P, _P, _SZ,
                                                _P, _P, _U32, _U32, _U32,
                                                _U32, _U32, _F]),
        "h3_gpu_token_expand_adaln_bf16": (_I, [_P, _P, _P, _P, _SZ, _P, _P,
                                                _SZ, _P, _P, _P, _P, _P, _U32,
                                                _U32, _U32, _U32, _U32, _F,
                                                _U32, _U32, _U32, _F]),
        "h3hip_refiner_create": (_P, [_P, _U32, _U32, _U32, _U32, _U32,
                                      C.c_char_p, _SZ]),
        "h3hip_refiner_free": (None, [_P]),
        "h3hip_refiner_error": (C.c_char_p, [_P]),
        "h3hip_refiner_tensor": (_P, [_P, C.c_char_p, _U32]),
        "h3hip_refiner_init_random": (_I, [_P, C.c_uint64, _F]),
        "h3hip_refiner_run": (_I, [_P, _P, _P, _U32]),
        "h3hip_dit_sampler_rows": (None, [_P, C.POINTER(_U32),
                                          C.POINTER(_U32), C.POINTER(_U32),
                                          C.POINTER(_U32)]),
        # host math
        "h3hip_temporal": (None, [_I, C.POINTER(_I), C.POINTER(_I),
                                  C.POINTER(_I)]),
        "h3hip_schedule_build": (_I, [_I, _P, _P]),
        "h3hip_serving_schedule_build": (_I, [_I, _P, _P]),
        "h3hip_layout_build": (_I, [_I, _I, _I, _I, _I, _I, _P, _SZ, _P, _SZ,
                                    C.POINTER(Layout), C.c_char_p, _SZ]),
        "h3hip_layout_free": (None, [C.POINTER(Layout)]),
        "h3hip_rng_seed": (None, [C.POINTER(Rng), C.c_uint64]),
        "h3hip_rng_u32": (_U32, [C.POINTER(Rng)]),
        "h3hip_rng_fill_normal": (None, [C.POINTER(Rng), _P, _SZ]),
        "h3hip_rope_tables": (None, [_P, _SZ, _P, _F, _P, _P]),
        "h3hip_default_inv_freq": (None, [_P]),
        "h3hip_time_rows": (_U32, [_I, _P, _P, _I, _I, _P, _P, _P, _P, _P]),
        "h3hip_timestep_features": (None, [_P, _U32, _P]),
        "h3hip_row_map": (_I, [C.POINTER(Layout), _U32, _U32, _U32, _U32, _P,
                               _SZ, _P, _SZ]),
        "h3hip_reuse_schedule": (_I, [_I, _I, _P, _SZ]),
        "h3hip_extrapolation_ratio": (_F, [_F, _F, _F, _I]),
        "h3hip_patchify_video": (_I, [_P, _I, _I, _I, _I, _P, _SZ]),
        "h3hip_unpatchify_video": (_I, [_P, _I, _I, _I, _I, _P, _SZ]),
        "h3hip_pack_audio": (_I, [_P, _I, _I, _P, _SZ]),
        "h3hip_unpack_audio": (_I, [_P, _I, _I, _P, _SZ]),
        "h3hip_euler_velocity_step": (_I, [_P, _P, _SZ, _F, _F]),
    }
    ns = _Prototyped()
    # H3HIP_ALLOW_MISSING=1 skips entry points an older build lacks (for
    # timing builds side by side); otherwise a missing one is an error
    allow_missing = os.environ.get("H3HIP_ALLOW_MISSING") == "1"
    for name, (res, args) in sig.items():
        if allow_missing and not hasattr(L, name):
            continue
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
        setattr(ns, name, fn)
    # the GEMM phase-trace build's extra entry points (make trace)
    for name, (res, args) in {
            "h3_hip_gemm_trace_clear": (_I, []),
            "h3_hip_gemm_trace_read": (_I, [_P, _SZ])}.items():
        if hasattr(L, name):
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
            setattr(ns, name, fn)
    _lib = ns
    return ns


class _Prototyped:
    """Only functions with a declared prototype are reachable: calling an
    undeclared one would let ctypes truncate 64-bit pointers to int."""

    def __getattr__(self, name):
        raise AttributeError(f"{name} has no ctypes prototype in h3hip.py")


def ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


# --------------------------------------------------------------- bf16 <-> f32

def f32_to_bf16(x):
    """RNE float32 -> bf16 bits (uint16), NaN kept quiet."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(x):
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32)
            << 16).view(np.float32)


# ------------------------------------------------------------------- device

class Gpu:
    """One h3_gpu context.  Tensors are raw handles (ints)."""

    def __init__(self):
        L = lib()
        err = C.create_string_buffer(512)
        self.h = L.h3_gpu_create(None, err, 512)
        if not self.h:
            raise RuntimeError("h3_gpu_create failed: " + err.value.decode())
        self.L = L
        self._owned = []

    def close(self):
        if self.h:
            for t in self._owned:
                self.L.h3_gpu_tensor_free(t)
            self._owned = []
            self.L.h3_gpu_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def error(self):
        return self.L.h3_gpu_error(self.h).decode()

    def check(self, ok, what="op"):
        if not ok:
            raise RuntimeError(f"{what} failed: {self.error()}")

    # tensors
    def bf16(self, values):
        """Upload uint16 bf16 bits (or float32 values, rounded RNE)."""
        a = np.ascontiguousarray(values)
        if a.dtype != np.uint16:
            a = f32_to_bf16(a)
        t = self.L.h3_gpu_tensor_from_bf16(self.h, ptr(a), a.size)
        self.check(t, "bf16 upload")
        self._owned.append(t)
        return t

    def f32(self, values):
        a = np.ascontiguousarray(values, dtype=np.float32)
        t = self.L.h3_gpu_tensor_from_f32(self.h, ptr(a), a.size)
        self.check(t, "f32 upload")
        self._owned.append(t)
        return t

    def u32(self, values):
        a = np.ascontiguousarray(values, dtype=np.uint32)
        t = self.L.h3_gpu_tensor_from_u32(self.h, ptr(a), a.size)
        self.check(t, "u32 upload")
        self._owned.append(t)
        return t

    def new_bf16(self, n):
        t = self.L.h3_gpu_tensor_new_bf16(self.h, n)
        self.check(t, "bf16 alloc")
        self._owned.append(t)
        return t

    def new_f32(self, n):
        t = self.L.h3_gpu_tensor_new_f32(self.h, n)
        self.check(t, "f32 alloc")
        self._owned.append(t)
        return t

    def load(self, path, offset, n, dtype="bf16"):
        """h3_gpu_tensor_load_{bf16,f32}: file bytes -> a new tensor."""
        fn = (self.L.h3_gpu_tensor_load_bf16 if dtype == "bf16"
              else self.L.h3_gpu_tensor_load_f32)
        t = fn(self.h, str(path).encode(), offset, n)
        self.check(t, f"{dtype} file load")
        self._owned.append(t)
        return t

    def read_file(self, t, path, offset, n, stream=False):
        """h3_gpu_tensor_{read,stream}_file_bf16 into an existing tensor."""
        err = C.create_string_buffer(512)
        fn = (self.L.h3_gpu_tensor_stream_file_bf16 if stream
              else self.L.h3_gpu_tensor_read_file_bf16)
        if not fn(t, str(path).encode(), offset, n, err, 512):
            raise RuntimeError("file read failed: " + err.value.decode())

    def free(self, t):
        if t in self._owned:
            self._owned.remove(t)
        self.L.h3_gpu_tensor_free(t)

    def read_bf16(self, t, n=None):
        n = self.L.h3_gpu_tensor_elements(t) if n is None else n
        out = np.empty(n, dtype=np.uint16)
        self.check(self.L.h3_gpu_tensor_read_bf16(t, ptr(out), n), "read")
        return out

    def read_f32(self, t, n=None):
        n = self.L.h3_gpu_tensor_elements(t) if n is None else n
        out = np.empty(n, dtype=np.float32)
        self.check(self.L.h3_gpu_tensor_read_f32(t, ptr(out), n), "read")
        return out

    # batches
    def begin(self):
        self.check(self.L.h3_gpu_begin(self.h), "begin")

    def submit(self):
        self.check(self.L.h3_gpu_submit(self.h), "submit")

    def run(self, name, *args):
        """begin; h3_gpu_<name>(gpu, *args); submit."""
        self.begin()
        ok = getattr(self.L, name)(self.h, *args)
        if not ok:
            msg = self.error()
            self.L.h3_gpu_submit(self.h)
            raise RuntimeError(f"{name} failed: {msg}")
        self.submit()

    def stats(self):
        s = Stats()
        self.check(self.L.h3_gpu_get_stats(self.h, C.byref(s)), "stats")
        return s


class Dit:
    """The DiT driver (h3hip_dit.h)."""

    def __init__(self, gpu, cfg):
        self.gpu = gpu
        self.cfg = cfg
        err = C.create_string_buffer(512)
        self.h = gpu.L.h3hip_dit_create(gpu.h, C.byref(cfg), err, 512)
        if not self.h:
            raise RuntimeError("h3hip_dit_create failed: " +
                               err.value.decode())

    def close(self):
        if self.h:
            self.gpu.L.h3hip_dit_free(self.h)
            self.h = None

    def error(self):
        return self.gpu.L.h3hip_dit_error(self.h).decode()

    def tensor(self, name, block=0):
        t = self.gpu.L.h3hip_dit_tensor(self.h, name.encode(), block)
        if not t:
            raise KeyError(name)
        return t

    def init_random(self, seed, weight_std=0.02, mod_std=0.02):
        if not self.gpu.L.h3hip_dit_init_random(self.h, seed, weight_std,
                                                mod_std):
            raise RuntimeError(self.error())

    def set_rope(self, cos, sin):
        c = np.ascontiguousarray(cos, dtype=np.float32)
        s = np.ascontiguousarray(sin, dtype=np.float32)
        if not self.gpu.L.h3hip_dit_set_rope(self.h, ptr(c), ptr(s)):
            raise RuntimeError(self.error())

    def set_row_map(self, row_map):
        m = np.ascontiguousarray(row_map, dtype=np.uint32)
        if not self.gpu.L.h3hip_dit_set_row_map(self.h, ptr(m)):
            raise RuntimeError(self.error())

    def write(self, name, values, block=0):
        t = self.tensor(name, block)
        a = np.ascontiguousarray(values)
        if a.dtype != np.uint16:
            a = f32_to_bf16(a)
        if not self.gpu.L.h3_gpu_tensor_write_bf16(t, ptr(a), a.size):
            raise RuntimeError(f"write {name}: {self.gpu.error()}")

    def read(self, name, block=0):
        return self.gpu.read_bf16(self.tensor(name, block))

    def run_blocks(self, first, count, submit=True):
        self.gpu.begin()
        ok = self.gpu.L.h3hip_dit_run_blocks(self.h, first, count)
        if not ok:
            msg = self.error()
            self.gpu.L.h3_gpu_submit(self.gpu.h)
            raise RuntimeError(msg)
        if submit:
            self.gpu.submit()

    def block_flops(self):
        return self.gpu.L.h3hip_dit_block_flops(C.byref(self.cfg))

    # ---- H3 sampler (h3hip_dit.h) ----
    def sampler_create(self, layout, video_sigmas, audio_sigmas,
                       reuse_interval=1, video_patch=96, audio_channels=32):
        """layout: a Layout structure (kept alive by the caller)."""
        steps = len(video_sigmas) - 1
        self._sig = (np.ascontiguousarray(video_sigmas, dtype=np.float32),
                     np.ascontiguousarray(audio_sigmas, dtype=np.float32))
        cfg = SamplerConfig(C.pointer(layout), steps,
                            self._sig[0].ctypes.data_as(C.POINTER(_F)),
                            self._sig[1].ctypes.data_as(C.POINTER(_F)),
                            reuse_interval, video_patch, audio_channels)
        if not self.gpu.L.h3hip_dit_sampler_create(self.h, C.byref(cfg)):
            raise RuntimeError(self.error())
        self.video_patch, self.audio_channels = video_patch, audio_channels

    def sampler_rows(self):
        v, a, vt, at = _U32(), _U32(), _U32(), _U32()
        self.gpu.L.h3hip_dit_sampler_rows(self.h, C.byref(v), C.byref(a),
                                          C.byref(vt), C.byref(at))
        return v.value, a.value, vt.value, at.value

    def sampler_init_random(self, seed, weight_std=0.02, mod_std=0.02):
        if not self.gpu.L.h3hip_dit_sampler_init_random(self.h, seed,
                                                        weight_std, mod_std):
            raise RuntimeError(self.error())

    def write_latents(self, video, audio):
        v = np.ascontiguousarray(video, dtype=np.float32)
        a = np.ascontiguousarray(audio, dtype=np.float32)
        if not self.gpu.L.h3hip_dit_sampler_write_latents(self.h, ptr(v),
                                                          ptr(a)):
            raise RuntimeError(self.error())

    def read_latents(self):
        vr, ar, _, _ = self.sampler_rows()
        v = np.empty(vr * self.video_patch, dtype=np.float32)
        a = np.empty(ar * self.audio_channels, dtype=np.float32)
        if not self.gpu.L.h3hip_dit_sampler_read_latents(self.h, ptr(v),
                                                         ptr(a)):
            raise RuntimeError(self.error())
        return v, a

    def forward_step(self, step, submit=True):
        self.gpu.begin()
        if not self.gpu.L.h3hip_dit_forward_step(self.h, step):
            msg = self.error()
            self.gpu.L.h3_gpu_submit(self.gpu.h)
            raise RuntimeError(msg)
        if submit:
            self.gpu.submit()

    def schedule_precompute(self, seed, weight_std=0.02):
        if not self.gpu.L.h3hip_dit_schedule_precompute(self.h, seed,
                                                        weight_std):
            raise RuntimeError(self.error())

    def denoise(self):
        n = self.gpu.L.h3hip_dit_denoise(self.h)
        if not n:
            raise RuntimeError(self.error())
        return n


def dit_config(family, hidden, heads, ffn, rows, blocks=1, text_rows=0,
               time_rows=1, head_dim=128, rope_half=48, epsilon=None):
    if epsilon is None:
        epsilon = 1e-6 if family == FAMILY_WAN else 1e-5
    return DitConfig(family, hidden, heads, head_dim, ffn, blocks, rows,
                     text_rows, time_rows, rope_half, epsilon)


def wan_positions(t, h, w):
    """(t, h, w) integer grid of the video tokens in row-major token order
    (the patchified latent's order), as float64 [rows][3]."""
    tt, hh, ww = np.meshgrid(np.arange(t), np.arange(h), np.arange(w),
                             indexing="ij")
    pos = np.stack([tt.ravel(), hh.ravel(), ww.ravel()], axis=1)
    return pos.astype(np.float64)


def rope_tables(positions, scale=1.0):
    """3D RoPE cos/sin tables [rows][48] (F32) for the given positions, from
    the backend's host math (h3hip_rope_tables, the reference's
    prepare_rope table, h3_dit.c:907-922)."""
    L = lib()
    rows = positions.shape[0]
    inv = np.empty(16, np.float32)
    L.h3hip_default_inv_freq(ptr(inv))
    pos = np.ascontiguousarray(positions, dtype=np.float64)
    cos = np.empty(rows * 48, np.float32)
    sin = np.empty(rows * 48, np.float32)
    L.h3hip_rope_tables(ptr(pos), rows, ptr(inv), scale, ptr(cos), ptr(sin))
    return cos, sin


def block_flops(cfg):
    """FLOPs of one block (host math only, no device needed)."""
    return lib().h3hip_dit_block_flops(C.byref(cfg))


class Refiner:
    """The text token refiner (h3hip_refiner_*)."""

    def __init__(self, gpu, hidden, heads, ffn, text_dim, head_dim=128):
        self.gpu = gpu
        err = C.create_string_buffer(512)
        self.h = gpu.L.h3hip_refiner_create(gpu.h, hidden, heads, head_dim,
                                            ffn, text_dim, err, 512)
        if not self.h:
            raise RuntimeError("h3hip_refiner_create failed: " +
                               err.value.decode())

    def close(self):
        if self.h:
            self.gpu.L.h3hip_refiner_free(self.h)
            self.h = None

    def _check(self, ok, what):
        if not ok:
            raise RuntimeError(what + ": " +
                               self.gpu.L.h3hip_refiner_error(self.h).decode())

    def tensor(self, name, block=0):
        t = self.gpu.L.h3hip_refiner_tensor(self.h, name.encode(), block)
        if not t:
            raise KeyError(name)
        return t

    def read(self, name, block=0):
        return self.gpu.read_bf16(self.tensor(name, block))

    def init_random(self, seed, weight_std=0.02):
        self._check(self.gpu.L.h3hip_refiner_init_random(self.h, seed,
                                                         weight_std), "init")

    def run(self, output, source, rows):
        self._check(self.gpu.L.h3hip_refiner_run(self.h, output, source,
                                                 rows), "refiner run")


def safetensors_index(path):
    """Tensor name -> (dtype, shape, absolute byte offset, byte count) from a
    safetensors header: an 8-byte little-endian length, then that many bytes
    of JSON whose data_offsets are relative to the end of the header (the
    format h3_weights.c reads)."""
    import json
    import struct
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
    base = 8 + n
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        a, b = info["data_offsets"]
        out[name] = (info["dtype"], tuple(info["shape"]), base + a, b - a)
    return out
