"""ctypes binding of libhl_attn.so (declarations mirror include/hl_attn.h).

The library is loaded from this package directory only; a missing library is
an error (there is no CPU fallback for any entry point).
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libhl_attn.so")

HL_OK, HL_EINVAL, HL_ECAPACITY, HL_EUNSUPPORTED, HL_EHIP, HL_ECAPTURE = 0, -1, -2, -3, -4, -5
HL_F32, HL_F16, HL_BF16, HL_FP8 = 0, 1, 2, 3
HL_ROPE_HALF_SPLIT, HL_ROPE_INTERLEAVED = 0, 1
HL_KV_COLMAJOR, HL_KV_TILED32, HL_KV_PAGED32 = 0, 1, 2
HL_GGML_F16, HL_GGML_Q5_0, HL_GGML_Q5_1, HL_GGML_Q8_0 = 1, 6, 7, 8
HL_GGML_Q2_K, HL_GGML_Q3_K, HL_GGML_Q4_K, HL_GGML_Q5_K, HL_GGML_Q6_K = 10, 11, 12, 13, 14
HL_GGML_IQ4_NL = 20

c_int, c_float, c_void_p, c_size_t, c_longlong = (
    ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_longlong)


class HLError(ValueError):
    """Raised for a negative status; the reference raises ValueError for the
    same preconditions (backends/naive.nim:3969-3976, 4594-4599)."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("device", c_int), ("cu_count", c_int), ("clock_khz", c_int),
        ("mem_clock_khz", c_int), ("l2_bytes", c_int), ("hbm_bytes", c_size_t),
        ("hbm_peak_gbs", ctypes.c_double), ("bf16_dense_tflops", ctypes.c_double),
        ("fp32_tflops", ctypes.c_double), ("arch", ctypes.c_char * 64),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_int), ("n_head", c_int), ("n_head_kv", c_int), ("head_dim", c_int),
        ("kv_dtype", c_int), ("max_len", c_int), ("seq_len", c_int),
        ("seq_lens", c_void_p), ("cache_batch_stride", c_longlong),
        ("q", c_void_p), ("k_cache", c_void_p), ("v_cache", c_void_p), ("out", c_void_p),
        ("scale", c_float), ("num_splits", c_int), ("kv_layout", c_int),
        ("block_table", c_void_p), ("blocks_per_seq", c_int),
    ]


class RopeStoreArgs(ctypes.Structure):
    _fields_ = [
        ("batch", c_int), ("n_head_q", c_int), ("n_head_kv", c_int), ("head_dim", c_int),
        ("rope_dim", c_int), ("rope_style", c_int), ("rope_base", c_float),
        ("use_installed_theta", c_int), ("kv_dtype", c_int), ("max_len", c_int),
        ("cache_batch_stride", c_longlong),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("k_cache", c_void_p), ("v_cache", c_void_p),
        ("positions", c_void_p), ("pos", c_int),
        ("q_norm_w", c_void_p), ("k_norm_w", c_void_p), ("eps", c_float),
        ("kv_layout", c_int), ("block_table", c_void_p), ("blocks_per_seq", c_int),
    ]


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "wq", "wk", "wv",
                                        "wo", "w_gate", "w_up", "w_down")] + \
               [(n, c_int) for n in ("wq_type", "wk_type", "wv_type", "wo_type", "w_gate_type",
                                     "w_up_type", "w_down_type")] + \
               [("k_cache", c_void_p), ("v_cache", c_void_p)]


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("n_layer", "n_emb", "n_head", "n_head_kv", "head_dim",
                                     "rope_dim", "n_ff", "n_vocab", "max_len")] + \
               [("rms_eps", c_float), ("rope_base", c_float), ("tok_emb", c_void_p),
                ("output_norm", c_void_p), ("output", c_void_p), ("output_type", c_int),
                ("layers", ctypes.POINTER(LayerDesc))]


class DecodeScratch(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("x", "x_norm", "tmp0", "tmp1", "tmp2")]


class KvCacheDesc(ctypes.Structure):
    _fields_ = [(n, c_int) for n in ("n_layer", "n_head_kv", "head_dim", "max_len", "kv_dtype",
                                     "kv_layout")] + \
               [("k", ctypes.POINTER(c_void_p)), ("v", ctypes.POINTER(c_void_p)),
                ("block_table", c_void_p), ("blocks_per_seq", c_int), ("cur_len", c_int)]


class ForwardScratch(ctypes.Structure):
    _fields_ = [("max_tokens", c_int)] + [(n, c_void_p) for n in ("x", "x_norm", "tmp0", "tmp1", "tmp2",
                                                                    "workspace")] + \
               [("workspace_bytes", c_size_t)]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("n_head", c_int), ("n_head_kv", c_int), ("head_dim", c_int), ("seq_len", c_int),
        ("io_dtype", c_int),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("out", c_void_p),
        ("q_norm_w", c_void_p), ("k_norm_w", c_void_p), ("eps", c_float),
        ("apply_rope", c_int), ("rope_dim", c_int), ("rope_style", c_int),
        ("rope_base", c_float), ("use_installed_theta", c_int),
        ("k_cache", c_void_p), ("v_cache", c_void_p), ("kv_dtype", c_int),
        ("max_len", c_int), ("start_pos", c_int), ("scale", c_float),
        ("write_back_qk", c_int), ("out_dtype", c_int), ("kv_layout", c_int),
        ("block_table", c_void_p),
    ]


# name -> (restype, argtypes); every symbol include/hl_attn.h declares.
SIGNATURES = {
    "hl_last_error": (ctypes.c_char_p, []),
    "hl_abi_version": (c_int, []),
    "hl_device_info_get": (c_int, [ctypes.POINTER(DeviceInfo)]),
    "hl_rope_theta_table": (c_int, [ctypes.POINTER(c_float), c_int, c_float]),
    "hl_set_rope_theta": (c_int, [c_int, c_float]),
    "hl_gpu_qk_norm": (c_int, [c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "hl_gpu_qk_norm_prefill": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_float, c_void_p]),
    "hl_gpu_rope_at_pos": (c_int, [c_void_p, c_int, c_int, c_int, c_float, c_int, c_int, c_void_p]),
    "hl_gpu_rope_at_pos_theta": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_rope_qk_decode": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_float, c_int,
                                      c_void_p]),
    "hl_gpu_fused_rope_store_kv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                           c_int, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_store_kv": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_store_kv_pair": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                     c_int, c_void_p]),
    "hl_gpu_attention_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                        c_int, c_int, c_void_p]),
    "hl_gpu_attention_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                        c_int, c_int, c_void_p]),
    "hl_gpu_attention_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                         c_int, c_void_p]),
    "hl_gpu_linear_col": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_linear_col_quant": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_rmsnorm_cols": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_void_p]),
    "hl_gpu_residual_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_float,
                                        c_void_p]),
    "hl_gpu_argmax": (c_int, [c_void_p, c_int, ctypes.POINTER(ctypes.c_int32), c_void_p]),
    "hl_argmax_async": (c_int, [c_void_p, c_int, c_void_p, c_void_p]),
    "hl_gpu_embedding": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "hl_gpu_silu_mul": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "hl_gpu_fused_gate_up_silu_quant": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                                c_int, c_void_p]),
    "hl_gpu_fused_kv_linear_quant": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                             c_int, c_int, c_int, c_void_p]),
    "hl_gpu_fused_gate_up_silu_q4k": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                              c_void_p]),
    "hl_gpu_fused_gate_up_silu_q3k": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                              c_void_p]),
    "hl_gpu_fused_kv_linear_q4k": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                           c_int, c_void_p]),
    "hl_gpu_fused_kv_linear_q2k_q3k": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                               c_int, c_void_p]),
    "hl_gpu_add": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "hl_forward_decode_token": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(DecodeScratch),
                                        c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "hl_kv_cache_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "hl_kv_cache_preferred_layout": (c_int, [c_int, c_int]),
    "hl_kv_cache_init": (c_int, [ctypes.POINTER(KvCacheDesc), ctypes.POINTER(ModelDesc)]),
    "hl_forward_workspace_bytes": (c_size_t, [ctypes.POINTER(ModelDesc), ctypes.POINTER(KvCacheDesc), c_int]),
    "hl_forward_prefill": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(KvCacheDesc),
                                   ctypes.POINTER(ForwardScratch), c_void_p, c_int, c_void_p, c_void_p]),
    "hl_forward_decode": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(KvCacheDesc),
                                  ctypes.POINTER(ForwardScratch), c_void_p, c_void_p, c_void_p, c_void_p]),
    "hl_forward_decode_timed": (c_int, [ctypes.POINTER(ModelDesc), ctypes.POINTER(KvCacheDesc),
                                        ctypes.POINTER(ForwardScratch), c_void_p, c_void_p, c_void_p,
                                        ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(c_float), c_void_p]),
    "hl_attn_decode_workspace_bytes": (c_size_t, [ctypes.POINTER(DecodeArgs)]),
    "hl_attn_decode": (c_int, [ctypes.POINTER(DecodeArgs), c_void_p, c_size_t, c_void_p]),
    "hl_attn_decode_workspace_init": (c_int, [c_void_p, c_size_t, c_void_p]),
    "hl_rope_store_decode": (c_int, [ctypes.POINTER(RopeStoreArgs), c_void_p]),
    "hl_decode_step_workspace_bytes": (c_size_t, [ctypes.POINTER(RopeStoreArgs),
                                                  ctypes.POINTER(DecodeArgs)]),
    "hl_decode_step": (c_int, [ctypes.POINTER(RopeStoreArgs), ctypes.POINTER(DecodeArgs), c_void_p,
                               c_size_t, c_void_p]),
    "hl_attn_prefill_workspace_bytes": (c_size_t, [ctypes.POINTER(PrefillArgs)]),
    "hl_attn_prefill": (c_int, [ctypes.POINTER(PrefillArgs), c_void_p, c_size_t, c_void_p]),
    "hl_attn_prefill_fallback_ran": (c_int, [ctypes.POINTER(PrefillArgs), c_void_p,
                                             ctypes.POINTER(c_int), c_void_p]),
    "hl_probe_stream_read": (c_int, [c_void_p, c_size_t, c_int, c_void_p, c_void_p]),
    "hl_probe_stream_read_ex": (c_int, [c_void_p, c_size_t, c_int, c_int, c_int, c_void_p, c_void_p]),
    "hl_kv_cache_to_f32": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads libhl_attn.so from the package directory (raises if it is absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m hippo_leap_amd.build` "
            "(the attention stage has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != HL_OK:
        msg = load().hl_last_error().decode(errors="replace")
        raise HLError(rc, msg)
