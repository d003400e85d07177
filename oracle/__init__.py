"""CPU oracle for the attention stage — TEST INFRASTRUCTURE ONLY.

A C restatement of the reference's fp32 math (src/hippo_leap/tensor.nim and
the attention semantics of backends/naive.nim; every function in
hl_oracle.c cites the lines it follows).  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it, always as the checker or the timed
CPU baseline; the product library (hippo_leap_amd) never calls it.

The reference itself is Nim (no nim toolchain in this image) and cannot be
built here, so there is no oracle/_ref build.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")
F32, F16, BF16, FP8 = 0, 1, 2, 3

_lib = None
_fp = ctypes.POINTER(ctypes.c_float)
_i, _f, _ll, _u64 = ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_uint64


def build() -> str:
    """Compiles hl_oracle.c with gcc -O2 (recipe: oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "-B", "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_fill_uniform": (None, [_fp, _ll, _u64, _f, _f]),
            "orc_fill_normal": (None, [_fp, _ll, _u64, _f, _f]),
            "orc_half_to_float": (_f, [ctypes.c_uint16]),
            "orc_float_to_half_trunc": (ctypes.c_uint16, [_f]),
            "orc_float_to_half_rne": (ctypes.c_uint16, [_f]),
            "orc_bf16_to_float": (_f, [ctypes.c_uint16]),
            "orc_float_to_bf16_rne": (ctypes.c_uint16, [_f]),
            "orc_convert_from_f32": (None, [_i, _fp, ctypes.c_void_p, _ll]),
            "orc_upcast_to_f32": (None, [_i, ctypes.c_void_p, _fp, _ll]),
            "orc_matmul": (None, [_fp, _fp, _fp, _i, _i, _i]),
            "orc_softmax_last_dim": (None, [_fp, _fp, _ll, _i]),
            "orc_rmsnorm": (None, [_fp, _fp, _fp, _ll, _i, _f]),
            "orc_rmsnorm_cols": (None, [_fp, _fp, _fp, _i, _i, _f]),
            "orc_rope_inplace": (None, [_fp, _ll, _i, _i, _f, _i]),
            "orc_rope_theta_table": (None, [_fp, _i, _f]),
            "orc_rope_heads": (None, [_fp, _i, _i, _i, _fp, _i, _i]),
            "orc_rope_cols": (None, [_fp, _i, _i, _i, _i, _fp, _i, _i]),
            "orc_qk_norm": (None, [_fp, _fp, _i, _i, _f]),
            "orc_qk_norm_cols": (None, [_fp, _fp, _i, _i, _i, _f]),
            "orc_store_kv": (None, [ctypes.c_void_p, _i, _fp, _i, _i, _i, _i]),
            "orc_attention_decode": (None, [_fp, _fp, _fp, _fp, _i, _i, _i, _i, _i, _f, _fp]),
            "orc_argmax": (_i, [_fp, _ll]),
            "orc_dequant_rows": (_ll, [_i, ctypes.c_void_p, _fp, _i, _i]),
            "orc_embedding": (None, [_fp, ctypes.POINTER(_i), _fp, _i, _i]),
            "orc_add": (None, [_fp, _fp, _fp, _ll]),
            "orc_silu_mul": (None, [_fp, _fp, _fp, _ll]),
            "orc_attention_prefill": (None, [_fp, _fp, _fp, _fp, _i, _i, _i, _i, _f, _i, _i, _i,
                                             _i, _i, _fp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_fp)


# ---- generators -----------------------------------------------------------
def uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform(_ptr(out), n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(_ptr(out), n, seed, mean, std)
    return out


# ---- storage conversions ----------------------------------------------------
def to_storage(x: np.ndarray, dtype: int) -> np.ndarray:
    """fp32 -> stored bits (float32 array for F32, uint16 bits otherwise), RNE."""
    x = _f32(x)
    if dtype == F32:
        return x.copy()
    out = np.empty(x.shape, np.uint8 if dtype == FP8 else np.uint16)
    lib().orc_convert_from_f32(dtype, _ptr(x), out.ctypes.data_as(ctypes.c_void_p), x.size)
    return out


def upcast(bits: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F32:
        return _f32(bits).copy()
    bits = np.ascontiguousarray(bits, dtype=np.uint8 if dtype == FP8 else np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_upcast_to_f32(dtype, bits.ctypes.data_as(ctypes.c_void_p), _ptr(out), bits.size)
    return out


def half_to_float(h: int) -> float:
    return lib().orc_half_to_float(h)


def float_to_half_trunc(f: float) -> int:
    return lib().orc_float_to_half_trunc(f)


# ---- tensor.nim ops -------------------------------------------------------------
def matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().orc_matmul(_ptr(a), _ptr(b), _ptr(c), m, k, n)
    return c


def softmax_last_dim(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_softmax_last_dim(_ptr(x), _ptr(out), x.size // x.shape[-1], x.shape[-1])
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_ptr(x), _ptr(w), _ptr(out), x.size // x.shape[-1], x.shape[-1], eps)
    return out


def rmsnorm_cols(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm_cols(_ptr(x), _ptr(w), _ptr(out), x.shape[0], x.shape[1], eps)
    return out


def rope_inplace(x: np.ndarray, base: float, start_pos: int = 0) -> np.ndarray:
    """tensor.nim ropeInplace on [..., seq, dim]; returns a rotated copy."""
    x = _f32(x).copy()
    dim, seq = x.shape[-1], x.shape[-2]
    lib().orc_rope_inplace(_ptr(x), x.size // (seq * dim), seq, dim, base, start_pos)
    return x


# ---- naive.nim semantics --------------------------------------------------------
def theta_table(rope_dim: int, base: float) -> np.ndarray:
    out = np.empty(rope_dim // 2, np.float32)
    lib().orc_rope_theta_table(_ptr(out), rope_dim, base)
    return out


def rope_heads(x: np.ndarray, n_head: int, head_dim: int, rope_dim: int, theta: np.ndarray,
               pos: int, style: int = 0) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_rope_heads(_ptr(x), n_head, head_dim, rope_dim, _ptr(_f32(theta)), pos, style)
    return x


def rope_cols(x: np.ndarray, n_head: int, head_dim: int, seq: int, rope_dim: int,
              theta: np.ndarray, pos0: int = 0, style: int = 0) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_rope_cols(_ptr(x), n_head, head_dim, seq, rope_dim, _ptr(_f32(theta)), pos0, style)
    return x


def qk_norm(x: np.ndarray, w: np.ndarray, n_head: int, head_dim: int, eps: float) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_qk_norm(_ptr(x), _ptr(_f32(w)), n_head, head_dim, eps)
    return x


def qk_norm_cols(x: np.ndarray, w: np.ndarray, n_head: int, head_dim: int, seq: int,
                 eps: float) -> np.ndarray:
    x = _f32(x).copy()
    lib().orc_qk_norm_cols(_ptr(x), _ptr(_f32(w)), n_head, head_dim, seq, eps)
    return x


def store_kv(cache: np.ndarray, dtype: int, src: np.ndarray, rows: int, src_cols: int,
             cache_cols: int, start_pos: int) -> None:
    assert cache.flags.c_contiguous
    lib().orc_store_kv(cache.ctypes.data_as(ctypes.c_void_p), dtype, _ptr(_f32(src)), rows,
                       src_cols, cache_cols, start_pos)


def attention_decode(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, n_head: int,
                     n_head_kv: int, head_dim: int, L: int, max_len: int,
                     scale: float | None = None) -> np.ndarray:
    """One sequence; fp32 caches [Hkv*D, max_len]; returns [Hq*D]."""
    q, kc, vc = _f32(q), _f32(k_cache), _f32(v_cache)
    out = np.empty(n_head * head_dim, np.float32)
    scores = np.empty(L, np.float32)
    s = np.float32(1.0) / np.sqrt(np.float32(head_dim)) if scale is None else scale
    lib().orc_attention_decode(_ptr(q), _ptr(kc), _ptr(vc), _ptr(out), n_head, n_head_kv,
                               head_dim, L, max_len, float(s), _ptr(scores))
    return out


def attention_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_head: int, n_head_kv: int,
                      head_dim: int, T: int, scale: float | None = None, heads=None,
                      rows=None) -> np.ndarray:
    """Col-major q [Hq*D, T], k/v [Hkv*D, T] fp32; returns O [Hq*D, T] (NaN where
    not computed).  heads=(h0,h1), rows=(r0,r1,step) select a subset."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.full((n_head * head_dim, T), np.nan, np.float32)
    scores = np.empty(T, np.float32)
    s = np.float32(1.0) / np.sqrt(np.float32(head_dim)) if scale is None else scale
    h0, h1 = heads if heads is not None else (0, n_head)
    r0, r1, rs = rows if rows is not None else (0, T, 1)
    lib().orc_attention_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n_head, n_head_kv, head_dim,
                                T, float(s), h0, h1, r0, r1, rs, _ptr(scores))
    return out


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """tensor.nim add (:42-47)."""
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    out = np.empty_like(a)
    lib().orc_add(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """gpuSiluMul (naive.nim:2179-2187): gate * (1 / (1 + exp(-gate))) * up."""
    g, u = _f32(gate), _f32(up)
    assert g.shape == u.shape
    out = np.empty_like(g)
    lib().orc_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


# ---- decode-step ends (naive.nim) ----------------------------------------------
def argmax(x: np.ndarray) -> int:
    """gpuArgmax's result (naive.nim:1922-2127), reduction tree and all."""
    x = _f32(x).reshape(-1)
    return lib().orc_argmax(_ptr(x), x.size)


def embedding(w: np.ndarray, tokens, n_emb: int) -> np.ndarray:
    """gpuEmbedding (naive.nim:2975-3001): col-major [n_emb, n_tokens]."""
    w = _f32(w).reshape(-1)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.empty((n_emb, tok.size), np.float32)
    lib().orc_embedding(_ptr(w), tok.ctypes.data_as(ctypes.POINTER(_i)), _ptr(out), n_emb,
                        tok.size)
    return out


# ---- GGUF weight rows (quant.nim) -------------------------------------------------
def dequant_rows(qtype: int, raw: np.ndarray, rows: int, k: int) -> np.ndarray:
    """quant.nim's dequantRow* of `rows` rows of GGUF type qtype -> fp32 [rows, k]."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((rows, k), np.float32)
    rb = lib().orc_dequant_rows(qtype, raw.ctypes.data_as(ctypes.c_void_p), _ptr(out), rows, k)
    assert rb and raw.size >= rb * rows
    return out
