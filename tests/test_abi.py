"""C-ABI checks that need no GPU: exports match include/hl_attn.h, and the
argument validation that runs before any HIP call reproduces the reference's
host prechecks (backends/naive.nim:3969-3976, 4594-4599) as status codes."""
import ctypes
import os
import re

import numpy as np
import pytest

from hippo_leap_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "hl_attn.h")
FAKE = 1 << 20  # a non-null, 16-byte aligned pointer value; validation never dereferences it


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(hl_\w+)\s*\(", text))


def test_exports_match_header(hl):
    declared = header_functions()
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(hl, name), name


def test_abi_version(hl):
    assert hl.hl_abi_version() == 3


def _err(hl):
    return hl.hl_last_error().decode()


def _decode_args(**kw):
    a = _lib.DecodeArgs()
    a.batch, a.n_head, a.n_head_kv, a.head_dim = 1, 32, 8, 64
    a.kv_dtype, a.max_len, a.seq_len = _lib.HL_F16, 2049, 2049
    a.q = a.k_cache = a.v_cache = a.out = FAKE
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_decode_gqa_divisibility(hl):
    a = _decode_args(n_head=6, n_head_kv=4)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert _err(hl) == "GQA requires head_count divisible by head_count_kv"


def test_decode_cache_full(hl):
    a = _decode_args(seq_len=2050)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_ECAPACITY
    assert _err(hl) == "KV cache full"
    assert hl.hl_gpu_attention_decode(FAKE, FAKE, FAKE, FAKE, 32, 4, 64, 513, 512, None) == \
        _lib.HL_ECAPACITY


def test_decode_unsupported_head_dim(hl):
    a = _decode_args(head_dim=96)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EUNSUPPORTED


def test_decode_workspace_required(hl):
    a = _decode_args()
    need = hl.hl_attn_decode_workspace_bytes(ctypes.byref(a))
    assert need > 0
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "workspace" in _err(hl)
    # one 4-byte arrival counter per (sequence, kv head), padded to 256 bytes,
    # then (D + 2) floats per split per query head per sequence
    assert (need - 256) % ((64 + 2) * 4 * 32) == 0
    assert hl.hl_attn_decode(ctypes.byref(a), FAKE + 2, need, None) == _lib.HL_EINVAL
    assert "4-byte aligned" in _err(hl)


def test_decode_null_pointer(hl):
    a = _decode_args(q=None)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL


def _prefill_args(**kw):
    a = _lib.PrefillArgs()
    a.n_head, a.n_head_kv, a.head_dim, a.seq_len = 32, 8, 128, 4096
    a.io_dtype = _lib.HL_BF16
    a.q = a.k = a.v = a.out = FAKE
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_prefill_empty(hl):
    a = _prefill_args(seq_len=0)
    assert hl.hl_attn_prefill(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert _err(hl) == "prefill requires at least one token"


def test_prefill_exceeds_cache(hl):
    a = _prefill_args(k_cache=FAKE, v_cache=FAKE, kv_dtype=_lib.HL_BF16, max_len=4095)
    assert hl.hl_attn_prefill(ctypes.byref(a), None, 0, None) == _lib.HL_ECAPACITY
    assert _err(hl) == "prefill exceeds KV cache capacity"
    a = _prefill_args(k_cache=FAKE, v_cache=FAKE, kv_dtype=_lib.HL_BF16, max_len=5000,
                      start_pos=1000)
    assert hl.hl_attn_prefill(ctypes.byref(a), None, 0, None) == _lib.HL_ECAPACITY


def test_prefill_gqa(hl):
    a = _prefill_args(n_head=30)
    assert hl.hl_attn_prefill(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert _err(hl) == "GQA requires head_count divisible by head_count_kv"


def test_prefill_workspace_size(hl):
    a = _prefill_args()
    # kt [Hkv][T][D] + vt [Hkv][D][T] fp16 (the MFMA kernel builds Q itself),
    # the fallback's fp32 Q, K, V ([Hq*D, T], [Hkv*D, T] x 2), then the
    # 16-byte range record of the call
    fb = (32 + 8 + 8) * 4096 * 128 * 4
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(a)) == (8 + 8) * 4096 * 128 * 2 + fb + 16
    # with RoPE: plus the (cos, sin) table [rope_dim/2][T] of float2
    r = _prefill_args(apply_rope=1, rope_base=5e5)
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(r)) == \
        (8 + 8) * 4096 * 128 * 2 + 4096 * 64 * 8 + fb + 16
    # half-split RoPE over part of the head: Q is prepared ahead, qt [Hq][T][D]
    h = _prefill_args(apply_rope=1, rope_base=5e5, rope_dim=64)
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(h)) == \
        (32 + 8 + 8) * 4096 * 128 * 2 + 4096 * 32 * 8 + fb + 16
    # fp32: no fused ops, only the K/V split images, 64 keys x D dims x (K, V)
    # x (hi, lo) fp16 per tile, then a record of 8 ints (shifts and flags of
    # its two halves) per tile (4096 tokens: 64 tiles per kv head)
    f = _prefill_args(io_dtype=_lib.HL_F32)
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(f)) == 8 * 64 * (64 * 128 * 8 + 32)
    # head dim 64, 1000 tokens (16 tiles), after the roped Q and K (256-aligned)
    s = _prefill_args(io_dtype=_lib.HL_F32, head_dim=64, seq_len=1000, n_head_kv=4)
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(s)) == 4 * 16 * (32768 + 32)
    sr = _prefill_args(io_dtype=_lib.HL_F32, head_dim=64, seq_len=1000, n_head_kv=4, apply_rope=1, rope_base=1e4)
    qk = (32 + 4) * 64 * 1000 * 4
    assert hl.hl_attn_prefill_workspace_bytes(ctypes.byref(sr)) == (qk + 255) // 256 * 256 + 4 * 16 * (32768 + 32)
    # and hl_attn_prefill asks for it
    assert hl.hl_attn_prefill(ctypes.byref(s), None, 0, None) == _lib.HL_EINVAL
    assert "workspace of 2099200 bytes needed" in _err(hl)


def test_rope_store_cache_full(hl):
    a = _lib.RopeStoreArgs()
    a.batch, a.n_head_q, a.n_head_kv, a.head_dim = 1, 32, 4, 128
    a.rope_base, a.kv_dtype, a.max_len, a.pos = 1e6, _lib.HL_BF16, 100, 100
    a.q = a.k = a.v = a.k_cache = a.v_cache = FAKE
    assert hl.hl_rope_store_decode(ctypes.byref(a), None) == _lib.HL_ECAPACITY
    assert _err(hl) == "KV cache full"
    assert hl.hl_gpu_fused_rope_store_kv(FAKE, FAKE, FAKE, FAKE, FAKE, 32, 4, 64, 64, 256, 512,
                                         512, None) == _lib.HL_ECAPACITY


def test_rope_dim_checks(hl):
    assert hl.hl_gpu_rope_at_pos(FAKE, 4, 64, 63, 1e4, 0, 1, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_rope_at_pos(FAKE, 4, 64, 66, 1e4, 0, 1, None) == _lib.HL_EINVAL


def test_theta_table_matches_oracle(hl, orc):
    for rd, base in ((64, 1e4), (64, 5e5), (128, 1e6)):
        buf = (ctypes.c_float * (rd // 2))()
        assert hl.hl_rope_theta_table(buf, rd, base) == 0
        assert np.array_equal(np.array(buf, np.float32), orc.theta_table(rd, base))


def test_installed_theta_dim_mismatch(hl):
    assert hl.hl_set_rope_theta(64, 1e4) == 0
    assert hl.hl_gpu_rope_at_pos_theta(FAKE, 4, 128, 128, 0, 1, None) == _lib.HL_EINVAL
    assert "theta" in _err(hl)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libhl_attn.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_kv_layout_validation(hl):
    """Tiled caches: fp16/bf16, max_len % 32 == 0, aligned; unknown layouts
    are rejected (decode, rope/store and prefill alike)."""
    T = _lib.HL_KV_TILED32
    a = _decode_args(kv_layout=T)  # max_len 2049
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "max_len % 32" in _err(hl)
    a = _decode_args(kv_layout=T, max_len=2080, kv_dtype=_lib.HL_F32)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EUNSUPPORTED
    a = _decode_args(kv_layout=T, max_len=2080, k_cache=FAKE + 8)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "aligned" in _err(hl)
    a = _decode_args(kv_layout=7)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "kv_layout" in _err(hl)
    a = _decode_args(kv_layout=T, max_len=2080)
    assert hl.hl_attn_decode_workspace_bytes(ctypes.byref(a)) > 0  # valid: plans normally

    r = _lib.RopeStoreArgs()
    r.batch, r.n_head_q, r.n_head_kv, r.head_dim = 1, 32, 4, 128
    r.rope_base, r.kv_dtype, r.max_len, r.pos = 1e6, _lib.HL_BF16, 100, 10
    r.q = r.k = r.v = r.k_cache = r.v_cache = FAKE
    r.kv_layout = T
    assert hl.hl_rope_store_decode(ctypes.byref(r), None) == _lib.HL_EINVAL
    assert "max_len % 32" in _err(hl)

    p = _prefill_args(k_cache=FAKE, v_cache=FAKE, kv_dtype=_lib.HL_F32, max_len=4096,
                      kv_layout=T)
    assert hl.hl_attn_prefill(ctypes.byref(p), None, 0, None) == _lib.HL_EUNSUPPORTED
    p = _prefill_args(kv_layout=3)
    assert hl.hl_attn_prefill(ctypes.byref(p), None, 0, None) == _lib.HL_EINVAL


def test_struct_sizes_match_header(tmp_path):
    """ctypes mirrors of the argument structs have the C compiler's size and
    kv_layout offset (the field the ABI version 2 added)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "sz.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "hl_attn.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu %zu\\n",'
                   ' sizeof(hl_decode_args), offsetof(hl_decode_args, kv_layout),'
                   ' sizeof(hl_rope_store_args), offsetof(hl_rope_store_args, kv_layout),'
                   ' sizeof(hl_prefill_args), offsetof(hl_prefill_args, kv_layout)); return 0; }\n')
    exe = tmp_path / "sz"
    subprocess.check_call([cc, "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)])
    got = [int(x) for x in subprocess.check_output([str(exe)], text=True).split()]
    want = []
    for cls in (_lib.DecodeArgs, _lib.RopeStoreArgs, _lib.PrefillArgs):
        want += [ctypes.sizeof(cls), cls.kv_layout.offset]
    assert got == want


def test_kv_layout_helpers_match_header_formula():
    """kv_to_tiled / kv_from_tiled (host side of HL_KV_TILED32) place element
    (sequence b, kv head h, row d, column t) at
    b*Hkv*D*M + h*D*M + ((t/32)*D + d)*32 + t%32, as the header states."""
    import torch
    from hippo_leap_amd import attention as A
    B, H, D, M = 2, 3, 8, 96
    x = torch.arange(B * H * D * M, dtype=torch.int32).reshape(B, H * D, M)
    t = A.kv_to_tiled(x, H, D, M).reshape(-1)
    rng = np.random.default_rng(5)
    for _ in range(200):
        b, h, d, c = (int(rng.integers(n)) for n in (B, H, D, M))
        assert t[b * H * D * M + h * D * M + ((c // 32) * D + d) * 32 + c % 32] == x[b, h * D + d, c]
    assert torch.equal(A.kv_from_tiled(A.kv_to_tiled(x, H, D, M), H, D, M), x)


def test_linear_col_validation(hl):
    """gpuLinearCol's arguments: shapes must be positive, dst may not alias
    the input it reads (the reference's in-place call, naive.nim:4115, races)."""
    F = FAKE
    assert hl.hl_gpu_linear_col(None, F, F, 64, 64, 1, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_linear_col(F, F + (1 << 24), F + (1 << 25), 0, 64, 1, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_linear_col(F, F + (1 << 24), F + (1 << 25), 64, 64, 0, None) == _lib.HL_EINVAL
    # dst [64, 8] overlaps x [64, 8] by one float; then dst inside w
    assert hl.hl_gpu_linear_col(F, F + 64 * 8 * 4 - 4, F + (1 << 25), 64, 64, 8, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_linear_col(F + 4096, F + (1 << 24), F, 64, 64, 1, None) == _lib.HL_EINVAL
    assert b"overlaps" in hl.hl_last_error()


def test_argmax_embedding_validation(hl):
    out = ctypes.c_int32(0)
    assert hl.hl_gpu_argmax(None, 10, ctypes.byref(out), None) == _lib.HL_EINVAL
    assert hl.hl_gpu_argmax(FAKE, -1, ctypes.byref(out), None) == _lib.HL_EINVAL
    assert hl.hl_argmax_async(FAKE, 10, None, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_embedding(FAKE, FAKE, FAKE, 0, 1, 10, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_embedding(FAKE, None, FAKE, 64, 1, 10, None) == _lib.HL_EINVAL


def test_rmsnorm_validation(hl):
    assert hl.hl_gpu_rmsnorm_cols(FAKE, FAKE, None, 64, 1, 1e-5, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_rmsnorm_cols(FAKE, FAKE, FAKE, 0, 1, 1e-5, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_rmsnorm_cols(FAKE + 4, FAKE, FAKE + (1 << 24), 64, 2, 1e-5, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_residual_rmsnorm(FAKE, FAKE + 64, FAKE + 4096, FAKE + 8192, 64, 1e-6,
                                      None) == _lib.HL_EINVAL


def test_fp8_kv_validation(hl):
    """fp8 KV caches: accepted in the tiled layout only; never as activations."""
    T = _lib.HL_KV_TILED32
    a = _decode_args(kv_dtype=_lib.HL_FP8, max_len=2080)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EUNSUPPORTED
    assert "tiled" in _err(hl)
    a = _decode_args(kv_dtype=_lib.HL_FP8, max_len=2080, kv_layout=T)
    assert hl.hl_attn_decode_workspace_bytes(ctypes.byref(a)) > 0
    p = _prefill_args(k_cache=FAKE, v_cache=FAKE, kv_dtype=_lib.HL_FP8, max_len=4096)
    assert hl.hl_attn_prefill(ctypes.byref(p), None, 0, None) == _lib.HL_EUNSUPPORTED
    p = _prefill_args(io_dtype=_lib.HL_FP8)
    assert hl.hl_attn_prefill(ctypes.byref(p), None, 0, None) == _lib.HL_EINVAL


def test_paged_kv_validation(hl):
    """Paged caches: a block table is required and must cover max_len."""
    P = _lib.HL_KV_PAGED32
    a = _decode_args(kv_layout=P, max_len=2080)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "block table" in _err(hl)
    a = _decode_args(kv_layout=P, max_len=2080, block_table=FAKE, blocks_per_seq=64)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EINVAL
    assert "blocks_per_seq" in _err(hl)
    a = _decode_args(kv_layout=P, max_len=2080, block_table=FAKE, blocks_per_seq=65)
    assert hl.hl_attn_decode_workspace_bytes(ctypes.byref(a)) > 0
    a = _decode_args(kv_layout=P, max_len=2080, block_table=FAKE, blocks_per_seq=65,
                     kv_dtype=_lib.HL_F32)
    assert hl.hl_attn_decode(ctypes.byref(a), None, 0, None) == _lib.HL_EUNSUPPORTED
    p = _prefill_args(k_cache=FAKE, v_cache=FAKE, kv_dtype=_lib.HL_BF16, max_len=4096, kv_layout=P)
    assert hl.hl_attn_prefill(ctypes.byref(p), None, 0, None) == _lib.HL_EINVAL


def _model_desc(layers, **kw):
    m = _lib.ModelDesc(2, 256, 4, 2, 64, 64, 512, 300, 16, 1e-6, 1e4, FAKE, FAKE, FAKE, 0,
                       ctypes.cast(layers, ctypes.POINTER(_lib.LayerDesc)))
    for k, v in kw.items():
        setattr(m, k, v)
    return m


def _fake_layers(n=2, **kw):
    """Layer descriptors whose pointers are all non-null stand-ins (the host
    checks never dereference them)."""
    layers = (_lib.LayerDesc * n)()
    for L in layers:
        for f, t in _lib.LayerDesc._fields_:
            if t is ctypes.c_void_p and f not in ("q_norm", "k_norm"):
                setattr(L, f, FAKE)
        for k, v in kw.items():
            setattr(L, k, v)
    return layers


def test_decode_token_validation(hl):
    """hl_forward_decode_token's host checks (forwardDecodeToken's
    preconditions, naive.nim:4594-4599): nulls, shapes, every layer's
    weights and caches, the cache capacity, all before the first launch."""
    layers = _fake_layers()
    s = _lib.DecodeScratch(FAKE, FAKE, FAKE, FAKE, FAKE)
    tok = logits = nxt = FAKE
    call = lambda m, sc=s, pos=0: hl.hl_forward_decode_token(
        ctypes.byref(m) if m is not None else None, ctypes.byref(sc), tok, pos, logits, nxt, None)
    assert call(None) == _lib.HL_EINVAL
    assert call(_model_desc(layers, tok_emb=None)) == _lib.HL_EINVAL
    assert call(_model_desc(layers), _lib.DecodeScratch(FAKE, None, FAKE, FAKE, FAKE)) == _lib.HL_EINVAL
    assert call(_model_desc(layers, n_layer=0)) == _lib.HL_EINVAL
    assert call(_model_desc(layers, n_head_kv=0)) == _lib.HL_EINVAL
    assert call(_model_desc(layers, n_head_kv=3)) == _lib.HL_EINVAL
    assert _err(hl) == "GQA requires head_count divisible by head_count_kv"
    assert call(_model_desc(layers, rope_dim=70)) == _lib.HL_EINVAL  # > head_dim
    assert call(_model_desc(_fake_layers(w_down=None))) == _lib.HL_EINVAL
    assert "w_down" in _err(hl)
    assert call(_model_desc(_fake_layers(wq_type=9))) == _lib.HL_EUNSUPPORTED
    assert call(_model_desc(layers), pos=16) == _lib.HL_ECAPACITY
    assert "outside the cache" in _err(hl)
    assert call(_model_desc(layers), pos=-1) == _lib.HL_ECAPACITY
    # a layer's attention call that would fail (head_dim 96 is not built) is
    # refused before anything is launched
    assert call(_model_desc(layers, head_dim=96, rope_dim=0)) == _lib.HL_EUNSUPPORTED


def _kv_desc(n_layer=2, n_head_kv=2, head_dim=64, max_len=16, dt=_lib.HL_F32, lay=0, ptrs=None):
    p = (ctypes.c_void_p * n_layer)(*([FAKE] * n_layer if ptrs is None else ptrs))
    d = _lib.KvCacheDesc(n_layer, n_head_kv, head_dim, max_len, dt, lay, p, p, None, 0, 7)
    d._keep = p
    return d


def test_kv_cache_descriptor(hl):
    """hl_kv_cache_bytes / hl_kv_cache_init: initKvCache's per-layer tensor
    [kvDim, maxLen] (naive.nim:3926-3927) in each dtype and layout."""
    assert hl.hl_kv_cache_bytes(8, 128, 4096, _lib.HL_F32, 0) == 8 * 128 * 4096 * 4
    assert hl.hl_kv_cache_bytes(8, 128, 4096, _lib.HL_BF16, 1) == 8 * 128 * 4096 * 2
    assert hl.hl_kv_cache_bytes(8, 128, 4096, _lib.HL_FP8, 2) == 8 * 128 * 4096
    assert hl.hl_kv_cache_bytes(8, 128, 4096, _lib.HL_FP8, 0) == 0  # fp8 needs tiles
    assert hl.hl_kv_cache_bytes(8, 128, 4008, _lib.HL_F16, 1) == 0  # tiles of 32 columns
    assert hl.hl_kv_cache_bytes(8, 128, 4096, _lib.HL_F32, 1) == 0
    T, C = _lib.HL_KV_TILED32, _lib.HL_KV_COLMAJOR
    assert hl.hl_kv_cache_preferred_layout(_lib.HL_BF16, 32768) == T
    assert hl.hl_kv_cache_preferred_layout(_lib.HL_FP8, 4096) == T
    assert hl.hl_kv_cache_preferred_layout(_lib.HL_F16, 4100) == C
    assert hl.hl_kv_cache_preferred_layout(_lib.HL_F32, 4096) == C
    m = _model_desc(_fake_layers())
    c = _kv_desc()
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_OK
    assert c.cur_len == 0
    c = _kv_desc(n_layer=3)
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_EINVAL
    assert "does not match" in _err(hl)
    c = _kv_desc(ptrs=[FAKE, None])
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_EINVAL
    c = _kv_desc(dt=_lib.HL_FP8, lay=0)
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_EUNSUPPORTED
    c = _kv_desc(dt=_lib.HL_BF16, lay=1, max_len=64)  # tiled: 16-byte aligned stand-ins
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_OK


def test_forward_prefill_and_decode_validation(hl):
    """hl_forward_prefill / hl_forward_decode refuse with the reference's
    ValueError messages (naive.nim:3969-3976, 4598-4599) before launching."""
    m = _model_desc(_fake_layers())
    c = _kv_desc()
    assert hl.hl_kv_cache_init(ctypes.byref(c), ctypes.byref(m)) == _lib.HL_OK
    s = _lib.ForwardScratch(16, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30)
    pre = lambda mm, T: hl.hl_forward_prefill(ctypes.byref(mm), ctypes.byref(c), ctypes.byref(s), FAKE, T,
                                              FAKE, None)
    assert pre(m, 0) == _lib.HL_EINVAL
    assert _err(hl) == "prefill requires at least one token"
    assert pre(m, 17) == _lib.HL_ECAPACITY
    assert _err(hl) == "prefill exceeds KV cache capacity"
    assert pre(_model_desc(_fake_layers(), n_head_kv=3), 4) == _lib.HL_EINVAL
    assert _err(hl) == "GQA requires head_count divisible by head_count_kv"
    assert pre(_model_desc(_fake_layers(w_up_type=12)), 4) == _lib.HL_EUNSUPPORTED
    assert "fp32 weights" in _err(hl)
    small = _lib.ForwardScratch(3, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 30)
    assert hl.hl_forward_prefill(ctypes.byref(m), ctypes.byref(c), ctypes.byref(small), FAKE, 4, FAKE,
                                 None) == _lib.HL_EINVAL
    c.cur_len = 16
    dec = hl.hl_forward_decode(ctypes.byref(m), ctypes.byref(c), ctypes.byref(s), FAKE, FAKE, FAKE, None)
    assert dec == _lib.HL_ECAPACITY
    assert _err(hl) == "KV cache full"
    assert c.cur_len == 16  # a refused call changes nothing


def test_fused_and_elementwise_validation(hl):
    assert hl.hl_gpu_fused_gate_up_silu_quant(FAKE, FAKE, FAKE, FAKE, 512, 8, 9, None) == \
        _lib.HL_EUNSUPPORTED
    assert "unsupported quant type for GPU GEMV: 9" in _err(hl)
    assert hl.hl_gpu_fused_gate_up_silu_quant(FAKE, FAKE, FAKE, FAKE, 300, 8, 12, None) == \
        _lib.HL_EINVAL
    assert "multiple of 256" in _err(hl)
    assert hl.hl_gpu_fused_gate_up_silu_quant(None, FAKE, FAKE, FAKE, 512, 8, 12, None) == \
        _lib.HL_EINVAL
    assert hl.hl_gpu_fused_kv_linear_quant(FAKE, FAKE, FAKE, FAKE, FAKE, 512, 8, 12, 9, None) == \
        _lib.HL_EUNSUPPORTED
    assert hl.hl_gpu_fused_kv_linear_q2k_q3k(FAKE, None, FAKE, FAKE, FAKE, 512, 8, None) == \
        _lib.HL_EINVAL
    assert hl.hl_gpu_silu_mul(FAKE, FAKE, FAKE, 0, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_silu_mul(FAKE, None, FAKE, 16, None) == _lib.HL_EINVAL
    assert hl.hl_gpu_add(FAKE, FAKE, FAKE, -1, None) == _lib.HL_EINVAL


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and one
    JSON line that says so, before touching a device."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=root)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]
