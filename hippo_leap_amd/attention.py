"""Host-side mirror of the reference's attention-stage procs over torch tensors.

Each function keeps the name (snake_case), argument order and meaning of the
Nim proc it replaces in backends/naive.nim and calls the matching C-ABI entry
point of libhl_attn.so on torch's current HIP stream.  Torch supplies device
memory and the stream only; all arithmetic runs in the HIP kernels.

Reference procs mirrored:
  gpu_qk_norm              gpuQkNorm              naive.nim:2918-2926
  gpu_qk_norm_prefill      gpuQkNormPrefill       naive.nim:2962-2971
  gpu_rope_at_pos          gpuRopeAtPos           naive.nim:3088-3101
  gpu_rope_at_pos_theta    gpuRopeAtPosTheta      naive.nim:3133-3144
  gpu_rope_qk_decode       gpuRopeQKDecode        naive.nim:3075-3086
  gpu_fused_rope_store_kv  gpuFusedRopeStoreKV    naive.nim:3203-3223
  gpu_store_kv             gpuStoreKV             naive.nim:3241-3253
  gpu_store_kv_pair        gpuStoreKVPair         naive.nim:3273-3285
  gpu_attention_decode     gpuAttentionDecode     naive.nim:3369-3383
  gpu_attention_prefill    gpuAttentionPrefill    naive.nim:3450-3464
Errors raise HLError (a ValueError), as the reference raises ValueError.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import (HL_BF16, HL_F16, HL_F32, HL_FP8, HL_KV_COLMAJOR, HL_KV_PAGED32,  # noqa: F401
                   HL_KV_TILED32, HL_ROPE_HALF_SPLIT, DecodeArgs, PrefillArgs, RopeStoreArgs,
                   HL_OK, check)

_DT = {torch.float32: HL_F32, torch.float16: HL_F16, torch.bfloat16: HL_BF16,
       torch.float8_e4m3fn: HL_FP8, torch.uint8: HL_FP8}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise _lib.HLError(_lib.HL_EINVAL, f"unsupported dtype {t.dtype}") from None


def _p(t):
    """Device pointer of a tensor (or None)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise _lib.HLError(_lib.HL_EINVAL, "tensor must live on the GPU")
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


# ---------------------------------------------------------------------------
# Reference-signature wrappers (fp32, one sequence)
# ---------------------------------------------------------------------------
def gpu_qk_norm(x, weight, n_head, head_dim, eps, stream=None):
    check(_lib.load().hl_gpu_qk_norm(_p(x), _p(weight), n_head, head_dim, eps, _stream(stream)))


def gpu_qk_norm_prefill(x, weight, n_head, head_dim, seq_len, eps, stream=None):
    check(_lib.load().hl_gpu_qk_norm_prefill(_p(x), _p(weight), n_head, head_dim, seq_len, eps,
                                             _stream(stream)))


def gpu_rope_at_pos(x, n_head, head_dim, rope_dim, rope_base, pos, seq_len, stream=None):
    check(_lib.load().hl_gpu_rope_at_pos(_p(x), n_head, head_dim, rope_dim, rope_base, pos,
                                         seq_len, _stream(stream)))


def gpu_rope_at_pos_theta(x, n_head, head_dim, rope_dim, pos, seq_len, stream=None):
    check(_lib.load().hl_gpu_rope_at_pos_theta(_p(x), n_head, head_dim, rope_dim, pos, seq_len,
                                               _stream(stream)))


def gpu_rope_qk_decode(q, k, n_head_q, n_head_k, head_dim, rope_dim, rope_base, pos, stream=None):
    check(_lib.load().hl_gpu_rope_qk_decode(_p(q), _p(k), n_head_q, n_head_k, head_dim, rope_dim,
                                            rope_base, pos, _stream(stream)))


def gpu_fused_rope_store_kv(q, k, v, k_cache, v_cache, n_head_q, n_head_k, head_dim, rope_dim,
                            kv_dim, cache_cols, pos, stream=None):
    check(_lib.load().hl_gpu_fused_rope_store_kv(
        _p(q), _p(k), _p(v), _p(k_cache), _p(v_cache), n_head_q, n_head_k, head_dim, rope_dim,
        kv_dim, cache_cols, pos, _stream(stream)))


def gpu_store_kv(cache, src, rows, src_cols, cache_cols, start_pos, stream=None):
    check(_lib.load().hl_gpu_store_kv(_p(cache), _p(src), rows, src_cols, cache_cols, start_pos,
                                      _stream(stream)))


def gpu_store_kv_pair(k_cache, k_src, v_cache, v_src, rows, src_cols, cache_cols, start_pos,
                      stream=None):
    check(_lib.load().hl_gpu_store_kv_pair(_p(k_cache), _p(k_src), _p(v_cache), _p(v_src), rows,
                                           src_cols, cache_cols, start_pos, _stream(stream)))


def gpu_attention_decode(dst, q, k_cache, v_cache, n_head, n_head_kv, head_dim, cur_len,
                         cache_cols, stream=None):
    check(_lib.load().hl_gpu_attention_decode(_p(dst), _p(q), _p(k_cache), _p(v_cache), n_head,
                                              n_head_kv, head_dim, cur_len, cache_cols,
                                              _stream(stream)))


def gpu_attention_prefill(dst, q, k, v, n_head, n_head_kv, head_dim, seq_len, stream=None):
    check(_lib.load().hl_gpu_attention_prefill(_p(dst), _p(q), _p(k), _p(v), n_head, n_head_kv,
                                               head_dim, seq_len, _stream(stream)))


def gpu_linear_col(dst, x, w, w_cols, w_rows, seq_len, stream=None):
    """gpuLinearCol (naive.nim:3519-3547): dst[w_rows, seq_len] = w . x, fp32."""
    check(_lib.load().hl_gpu_linear_col(_p(dst), _p(x), _p(w), w_cols, w_rows, seq_len,
                                        _stream(stream)))


def gpu_linear_col_quant(dst, x, w_quant, w_cols, w_rows, quant_type, stream=None):
    """gpuLinearColQuant (naive.nim:1580-1592): dst[w_rows] = dequant(w) . x, one token."""
    check(_lib.load().hl_gpu_linear_col_quant(_p(dst), _p(x), _p(w_quant), w_cols, w_rows,
                                              quant_type, _stream(stream)))


def gpu_silu_mul(dst, gate, up, n, stream=None):
    """gpuSiluMul (naive.nim:2179-2193): dst = silu(gate) * up, fp32."""
    check(_lib.load().hl_gpu_silu_mul(_p(dst), _p(gate), _p(up), n, _stream(stream)))


def gpu_fused_gate_up_silu_quant(dst, x, gate_q, up_q, w_cols, w_rows, quant_type, stream=None):
    """gpuFusedGateUpSiluQ4K/Q3K (naive.nim:1905-1920, 1693-1708), any GGUF type."""
    check(_lib.load().hl_gpu_fused_gate_up_silu_quant(_p(dst), _p(x), _p(gate_q), _p(up_q), w_cols,
                                                      w_rows, quant_type, _stream(stream)))


def gpu_fused_kv_linear_quant(k_dst, v_dst, x, k_q, v_q, w_cols, w_rows, k_type, v_type,
                              stream=None):
    """gpuFusedKVLinearQ4K/Q2KQ3K (naive.nim:1799-1814, 853-868), any GGUF types."""
    check(_lib.load().hl_gpu_fused_kv_linear_quant(_p(k_dst), _p(v_dst), _p(x), _p(k_q), _p(v_q),
                                                   w_cols, w_rows, k_type, v_type, _stream(stream)))


def gpu_add(dst, a, b, n, stream=None):
    """gpuAdd (naive.nim:2132-2145): dst = a + b, fp32."""
    check(_lib.load().hl_gpu_add(_p(dst), _p(a), _p(b), n, _stream(stream)))


def gpu_rmsnorm_cols(dst, x, weight, dim, seq_len, eps, stream=None):
    """gpuRmsnormCols (naive.nim:2834-2843) on col-major [dim, seq_len] fp32."""
    check(_lib.load().hl_gpu_rmsnorm_cols(_p(dst), _p(x), _p(weight), dim, seq_len, eps,
                                          _stream(stream)))


def gpu_residual_rmsnorm(norm_out, x, residual, weight, dim, eps, stream=None):
    """gpuResidualRmsnorm (naive.nim:2874-2882): x += residual; norm_out = rmsnorm(x) * w."""
    check(_lib.load().hl_gpu_residual_rmsnorm(_p(norm_out), _p(x), _p(residual), _p(weight), dim,
                                              eps, _stream(stream)))


def gpu_argmax(logits, n_vocab, stream=None) -> int:
    """gpuArgmax (naive.nim:2105-2127): greedy token index (waits for the stream)."""
    out = ctypes.c_int32(0)
    check(_lib.load().hl_gpu_argmax(_p(logits), n_vocab, ctypes.byref(out), _stream(stream)))
    return out.value


def argmax_async(logits, n_vocab, result, stream=None) -> None:
    """Greedy token index into result (an int32 device tensor), no host wait."""
    check(_lib.load().hl_argmax_async(_p(logits), n_vocab, _p(result), _stream(stream)))


def gpu_embedding(dst, weight, token_ids, n_emb, n_tokens, n_vocab, stream=None):
    """gpuEmbedding (naive.nim:2975-3001): dst[nEmb, nTokens] = weight rows of the tokens."""
    check(_lib.load().hl_gpu_embedding(_p(dst), _p(weight), _p(token_ids), n_emb, n_tokens,
                                       n_vocab, _stream(stream)))


def set_rope_theta(rope_dim: int, rope_base: float) -> None:
    """Installs the theta table (naive.nim:3850-3861) used by the *_theta procs."""
    check(_lib.load().hl_set_rope_theta(rope_dim, rope_base))


def rope_theta_table(rope_dim: int, rope_base: float) -> list[float]:
    buf = (ctypes.c_float * (rope_dim // 2))()
    check(_lib.load().hl_rope_theta_table(buf, rope_dim, rope_base))
    return list(buf)


def kv_cache_to_f32(cache, rows, max_len, col0, ncols, stream=None) -> torch.Tensor:
    out = torch.empty(rows, ncols, dtype=torch.float32, device=cache.device)
    check(_lib.load().hl_kv_cache_to_f32(_p(out), _p(cache), dtype_code(cache), rows, max_len, col0,
                                         ncols, _stream(stream)))
    return out


def device_info() -> dict:
    info = _lib.DeviceInfo()
    check(_lib.load().hl_device_info_get(ctypes.byref(info)))
    return {name: (getattr(info, name).decode() if name == "arch" else getattr(info, name))
            for name, _ in _lib.DeviceInfo._fields_}


# ---------------------------------------------------------------------------
# Batched / typed API
# ---------------------------------------------------------------------------
def decode_args(q, k_cache, v_cache, out, n_head, n_head_kv, head_dim, max_len, seq_len,
                seq_lens=None, cache_batch_stride=0, scale=0.0, num_splits=0,
                kv_layout=HL_KV_COLMAJOR, block_table=None) -> DecodeArgs:
    """Arguments of hl_attn_decode.  block_table (paged layout): int32
    device tensor [B, blocks_per_seq] of page indices."""
    a = DecodeArgs()
    a.batch = q.numel() // (n_head * head_dim)
    a.n_head, a.n_head_kv, a.head_dim = n_head, n_head_kv, head_dim
    a.kv_dtype = dtype_code(k_cache)
    a.max_len, a.seq_len = max_len, seq_len
    a.seq_lens = seq_lens.data_ptr() if seq_lens is not None else None
    a.cache_batch_stride = cache_batch_stride
    a.q, a.k_cache, a.v_cache, a.out = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr()
    a.scale, a.num_splits = scale, num_splits
    a.kv_layout = kv_layout
    _set_table(a, block_table)
    a._tensors = (q, k_cache, v_cache, out, seq_lens, block_table)  # the struct holds raw pointers
    return a


def _set_table(a, block_table, per_seq=True):
    if block_table is None:
        return
    a.block_table = block_table.data_ptr()
    if per_seq:
        a.blocks_per_seq = block_table.shape[-1]


def kv_to_paged(cache, n_head_kv, head_dim, max_len, block_table, n_pages):
    """Column-major caches [B][Hkv*D, max_len] -> an HL_KV_PAGED32 pool of
    n_pages pages [Hkv][D][32]: tile j of sequence b goes to page
    block_table[b, j] (pages no entry names stay zero)."""
    B = cache.numel() // (n_head_kv * head_dim * max_len)
    nt = max_len // 32
    t = cache.reshape(B, n_head_kv, head_dim, nt, 32).permute(0, 3, 1, 2, 4)  # [B, nt, Hkv, D, 32]
    pool = torch.zeros(n_pages, n_head_kv, head_dim, 32, dtype=cache.dtype, device=cache.device)
    pool[block_table[:, :nt].reshape(-1).long()] = t.reshape(B * nt, n_head_kv, head_dim, 32)
    return pool.reshape(-1)


def kv_from_paged(pool, n_head_kv, head_dim, max_len, block_table):
    """Inverse of kv_to_paged: the column-major caches [B][Hkv*D, max_len]."""
    B, nt = block_table.shape[0], max_len // 32
    pages = pool.reshape(-1, n_head_kv, head_dim, 32)[block_table[:, :nt].reshape(-1).long()]
    return pages.reshape(B, nt, n_head_kv, head_dim, 32).permute(0, 2, 3, 1, 4).reshape(-1)


def kv_to_tiled(cache, n_head_kv, head_dim, max_len):
    """Column-major cache [..., Hkv*D, max_len] -> the HL_KV_TILED32 layout
    (per kv head, max_len/32 tiles of [D][32]); same numel, new tensor."""
    lead = cache.numel() // (n_head_kv * head_dim * max_len)
    t = cache.reshape(lead, n_head_kv, head_dim, max_len // 32, 32)
    return t.permute(0, 1, 3, 2, 4).contiguous().reshape(cache.shape)


def kv_from_tiled(cache, n_head_kv, head_dim, max_len):
    """Inverse of kv_to_tiled."""
    lead = cache.numel() // (n_head_kv * head_dim * max_len)
    t = cache.reshape(lead, n_head_kv, max_len // 32, head_dim, 32)
    return t.permute(0, 1, 3, 2, 4).contiguous().reshape(cache.shape)


def decode_workspace_bytes(args: DecodeArgs) -> int:
    return int(_lib.load().hl_attn_decode_workspace_bytes(ctypes.byref(args)))


def decode_workspace(args: DecodeArgs, device="cuda", stream=None):
    """Allocates and zero-initialises a decode workspace (None if not needed)."""
    nbytes = decode_workspace_bytes(args)
    if nbytes <= 0:
        return None
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    check(_lib.load().hl_attn_decode_workspace_init(ws.data_ptr(), nbytes, _stream(stream)))
    return ws


def attn_decode(args: DecodeArgs, workspace=None, stream=None) -> None:
    """Batched split-K decode (hl_attn_decode); workspace is a uint8 device tensor."""
    ws = workspace.data_ptr() if workspace is not None else None
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(_lib.load().hl_attn_decode(ctypes.byref(args), ws, nbytes, _stream(stream)))


def rope_store_args(q, k, v, k_cache, v_cache, n_head_q, n_head_kv, head_dim, max_len, pos,
                    rope_base, rope_dim=0, rope_style=HL_ROPE_HALF_SPLIT, positions=None,
                    q_norm_w=None, k_norm_w=None, eps=1e-6, cache_batch_stride=0,
                    use_installed_theta=False, kv_layout=HL_KV_COLMAJOR,
                    block_table=None) -> RopeStoreArgs:
    a = RopeStoreArgs()
    a.batch = q.numel() // (n_head_q * head_dim)
    a.n_head_q, a.n_head_kv, a.head_dim = n_head_q, n_head_kv, head_dim
    a.rope_dim, a.rope_style, a.rope_base = rope_dim, rope_style, rope_base
    a.use_installed_theta = int(use_installed_theta)
    a.kv_dtype, a.max_len, a.cache_batch_stride = dtype_code(k_cache), max_len, cache_batch_stride
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.k_cache, a.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    a.positions = positions.data_ptr() if positions is not None else None
    a.pos = pos
    a.q_norm_w = q_norm_w.data_ptr() if q_norm_w is not None else None
    a.k_norm_w = k_norm_w.data_ptr() if k_norm_w is not None else None
    a.eps = eps
    a.kv_layout = kv_layout
    _set_table(a, block_table)
    a._tensors = (q, k, v, k_cache, v_cache, positions, q_norm_w, k_norm_w, block_table)
    return a


def rope_store_decode(*args, stream=None, **kw) -> None:
    """hl_rope_store_decode; arguments as rope_store_args."""
    a = rope_store_args(*args, **kw)
    check(_lib.load().hl_rope_store_decode(ctypes.byref(a), _stream(stream)))


def decode_step_workspace(rs: RopeStoreArgs, at: DecodeArgs, device="cuda", stream=None):
    """Allocates and zero-initialises the workspace of hl_decode_step (None if not needed)."""
    lib = _lib.load()
    nbytes = int(lib.hl_decode_step_workspace_bytes(ctypes.byref(rs), ctypes.byref(at)))
    if nbytes <= 0:
        return None
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    check(lib.hl_attn_decode_workspace_init(ws.data_ptr(), nbytes, _stream(stream)))
    return ws


def decode_step(rs: RopeStoreArgs, at: DecodeArgs, workspace=None, stream=None) -> None:
    """hl_decode_step: qkNorm + RoPE + KV store + attention for the new token."""
    ws = workspace.data_ptr() if workspace is not None else None
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(_lib.load().hl_decode_step(ctypes.byref(rs), ctypes.byref(at), ws, nbytes,
                                     _stream(stream)))


def prefill_args(q, k, v, out, n_head, n_head_kv, head_dim, seq_len, rope_base=0.0,
                 apply_rope=False, rope_dim=0, rope_style=HL_ROPE_HALF_SPLIT, q_norm_w=None,
                 k_norm_w=None, eps=1e-6, k_cache=None, v_cache=None, max_len=0, start_pos=0,
                 scale=0.0, write_back_qk=False, use_installed_theta=False,
                 kv_layout=HL_KV_COLMAJOR, block_table=None) -> PrefillArgs:
    """Arguments of hl_attn_prefill; the output dtype is taken from `out`.
    block_table (paged layout): int32 device tensor of this sequence's pages."""
    a = PrefillArgs()
    a.n_head, a.n_head_kv, a.head_dim, a.seq_len = n_head, n_head_kv, head_dim, seq_len
    a.io_dtype = dtype_code(q)
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.q_norm_w = q_norm_w.data_ptr() if q_norm_w is not None else None
    a.k_norm_w = k_norm_w.data_ptr() if k_norm_w is not None else None
    a.eps = eps
    a.apply_rope, a.rope_dim, a.rope_style, a.rope_base = int(apply_rope), rope_dim, rope_style, rope_base
    a.use_installed_theta = int(use_installed_theta)
    a.k_cache = k_cache.data_ptr() if k_cache is not None else None
    a.v_cache = v_cache.data_ptr() if v_cache is not None else None
    a.kv_dtype = dtype_code(k_cache) if k_cache is not None else HL_F32
    a.max_len, a.start_pos, a.scale = max_len, start_pos, scale
    a.write_back_qk = int(write_back_qk)
    a.out_dtype = dtype_code(out)
    a.kv_layout = kv_layout
    _set_table(a, block_table, per_seq=False)
    a._tensors = (q, k, v, out, q_norm_w, k_norm_w, k_cache, v_cache, block_table)
    return a


def prefill_workspace_bytes(args: PrefillArgs) -> int:
    return int(_lib.load().hl_attn_prefill_workspace_bytes(ctypes.byref(args)))


def attn_prefill(args: PrefillArgs, workspace=None, stream=None) -> None:
    ws = workspace.data_ptr() if workspace is not None else None
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(_lib.load().hl_attn_prefill(ctypes.byref(args), ws, nbytes, _stream(stream)))


def prefill_fallback_ran(args: PrefillArgs, workspace=None, stream=None) -> bool:
    """Waits for the stream; True when the last hl_attn_prefill on
    `workspace` with these args recomputed its output on the fp32 fallback
    (an fp16 operand would have overflowed)."""
    ws = workspace.data_ptr() if workspace is not None else None
    ran = ctypes.c_int(0)
    check(_lib.load().hl_attn_prefill_fallback_ran(ctypes.byref(args), ws, ctypes.byref(ran),
                                                   _stream(stream)))
    return bool(ran.value)


def probe_stream_read(buf: torch.Tensor, sink: torch.Tensor, blocks: int = 0, stream=None,
                      inflight: int = 4, contiguous: bool = False) -> None:
    """One launch that only streams `buf` (measurement probe)."""
    nbytes = buf.numel() * buf.element_size()
    check(_lib.load().hl_probe_stream_read_ex(buf.data_ptr(), nbytes, blocks, inflight, int(contiguous),
                                              sink.data_ptr(), _stream(stream)))


def workspace(nbytes: int, device="cuda") -> torch.Tensor | None:
    """Allocates a zero-filled caller-owned workspace (GpuContext.attnScratch's role)."""
    if nbytes <= 0:
        return None
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)
