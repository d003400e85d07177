"""Greedy decode of a dense decoder through hl_forward_decode_token: the
reference's forwardDecodeToken for layers of kind lkAttentionFfn
(backends/naive.nim:4592-4760, 5520-5545).

DenseDecoder holds the ctypes descriptors of one model's device tensors and
the decode scratch; step() runs one token on the device and leaves the next
token on the device, so steps chain without host round trips.
"""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import check
from .attention import _p, _stream

c_void_p = ctypes.c_void_p

LAYER_WEIGHTS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


class DenseDecoder:
    """cfg: n_layer, n_emb, n_head, n_head_kv, head_dim, rope_dim, n_ff,
    n_vocab, max_len, rms_eps, rope_base.  layers: one dict per layer with
    attn_norm, ffn_norm, optional q_norm / k_norm (fp32 device tensors), the
    seven weights (fp32 [rows, cols] tensors, or uint8 GGUF rows) and their
    types under "<name>_type" (0 = fp32), and k_cache / v_cache fp32
    [n_head_kv*head_dim, max_len].  tok_emb fp32 [n_vocab, n_emb];
    output_norm [n_emb]; output weight and output_type as the layers'."""

    def __init__(self, torch, cfg: dict, tok_emb, output_norm, output, output_type: int,
                 layers: list[dict]):
        self.torch = torch
        self.cfg = dict(cfg)
        self.keep = [tok_emb, output_norm, output, layers]
        arr = (_lib.LayerDesc * len(layers))()
        for i, L in enumerate(layers):
            d = arr[i]
            for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm", "k_cache", "v_cache"):
                setattr(d, n, _p(L.get(n)))
            for n in LAYER_WEIGHTS:
                setattr(d, n, _p(L[n]))
                setattr(d, n + "_type", int(L.get(n + "_type", 0)))
        self.layer_arr = arr
        c = self.cfg
        self.desc = _lib.ModelDesc(
            c["n_layer"], c["n_emb"], c["n_head"], c["n_head_kv"], c["head_dim"], c["rope_dim"],
            c["n_ff"], c["n_vocab"], c["max_len"], c["rms_eps"], c["rope_base"], _p(tok_emb),
            _p(output_norm), _p(output), int(output_type),
            ctypes.cast(arr, ctypes.POINTER(_lib.LayerDesc)))
        E, q, kv, ff = c["n_emb"], c["n_head"] * c["head_dim"], c["n_head_kv"] * c["head_dim"], c["n_ff"]
        f = lambda n: torch.zeros(n, device="cuda")
        self.bufs = [f(E), f(max(E, q)), f(max(E, q, ff)), f(max(kv, ff)), f(max(kv, ff))]
        self.scratch = _lib.DecodeScratch(*[_p(b) for b in self.bufs])
        self.logits = f(c["n_vocab"])
        self.tokens = torch.zeros(2, dtype=torch.int32, device="cuda")  # current, next

    def step(self, pos: int, token_dev=None, next_dev=None, stream=None):
        """One token at position pos: reads token_dev (default: this
        decoder's current-token slot), writes logits and next_dev (default:
        the next-token slot)."""
        tok = self.tokens[0:1] if token_dev is None else token_dev
        nxt = self.tokens[1:2] if next_dev is None else next_dev
        check(_lib.load().hl_forward_decode_token(ctypes.byref(self.desc), ctypes.byref(self.scratch),
                                                  _p(tok), pos, _p(self.logits), _p(nxt),
                                                  _stream(stream)))

    def generate(self, first_token: int, n_steps: int, stream=None) -> list[int]:
        """Greedy tokens after first_token for positions 0 .. n_steps-1,
        chained on the device (one host read at the end)."""
        out = self.torch.zeros(n_steps + 1, dtype=self.torch.int32, device="cuda")
        out[0] = first_token
        for p in range(n_steps):
            self.step(p, out[p:p + 1], out[p + 1:p + 2], stream)
        return out.cpu().tolist()[1:]


class KvCache:
    """initKvCache (backends/naive.nim:3912-3931) with a storage dtype and
    layout: one K and one V device buffer of hl_kv_cache_bytes() per layer,
    described by an hl_kv_cache_desc checked against the model."""

    def __init__(self, torch, model: "DenseDecoder", kv_dtype: int = _lib.HL_F32,
                 kv_layout: int | None = None, max_len: int | None = None, block_table=None):
        """kv_layout None: the library's preferred layout for the dtype (tiled
        for fp16/bf16/fp8 when max_len % 32 == 0, else column-major)."""
        c = model.cfg
        self.max_len = int(max_len or c["max_len"])
        lib = _lib.load()
        if kv_layout is None:
            kv_layout = int(lib.hl_kv_cache_preferred_layout(kv_dtype, self.max_len))
        nbytes = int(lib.hl_kv_cache_bytes(c["n_head_kv"], c["head_dim"], self.max_len, kv_dtype, kv_layout))
        if nbytes == 0:
            raise _lib.HLError(_lib.HL_EUNSUPPORTED, f"kv cache dtype {kv_dtype} / layout {kv_layout} not built")
        n = c["n_layer"]
        self.k = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(n)]
        self.v = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(n)]
        self.table = block_table
        self._kp = (c_void_p * n)(*[t.data_ptr() for t in self.k])
        self._vp = (c_void_p * n)(*[t.data_ptr() for t in self.v])
        self.desc = _lib.KvCacheDesc(n, c["n_head_kv"], c["head_dim"], self.max_len, kv_dtype, kv_layout,
                                     self._kp, self._vp, _p(block_table),
                                     0 if block_table is None else int(block_table.numel()), 0)
        check(lib.hl_kv_cache_init(ctypes.byref(self.desc), ctypes.byref(model.desc)))

    @property
    def cur_len(self) -> int:
        return int(self.desc.cur_len)


class DenseModel(DenseDecoder):
    """The backend contract over a KV-cache descriptor: prefill() is the
    reference's forwardPrefill and decode() its forwardDecodeToken
    (backends/naive.nim:3967-4590, 4592-4760) for lkAttentionFfn layers,
    through hl_forward_prefill / hl_forward_decode.  The activation scratch
    and attention workspace are allocated here once for max_tokens columns,
    so no call allocates."""

    def __init__(self, torch, cfg: dict, tok_emb, output_norm, output, output_type: int,
                 layers: list[dict], cache: KvCache | None = None, max_tokens: int = 1,
                 kv_dtype: int = _lib.HL_F32, kv_layout: int | None = None):
        super().__init__(torch, cfg, tok_emb, output_norm, output, output_type, layers)
        self.cache = cache if cache is not None else KvCache(torch, self, kv_dtype, kv_layout)
        c, T = self.cfg, max(1, int(max_tokens))
        E, q, kv, ff = c["n_emb"], c["n_head"] * c["head_dim"], c["n_head_kv"] * c["head_dim"], c["n_ff"]
        f = lambda n: torch.zeros(n * T, device="cuda")
        self.fbufs = [f(E), f(max(E, q)), f(max(E, q, ff)), f(max(kv, ff)), f(max(kv, ff))]
        lib = _lib.load()
        nws = int(lib.hl_forward_workspace_bytes(ctypes.byref(self.desc), ctypes.byref(self.cache.desc), T))
        self.ws = torch.zeros(max(nws, 256), dtype=torch.uint8, device="cuda")
        check(lib.hl_attn_decode_workspace_init(self.ws.data_ptr(), nws, None))
        self.fscratch = _lib.ForwardScratch(T, *[_p(b) for b in self.fbufs], self.ws.data_ptr(), nws)
        self.max_tokens = T

    def prefill(self, tokens, stream=None):
        """forwardPrefill: tokens (host list or device int32 tensor) at
        positions 0 .. T-1; returns the logits [n_vocab, T] (device)."""
        torch = self.torch
        tok = tokens if torch.is_tensor(tokens) else torch.tensor(list(tokens), dtype=torch.int32, device="cuda")
        T = int(tok.numel())
        logits = torch.empty(self.cfg["n_vocab"], max(T, 1), device="cuda")
        check(_lib.load().hl_forward_prefill(ctypes.byref(self.desc), ctypes.byref(self.cache.desc),
                                             ctypes.byref(self.fscratch), _p(tok), T, _p(logits),
                                             _stream(stream)))
        return logits

    def decode(self, token_dev=None, next_dev=None, stream=None):
        """forwardDecodeToken at position cache.cur_len: reads token_dev
        (default: the current-token slot), writes self.logits and next_dev
        (default: the next-token slot), advances the cache."""
        tok = self.tokens[0:1] if token_dev is None else token_dev
        nxt = self.tokens[1:2] if next_dev is None else next_dev
        check(_lib.load().hl_forward_decode(ctypes.byref(self.desc), ctypes.byref(self.cache.desc),
                                            ctypes.byref(self.fscratch), _p(tok), _p(self.logits), _p(nxt),
                                            _stream(stream)))

    def decode_timed(self, token_dev=None, stream=None) -> tuple[int, float]:
        """forwardDecodeTokenTimed: decode() bracketed by GPU events; waits
        for the stream and returns (next token, GPU ms)."""
        tok = self.tokens[0:1] if token_dev is None else token_dev
        nxt = ctypes.c_int32(0)
        ms = ctypes.c_float(0.0)
        check(_lib.load().hl_forward_decode_timed(ctypes.byref(self.desc), ctypes.byref(self.cache.desc),
                                                  ctypes.byref(self.fscratch), _p(tok), _p(self.logits),
                                                  _p(self.tokens[1:2]), ctypes.byref(nxt), ctypes.byref(ms),
                                                  _stream(stream)))
        return int(nxt.value), float(ms.value)
