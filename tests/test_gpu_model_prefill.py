"""End-to-end forwardPrefill followed by forwardDecodeToken on the same KV
cache (backends/naive.nim:3967-4590, 4592-4760; lkAttentionFfn layers),
through hl_forward_prefill / hl_forward_decode over an hl_kv_cache_desc,
against an oracle composed from the pinned oracle pieces in the
reference's order: embedding; per layer rmsnorm, Q/K/V (tensor.nim
matmul), qk-norm, RoPE at positions 0 .. T-1, K/V into the cache, causal
attention, O projection + residual (add), rmsnorm, SiLU(gate) * up, down +
residual; final norm, output projection -> logits [n_vocab, T].  Then
decode steps continue at position T on the cache the prefill left.

The cache may hold fp32 (the reference's), bf16 or fp8 values in the
column-major or tiled layout; the oracle stores the same rounded values
(round to nearest even), so the GPU and the oracle read identical caches.
Bars: 1e-4 for fp32 caches, 2e-3 for bf16/fp8 caches (north star), on the
logits of every column and every decode step; the greedy token of each
step equals the reference argmax of the GPU's logits."""
import numpy as np
import pytest
import torch

from test_gpu_model import _build
from util import TOL_F32, TOL_LOWP, rel_err

pytestmark = pytest.mark.gpu

CFG = dict(n_layer=2, n_emb=256, n_head=4, n_head_kv=2, head_dim=64, rope_dim=0, n_ff=512,
           n_vocab=300, max_len=32, rms_eps=1e-6, rope_base=1e4)


def _stored(orc, x, dt):
    """The values a cache of dtype dt holds for fp32 x (RNE), as fp32."""
    return x if dt == orc.F32 else orc.upcast(orc.to_storage(x, dt), dt).reshape(x.shape)


def _oracle_prefill(orc, cfg, ref, tokens, dt):
    E, D, eps, T = cfg["n_emb"], cfg["head_dim"], cfg["rms_eps"], len(tokens)
    H, Hkv = cfg["n_head"], cfg["n_head_kv"]
    rd = cfg["rope_dim"] or D
    theta = orc.theta_table(rd, cfg["rope_base"])
    x = orc.embedding(ref["tok_emb"], tokens, E)
    for lw in ref["layers"]:
        xn = orc.rmsnorm_cols(x, lw["attn_norm"], eps)
        q, k, v = orc.matmul(lw["wq"], xn), orc.matmul(lw["wk"], xn), orc.matmul(lw["wv"], xn)
        if "q_norm" in lw:
            q = orc.qk_norm_cols(q, lw["q_norm"], H, D, T, eps)
            k = orc.qk_norm_cols(k, lw["k_norm"], Hkv, D, T, eps)
        q = orc.rope_cols(q, H, D, T, rd, theta, 0)
        k = orc.rope_cols(k, Hkv, D, T, rd, theta, 0)
        lw["k_cache"][:, :T] = _stored(orc, k, dt)  # gpuStoreKV at columns 0 .. T-1
        lw["v_cache"][:, :T] = _stored(orc, v, dt)
        a = orc.attention_prefill(q, k, v, H, Hkv, D, T)
        x = orc.add(x, orc.matmul(lw["wo"], a))
        xn = orc.rmsnorm_cols(x, lw["ffn_norm"], eps)
        h = orc.silu_mul(orc.matmul(lw["w_gate"], xn), orc.matmul(lw["w_up"], xn))
        x = orc.add(x, orc.matmul(lw["w_down"], h))
    return orc.matmul(ref["output"], orc.rmsnorm_cols(x, ref["output_norm"], eps))


def _oracle_decode(orc, cfg, ref, tok, pos, dt):
    E, D, eps = cfg["n_emb"], cfg["head_dim"], cfg["rms_eps"]
    H, Hkv, L = cfg["n_head"], cfg["n_head_kv"], cfg["max_len"]
    rd = cfg["rope_dim"] or D
    theta = orc.theta_table(rd, cfg["rope_base"])
    mv = lambda w, v: orc.matmul(w, v.reshape(-1, 1)).reshape(-1)
    norm = lambda v, w: orc.rmsnorm_cols(v.reshape(-1, 1), w, eps).reshape(-1)
    x = orc.embedding(ref["tok_emb"], [tok], E).reshape(-1)
    for lw in ref["layers"]:
        xn = norm(x, lw["attn_norm"])
        q, k, v = mv(lw["wq"], xn), mv(lw["wk"], xn), mv(lw["wv"], xn)
        if "q_norm" in lw:
            q = orc.qk_norm(q, lw["q_norm"], H, D, eps)
            k = orc.qk_norm(k, lw["k_norm"], Hkv, D, eps)
        q = orc.rope_heads(q, H, D, rd, theta, pos)
        k = orc.rope_heads(k, Hkv, D, rd, theta, pos)
        lw["k_cache"][:, pos] = _stored(orc, k, dt)
        lw["v_cache"][:, pos] = _stored(orc, v, dt)
        a = orc.attention_decode(q, lw["k_cache"], lw["v_cache"], H, Hkv, D, pos + 1, L)
        x = orc.add(x, mv(lw["wo"], a))
        xn = norm(x, lw["ffn_norm"])
        h = orc.silu_mul(mv(lw["w_gate"], xn), mv(lw["w_up"], xn))
        x = orc.add(x, mv(lw["w_down"], h))
    return mv(ref["output"], norm(x, ref["output_norm"]))


CASES = [  # (name, kv dtype, layout, qk-norm)
    ("fp32_colmajor", 0, 0, False),
    ("fp32_colmajor_qknorm", 0, 0, True),
    ("bf16_colmajor", 2, 0, False),
    ("f16_tiled_qknorm", 1, 1, True),
    ("fp8_tiled", 3, 1, False),
]


# head dim 128 (the Llama-3-8B / Qwen3 head) with fp32 activations and caches:
# the split-operand prefill kernel at 128 (q dim 512 != n_emb 256)
CFG128 = dict(CFG, head_dim=128)
CASES128 = [("fp32_colmajor_d128", 0, 0, False), ("fp32_colmajor_qknorm_d128", 0, 0, True)]


@pytest.mark.parametrize("name,dt,lay,qk", CASES + CASES128, ids=[c[0] for c in CASES + CASES128])
def test_prefill_then_decode_matches_oracle(hl, orc, name, dt, lay, qk):
    from hippo_leap_amd.model import DenseModel
    print(f"prefill+decode case {name}", flush=True)
    CFG = CFG128 if name.endswith("_d128") else globals()["CFG"]
    dev, ref = _build(orc, CFG, {}, qk, 77 + len(name))
    T = 12
    m = DenseModel(torch, CFG, dev["tok_emb"], dev["output_norm"], dev["output"], 0, dev["layers"],
                   max_tokens=T, kv_dtype=dt, kv_layout=lay)
    for lw in ref["layers"]:
        lw["k_cache"] = np.zeros((CFG["n_head_kv"] * CFG["head_dim"], CFG["max_len"]), np.float32)
        lw["v_cache"] = np.zeros_like(lw["k_cache"])
    tokens = [int(t) for t in np.random.default_rng(5).integers(0, CFG["n_vocab"], T)]
    logits = m.prefill(tokens)
    torch.cuda.synchronize()
    assert m.cache.cur_len == T
    tol = TOL_F32 if dt == 0 else TOL_LOWP
    ref_logits = _oracle_prefill(orc, CFG, ref, tokens, dt)
    got = logits.cpu().numpy()
    for t in range(T):  # every column (token) against the oracle's
        assert rel_err(got[:, t], ref_logits[:, t]) < tol, f"prefill column {t}"
    # the reference's generate: first token = argmax of the last column
    tok = orc.argmax(got[:, T - 1])
    m.tokens[0] = tok
    for step in range(5):
        pos = T + step
        m.decode()
        torch.cuda.synchronize()
        assert m.cache.cur_len == pos + 1
        lg = m.logits.cpu().numpy()
        assert rel_err(lg, _oracle_decode(orc, CFG, ref, tok, pos, dt)) < tol, f"decode step {step}"
        nxt = int(m.tokens[1].item())
        assert nxt == orc.argmax(lg)
        m.tokens[0] = nxt
        tok = nxt


def test_decode_full_cache_is_refused(hl, orc):
    """A decode step at cur_len == max_len returns "KV cache full" (the
    reference's ValueError, naive.nim:4598-4599) and changes nothing."""
    from hippo_leap_amd import _lib
    from hippo_leap_amd.model import DenseModel
    dev, _ = _build(orc, CFG, {}, False, 99)
    m = DenseModel(torch, CFG, dev["tok_emb"], dev["output_norm"], dev["output"], 0, dev["layers"],
                   max_tokens=CFG["max_len"])
    m.prefill(list(range(CFG["max_len"])))
    torch.cuda.synchronize()
    with pytest.raises(_lib.HLError, match="KV cache full"):
        m.decode()
    assert m.cache.cur_len == CFG["max_len"]


def test_decode_only_with_gguf_weights(hl, orc):
    """hl_forward_decode with quantized weights (the reference's decode
    takes GGUF rows through gpuLinearColQuant) and a bf16 cache, from an
    empty cache: every step writes its column and attends over the columns
    before it."""
    from hippo_leap_amd.model import DenseModel
    types = {"wq": 12, "wk": 12, "wv": 12, "wo": 8, "w_gate": 14, "w_up": 14, "w_down": 13, "output": 14}
    dev, ref = _build(orc, CFG, types, True, 123)
    m = DenseModel(torch, CFG, dev["tok_emb"], dev["output_norm"], dev["output"], 14, dev["layers"],
                   kv_dtype=2)
    for lw in ref["layers"]:
        lw["k_cache"] = np.zeros((CFG["n_head_kv"] * CFG["head_dim"], CFG["max_len"]), np.float32)
        lw["v_cache"] = np.zeros_like(lw["k_cache"])
    tok = 3
    m.tokens[0] = tok
    for pos in range(6):
        m.decode()
        torch.cuda.synchronize()
        lg = m.logits.cpu().numpy()
        assert rel_err(lg, _oracle_decode(orc, CFG, ref, tok, pos, 2)) < TOL_LOWP, f"step {pos}"
        tok = int(m.tokens[1].item())
        assert tok == orc.argmax(lg)
        m.tokens[0] = tok


def test_decode_timed_matches_decode(hl, orc):
    """hl_forward_decode_timed (forwardDecodeTokenTimed, megakernel.nim:
    2514-2529): the same tokens and logits as hl_forward_decode on a twin
    model, a positive GPU time below the host's wall time of the call, and
    HL_ECAPTURE under stream capture."""
    import time
    from hippo_leap_amd import _lib
    from hippo_leap_amd.model import DenseModel
    dev, ref = _build(orc, CFG, {}, True, 321)
    twins = [DenseModel(torch, CFG, dev["tok_emb"], dev["output_norm"], dev["output"], 0, dev["layers"],
                        max_tokens=4, kv_dtype=2) for _ in range(2)]
    for m in twins:
        m.prefill([1, 2, 3, 4])
        m.tokens[0] = 7
    torch.cuda.synchronize()
    for step in range(4):
        twins[0].decode()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tok, ms = twins[1].decode_timed()
        wall_ms = (time.perf_counter() - t0) * 1e3
        assert 0.0 < ms < wall_ms, (ms, wall_ms)
        assert tok == int(twins[0].tokens[1].item()) == int(twins[1].tokens[1].item())
        assert np.array_equal(twins[0].logits.cpu().numpy(), twins[1].logits.cpu().numpy())
        assert twins[1].cache.cur_len == twins[0].cache.cur_len == 5 + step
        for m in twins:
            m.tokens[0] = tok
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(_lib.HLError, match="capture"):
        with torch.cuda.graph(g, stream=s):
            twins[1].decode_timed(stream=s)
