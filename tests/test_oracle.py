"""Pins the CPU oracle (oracle/hl_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
the reference's known-answer test, the committed golden fixtures (fp64,
cross-checked with torch SDPA when written), NumPy/torch library routines,
closed forms and invariants chosen so that a dropped term, wrong sign, wrong
index or transposed operand fails.
"""
import numpy as np
import pytest
import torch

from util import golden, rel_err

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


# ---------------------------------------------------------------------------
# fp16 / bf16 storage
# ---------------------------------------------------------------------------
def test_half_to_float_reference_kat(orc):
    """tests/test_quant.nim:5-15 of the reference, value for value."""
    assert orc.half_to_float(0x0000) == 0.0
    assert orc.half_to_float(0x3C00) == 1.0
    assert orc.half_to_float(0xBC00) == -1.0
    assert orc.half_to_float(0x4000) == 2.0
    assert orc.half_to_float(0x3800) == 0.5
    assert orc.half_to_float(0x7C00) == float("inf")
    assert orc.half_to_float(0xFC00) == float("-inf")
    assert np.isnan(orc.half_to_float(0x7C01))


def test_half_to_float_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.upcast(bits, orc.F16)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _sweep():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10,
        rng.standard_normal(5000).astype(np.float32) * 1e-5,      # fp16 subnormals
        np.float32(2.0) ** rng.integers(-30, 20, 2000).astype(np.float32),
        np.array([65504, 65519, 65520, 70000, -65520, 6.1035156e-05, 5.96e-08, 2.98e-08,
                  1 + 2**-11, 1 + 3 * 2**-11, 1 + 2**-8, 1 + 3 * 2**-8, 0.0, -0.0,
                  np.inf, -np.inf], dtype=np.float32),
    ])
    return x


def test_float_to_half_rne_matches_numpy(orc):
    x = _sweep()
    got = orc.to_storage(x, orc.F16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_float_to_bf16_rne_matches_torch(orc):
    x = _sweep()
    got = orc.to_storage(x, orc.BF16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = orc.upcast(got, orc.BF16)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())


def test_reference_float_to_half_truncates(orc):
    """quant.nim:98-107 truncates and flushes; the caches use RNE instead."""
    x = np.float32(1 + 3 * 2**-11)  # halfway case: RNE rounds up, truncation down
    assert orc.float_to_half_trunc(float(x)) == 0x3C01
    assert int(orc.to_storage(np.array([x]), orc.F16)[0]) == 0x3C02
    assert orc.float_to_half_trunc(3e-5) == 0  # below 2^-14: flushed
    assert int(orc.to_storage(np.array([3e-5], np.float32), orc.F16)[0]) != 0


# ---------------------------------------------------------------------------
# tensor.nim ops
# ---------------------------------------------------------------------------
def test_matmul(orc):
    a = orc.normal(7 * 13, 1).reshape(7, 13)
    b = orc.normal(13 * 5, 2).reshape(13, 5)
    assert rel_err(orc.matmul(a, b), a.astype(np.float64) @ b) < 1e-6
    assert np.array_equal(orc.matmul(np.eye(7, dtype=np.float32), a), a)
    # (a b)^T = b^T a^T catches a transposed operand
    assert rel_err(orc.matmul(b.T, a.T), orc.matmul(a, b).T) < 1e-6


def test_softmax(orc):
    x = orc.normal(4 * 33, 3, 0, 5).reshape(4, 33)
    y = orc.softmax_last_dim(x)
    e = np.exp(x.astype(np.float64) - x.max(-1, keepdims=True))
    assert rel_err(y, e / e.sum(-1, keepdims=True)) < 1e-6
    assert np.allclose(y.sum(-1), 1.0, atol=1e-6)
    assert rel_err(orc.softmax_last_dim(x + 7.5), y) < 1e-5  # shift invariance
    assert np.all(orc.softmax_last_dim(np.zeros((1, 9), np.float32)) == np.float32(1 / 9))


def test_rmsnorm(orc):
    w = orc.uniform(64, 4, 0.5, 1.5)
    c, eps = 0.75, 1e-6
    got = orc.rmsnorm(np.full((2, 64), c, np.float32), w, eps)
    assert rel_err(got[0], w * c / np.sqrt(c * c + eps)) < 1e-6  # closed form
    x = orc.normal(3 * 64, 5).reshape(3, 64)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + eps) * w
    assert rel_err(orc.rmsnorm(x, w, eps), ref) < 1e-6
    # column form on the transpose
    assert rel_err(orc.rmsnorm_cols(np.ascontiguousarray(x.T), w, eps), ref.T) < 1e-6


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------
def test_theta_table(orc):
    for rd, base in ((64, 1e4), (128, 5e5), (128, 1e6)):
        th = orc.theta_table(rd, base)
        i = np.arange(rd // 2, dtype=np.float64)
        ref = (1.0 / base) ** (2 * i / rd)
        assert np.all(np.abs(th - ref) <= 2 * np.spacing(th.astype(np.float32)))
        assert th[0] == 1.0


def test_rope_identity_norm_composition(orc):
    H, D = 3, 64
    th = orc.theta_table(D, 1e4)
    x = orc.normal(H * D, 6)
    assert np.array_equal(orc.rope_heads(x, H, D, D, th, 0), x)  # pos 0 = identity
    for style in (0, 1):
        y = orc.rope_heads(x, H, D, D, th, 17, style)
        xr, yr = x.reshape(H, D).astype(np.float64), y.reshape(H, D).astype(np.float64)
        half = D // 2
        if style == 0:
            px, py = xr[:, :half] ** 2 + xr[:, half:] ** 2, yr[:, :half] ** 2 + yr[:, half:] ** 2
        else:
            px, py = xr[:, 0::2] ** 2 + xr[:, 1::2] ** 2, yr[:, 0::2] ** 2 + yr[:, 1::2] ** 2
        assert np.allclose(px, py, rtol=1e-5)  # rotation preserves each pair's norm
        y2 = orc.rope_heads(orc.rope_heads(x, H, D, D, th, 5, style), H, D, D, th, 12, style)
        assert rel_err(y2, y) < 1e-5  # R(5) R(12) = R(17)
        assert rel_err(y, x) > 1e-2  # and it does rotate


def test_rope_half_split_vs_interleaved_permutation(orc):
    H, D = 2, 16
    th = orc.theta_table(D, 1e4)
    x = orc.normal(H * D, 7).reshape(H, D)
    perm = np.empty(D, np.int64)  # interleaved slot 2i <- i, 2i+1 <- i+D/2
    perm[0::2], perm[1::2] = np.arange(D // 2), np.arange(D // 2) + D // 2
    a = orc.rope_heads(x.reshape(-1), H, D, D, th, 9, 0).reshape(H, D)
    b = orc.rope_heads(x[:, perm].reshape(-1), H, D, D, th, 9, 1).reshape(H, D)
    assert np.array_equal(a[:, perm], b)


def test_rope_partial_rotary_passthrough(orc):
    H, D, rd = 2, 64, 32
    th = orc.theta_table(rd, 1e4)
    x = orc.normal(H * D, 8)
    y = orc.rope_heads(x, H, D, rd, th, 11).reshape(H, D)
    assert np.array_equal(y[:, rd:], x.reshape(H, D)[:, rd:])


def test_rope_inplace_tensor_nim_matches_interleaved_cols(orc):
    """tensor.nim ropeInplace ([outer, seq, dim]) == the interleaved column form."""
    H, D, T = 2, 32, 9
    x = orc.normal(H * T * D, 9).reshape(H, T, D)
    a = orc.rope_inplace(x, 1e4, 3)
    th = orc.theta_table(D, 1e4)
    cols = np.ascontiguousarray(x.transpose(0, 2, 1)).reshape(H * D, T)
    b = orc.rope_cols(cols, H, D, T, D, th, 3, 1).reshape(H, D, T).transpose(0, 2, 1)
    assert rel_err(a, b) < 1e-6


@pytest.mark.parametrize("name", ["prefill_f32_halfsplit", "prefill_f32_interleaved"])
def test_rope_cols_golden(orc, name):
    g = golden(name)
    hq, hkv, d, T, style = (int(v) for v in g["shape"])
    th = orc.theta_table(d, float(g["base"][0]))
    assert rel_err(orc.rope_cols(g["q"], hq, d, T, d, th, 0, style), g["q_roped"]) < 1e-5
    assert rel_err(orc.rope_cols(g["k"], hkv, d, T, d, th, 0, style), g["k_roped"]) < 1e-5


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["decode_f32", "decode_f16", "decode_bf16"])
def test_decode_golden(orc, name):
    g = golden(name)
    hq, hkv, d, L, max_len, dt = (int(v) for v in g["shape"])
    kc, vc = orc.upcast(g["k_cache"], dt), orc.upcast(g["v_cache"], dt)
    out = orc.attention_decode(g["q"], kc, vc, hq, hkv, d, L, max_len)
    assert rel_err(out, g["expected"]) < 1e-5


@pytest.mark.parametrize("name", ["prefill_f32_halfsplit", "prefill_f32_interleaved"])
def test_prefill_golden(orc, name):
    g = golden(name)
    hq, hkv, d, T, style = (int(v) for v in g["shape"])
    out = orc.attention_prefill(g["q_roped"], g["k_roped"], g["v"], hq, hkv, d, T)
    assert rel_err(out, g["expected"]) < 1e-5


def test_decode_closed_forms(orc):
    hq, hkv, d, M = 4, 2, 64, 40
    q = orc.uniform(hq * d, 30)
    kc = orc.uniform(hkv * d * M, 31).reshape(hkv, d, M)
    vc = orc.uniform(hkv * d * M, 32).reshape(hkv, d, M)
    g = hq // hkv
    # L = 1: output is v_0 of the head's kv head
    o = orc.attention_decode(q, kc, vc, hq, hkv, d, 1, M).reshape(hq, d)
    for h in range(hq):
        assert np.array_equal(o[h], vc[h // g, :, 0])
    # identical K columns: uniform weights -> mean of V over L
    kc_same = np.repeat(kc[:, :, :1], M, axis=2)
    o = orc.attention_decode(q, kc_same, vc, hq, hkv, d, 23, M).reshape(hq, d)
    for h in range(hq):
        assert rel_err(o[h], vc[h // g, :, :23].astype(np.float64).mean(-1)) < 1e-5
    # q = 0: same mean
    o = orc.attention_decode(np.zeros_like(q), kc, vc, hq, hkv, d, 23, M).reshape(hq, d)
    assert rel_err(o[1], vc[0, :, :23].astype(np.float64).mean(-1)) < 1e-5
    # GQA mapping: replicating kv heads to MHA gives the same result
    o_gqa = orc.attention_decode(q, kc, vc, hq, hkv, d, 31, M)
    o_mha = orc.attention_decode(q, np.repeat(kc, g, 0), np.repeat(vc, g, 0), hq, hq, d, 31, M)
    assert np.array_equal(o_gqa, o_mha)
    # a wrong group mapping (h % Hkv) would differ
    assert rel_err(o_gqa.reshape(hq, d)[1], o_gqa.reshape(hq, d)[2]) > 1e-3


def test_prefill_closed_forms_and_causality(orc):
    hq, hkv, d, T = 4, 2, 64, 40
    q = orc.normal(hq * d * T, 40).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 41).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 42).reshape(hkv * d, T)
    o = orc.attention_prefill(q, k, v, hq, hkv, d, T)
    g = hq // hkv
    o3, v3 = o.reshape(hq, d, T), v.reshape(hkv, d, T)
    for h in range(hq):
        assert np.array_equal(o3[h, :, 0], v3[h // g, :, 0])  # row 0 = v_0
    # last row equals decode with L = T over the same K/V
    dec = orc.attention_decode(np.ascontiguousarray(q[:, T - 1]), k, v, hq, hkv, d, T, T)
    assert rel_err(o[:, T - 1], dec) < 1e-6
    # causality: perturbing K/V at j > i leaves row i unchanged
    i = 17
    k2, v2 = k.copy(), v.copy()
    k2[:, i + 1:] += 3.0
    v2[:, i + 1:] -= 2.0
    o2 = orc.attention_prefill(q, k2, v2, hq, hkv, d, T)
    assert np.array_equal(o2[:, :i + 1], o[:, :i + 1])
    assert not np.allclose(o2[:, i + 1:], o[:, i + 1:])
    # row subsets reproduce the full computation
    sub = orc.attention_prefill(q, k, v, hq, hkv, d, T, heads=(1, 3), rows=(3, T, 7))
    assert np.array_equal(sub[64:192, 3::7], o[64:192, 3::7])


def test_decode_step_golden(orc):
    for name in ("decode_step_bf16_qknorm", "decode_step_f16_qknorm"):
        g = golden(name)
        hq, hkv, d, prev, max_len, dt = (int(v) for v in g["shape"])
        eps, base = float(g["eps"][0]), float(g["base"][0])
        th = orc.theta_table(d, base)
        qn = orc.rope_heads(orc.qk_norm(g["q"], g["wq"], hq, d, eps), hq, d, d, th, prev)
        kn = orc.rope_heads(orc.qk_norm(g["k"], g["wk"], hkv, d, eps), hkv, d, d, th, prev)
        assert rel_err(qn, g["q_rot"]) < 1e-5 and rel_err(kn, g["k_rot"]) < 1e-5
        kc, vc = g["k_cache"].copy(), g["v_cache"].copy()
        orc.store_kv(kc, dt, kn, hkv * d, 1, max_len, prev)
        orc.store_kv(vc, dt, g["v"], hkv * d, 1, max_len, prev)
        out = orc.attention_decode(qn, orc.upcast(kc, dt), orc.upcast(vc, dt), hq, hkv, d,
                                   prev + 1, max_len)
        assert rel_err(out, g["expected"]) < 1e-5


def test_decode_fp64_brute_force(orc):
    rng = np.random.default_rng(0)
    for hq, hkv, d, L in ((6, 3, 64, 5), (8, 1, 128, 129)):
        M = L + 3
        q = rng.standard_normal(hq * d).astype(np.float32)
        kc = rng.standard_normal(hkv * d * M).astype(np.float32)
        vc = rng.standard_normal(hkv * d * M).astype(np.float32)
        out = orc.attention_decode(q, kc, vc, hq, hkv, d, L, M).reshape(hq, d)
        K = kc.reshape(hkv, d, M).astype(np.float64)
        V = vc.reshape(hkv, d, M).astype(np.float64)
        for h in range(hq):
            kv = h // (hq // hkv)
            s = q.reshape(hq, d)[h].astype(np.float64) @ K[kv, :, :L] / np.sqrt(d)
            p = np.exp(s - s.max())
            assert rel_err(out[h], V[kv, :, :L] @ (p / p.sum())) < 1e-5


# ---------------------------------------------------------------------------
# decode-step ends: argmax (naive.nim:1922-2127), embedding (:2975-3001)
# ---------------------------------------------------------------------------
def _bitrev8(v):
    return int(f"{v:08b}"[::-1], 2)


def _argmax_closed_form(x):
    """Winner implied by the reference's reduction tree: among the maxima of
    the values > -3.4e38, the smallest (bitrev8(b), bitrev8(t), r) for
    i = 65536 r + 256 b + t; -1 when no value qualifies."""
    x = np.asarray(x, np.float32)
    ok = x > np.float32(-3.4e38)
    if not ok.any():
        return -1
    m = x[ok].max()
    cand = np.nonzero(ok & (x == m))[0]
    return int(min(cand, key=lambda i: (_bitrev8((i >> 8) & 255), _bitrev8(i & 255), i >> 16)))


def test_argmax_tie_free_matches_numpy(orc):
    for n, seed in ((1, 1), (7, 2), (300, 3), (65536, 4), (128256, 5), (152064, 6)):
        x = orc.normal(n, 3400 + seed)
        assert orc.argmax(x) == int(np.argmax(x))


@pytest.mark.parametrize("n,levels,seed", [(200000, 3, 1), (70000, 2, 2), (131072, 1, 3),
                                           (1000, 2, 4), (65537, 1, 5)])
def test_argmax_ties_follow_the_reduction_tree(orc, n, levels, seed):
    """Tie-heavy inputs (values drawn from `levels` integers): the literal
    simulation of the two-pass kernel agrees with the tie order derived
    from its merge structure."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, levels, n).astype(np.float32)
    assert orc.argmax(x) == _argmax_closed_form(x)


def test_argmax_hand_cases(orc):
    x = np.zeros(300, np.float32)
    # all equal: bitrev8 favours even thread indices; thread 0 of block 0 is index 0
    assert orc.argmax(x) == 0
    x = np.full(300, -1.0, np.float32)
    x[[5, 260, 129]] = 2.0        # i=129: b=0, t=129 (bitrev 0b10000001); i=5: t=5 (0b10100000)
    assert orc.argmax(x) == 129  # t=129 -> bitrev 129; t=5 -> bitrev 160; i=260: b=1 -> bitrev 128 > 0
    x = np.full(70000, 0.0, np.float32)
    x[0] = -1.0                  # index 0 loses; 65536 shares slot 0 (r = 1) and wins over slot 1
    assert orc.argmax(x) == 65536
    # NaN and values <= -3.4e38 are never chosen; all of them -> -1
    assert orc.argmax(np.array([np.nan, -np.inf, -3.4e38, 1.0], np.float32)) == 3
    assert orc.argmax(np.array([np.nan, -np.inf, -3.4e38], np.float32)) == -1
    assert orc.argmax(np.zeros(0, np.float32)) == -1
    # -0.0 and +0.0 are equal to the reference's >: the tree order decides
    assert orc.argmax(np.array([-0.0, 0.0], np.float32)) == 0


def test_embedding_matches_indexing(orc):
    n_vocab, n_emb = 50, 24
    w = orc.normal(n_vocab * n_emb, 3500).reshape(n_vocab, n_emb)
    tok = np.array([3, 0, 49, 3, 17], np.int32)
    out = orc.embedding(w, tok, n_emb)
    assert np.array_equal(out, w[tok].T)


# ---------------------------------------------------------------------------
# fp8 e4m3 KV storage (the library's extension; no reference counterpart)
# ---------------------------------------------------------------------------
def test_e4m3_decode_all_codes_match_torch(orc):
    import torch
    codes = np.arange(256, dtype=np.uint8)
    got = orc.upcast(codes, orc.FP8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok]) and np.array_equal(np.signbit(got[ok]), np.signbit(ref[ok]))


def test_e4m3_encode_matches_torch_below_overflow(orc):
    """Round to nearest even, bit for bit with torch's float8_e4m3fn cast for
    every |x| < 464 (where torch does not overflow), over a dense sweep that
    includes every rounding midpoint; saturation at +-448 above it."""
    import torch
    rng = np.random.default_rng(0)
    codes = torch.arange(0, 126, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mids = (codes[:-1] + codes[1:]) / 2                     # exact ties
    x = np.concatenate([rng.uniform(-463.9, 463.9, 200000), rng.normal(0, 0.01, 100000),
                        codes, -codes, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                        [0.0, -0.0, 448.0, -448.0, 463.99]]).astype(np.float32)
    got = orc.to_storage(x, orc.FP8)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)
    big = np.array([464.0, 480.0, 1e30, np.inf, -np.inf, -1e9], np.float32)
    assert orc.to_storage(big, orc.FP8).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert orc.to_storage(np.array([np.nan], np.float32), orc.FP8)[0] & 0x7F == 0x7F


# ---------------------------------------------------------------------------
# GGUF weight rows (quant.nim:235-355)
# ---------------------------------------------------------------------------
def test_dequant_q8_0_packed(orc):
    from gguf_pack import pack_q8_0
    rng = np.random.default_rng(10)
    d = np.asarray(rng.uniform(0.01, 1.0, 3), np.float16)
    q = rng.integers(-128, 128, (3, 32))
    got = orc.dequant_rows(8, pack_q8_0(d, q), 1, 96)
    assert np.array_equal(got.reshape(3, 32), (q * d.astype(np.float32)[:, None]).astype(np.float32))


def test_dequant_q4_k_packed(orc):
    """Every 6-bit scale and min position, including the split high-index
    ones, round-trips through the format's packing."""
    from gguf_pack import pack_q4_k, q4_k_values
    rng = np.random.default_rng(11)
    nb = 4
    d = np.asarray(rng.uniform(0.01, 0.1, nb), np.float16)
    dmin = np.asarray(rng.uniform(0.0, 0.1, nb), np.float16)
    sc = rng.integers(0, 64, (nb, 8))
    mn = rng.integers(0, 64, (nb, 8))
    sc[0] = [63, 0, 1, 62, 32, 33, 16, 47]   # top bits of every high-index scale exercised
    mn[0] = [0, 63, 31, 32, 48, 15, 63, 1]
    q = rng.integers(0, 16, (nb, 256))
    got = orc.dequant_rows(12, pack_q4_k(d, dmin, sc, mn, q), 1, 256 * nb).reshape(nb, 256)
    assert np.allclose(got, q4_k_values(d, dmin, sc, mn, q), rtol=1e-6, atol=1e-6)


def test_dequant_q6_k_packed(orc):
    from gguf_pack import pack_q6_k, q6_k_values
    rng = np.random.default_rng(12)
    nb = 3
    d = np.asarray(rng.uniform(0.001, 0.05, nb), np.float16)
    sc = rng.integers(-128, 128, (nb, 16))
    q = rng.integers(-32, 32, (nb, 256))
    q[0, :8] = [-32, 31, 0, -1, 15, 16, -17, 30]
    got = orc.dequant_rows(14, pack_q6_k(d, sc, q), 1, 256 * nb).reshape(nb, 256)
    assert np.allclose(got, q6_k_values(d, sc, q), rtol=1e-6, atol=1e-6)


def test_dequant_f16(orc):
    x = np.asarray(np.random.default_rng(13).standard_normal(64), np.float16)
    assert np.array_equal(orc.dequant_rows(1, x.view(np.uint8), 2, 32).reshape(-1), x.astype(np.float32))


def test_dequant_q5_0_q5_1_iq4nl_packed(orc):
    from gguf_pack import IQ4NL_LEVELS, pack_iq4nl, pack_q5_0, pack_q5_1
    rng = np.random.default_rng(14)
    nb = 3
    d = np.asarray(rng.uniform(0.01, 0.5, nb), np.float16)
    m = np.asarray(rng.uniform(-1, 1, nb), np.float16)
    q = rng.integers(0, 32, (nb, 32))
    q[0] = np.arange(32)  # every 5-bit value, high bit in every position
    d64 = d.astype(np.float64)[:, None]
    got = orc.dequant_rows(6, pack_q5_0(d, q), 1, 32 * nb).reshape(nb, 32)
    assert np.allclose(got, d64 * (q - 16), rtol=1e-6, atol=1e-7)
    got = orc.dequant_rows(7, pack_q5_1(d, m, q), 1, 32 * nb).reshape(nb, 32)
    assert np.allclose(got, d64 * q + m.astype(np.float64)[:, None], rtol=1e-6, atol=1e-6)
    idx = rng.integers(0, 16, (nb, 32))
    idx[0, :16] = np.arange(16)
    got = orc.dequant_rows(20, pack_iq4nl(d, idx), 1, 32 * nb).reshape(nb, 32)
    assert np.allclose(got, d64 * IQ4NL_LEVELS[idx], rtol=1e-6, atol=1e-7)


def test_dequant_q2_k_packed(orc):
    from gguf_pack import pack_q2_k, scaled_values
    rng = np.random.default_rng(15)
    nb = 3
    d = np.asarray(rng.uniform(0.01, 0.1, nb), np.float16)
    dmin = np.asarray(rng.uniform(0.0, 0.1, nb), np.float16)
    sc, mn = rng.integers(0, 16, (nb, 16)), rng.integers(0, 16, (nb, 16))
    sc[0], mn[0] = np.arange(16), np.arange(16)[::-1]
    q = rng.integers(0, 4, (nb, 256))
    got = orc.dequant_rows(10, pack_q2_k(d, dmin, sc, mn, q), 1, 256 * nb).reshape(nb, 256)
    assert np.allclose(got, scaled_values(d, sc, q, 16, dmin, mn), rtol=1e-6, atol=1e-6)


def test_dequant_q3_k_packed(orc):
    """All 16 6-bit scales (4 low bits in two nibble halves, 2 high bits in
    shared bytes) and every hmask bit position."""
    from gguf_pack import pack_q3_k, scaled_values
    rng = np.random.default_rng(16)
    nb = 3
    d = np.asarray(rng.uniform(0.01, 0.1, nb), np.float16)
    sc = rng.integers(0, 64, (nb, 16))
    sc[0] = [0, 63, 1, 62, 16, 47, 32, 31, 15, 48, 5, 58, 33, 30, 7, 56]
    q = rng.integers(-4, 4, (nb, 256))
    got = orc.dequant_rows(11, pack_q3_k(d, sc, q), 1, 256 * nb).reshape(nb, 256)
    assert np.allclose(got, scaled_values(d, sc - 32, q, 16), rtol=1e-6, atol=1e-6)


def test_dequant_q5_k_packed(orc):
    """Q5_K as the format (and the reference's GPU kernel,
    naive.nim:1267-1323) defines it: bit s of qh[l] is the high bit of
    element 32s + l."""
    from gguf_pack import pack_q5_k, scaled_values
    rng = np.random.default_rng(17)
    nb = 3
    d = np.asarray(rng.uniform(0.01, 0.1, nb), np.float16)
    dmin = np.asarray(rng.uniform(0.0, 0.1, nb), np.float16)
    sc, mn = rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8))
    sc[0], mn[0] = [63, 0, 1, 62, 32, 33, 16, 47], [0, 63, 31, 32, 48, 15, 63, 1]
    q = rng.integers(0, 32, (nb, 256))
    q[1] = 16  # only the high bits set: a misplaced qh bit shows directly
    got = orc.dequant_rows(13, pack_q5_k(d, dmin, sc, mn, q), 1, 256 * nb).reshape(nb, 256)
    assert np.allclose(got, scaled_values(d, sc, q, 32, dmin, mn), rtol=1e-6, atol=1e-6)


def test_add_is_ieee_fp32_addition(orc):
    """tensor.nim add (:42-47): one fp32 addition per element, so the result
    is numpy's float32 sum bit for bit (ties, signed zeros, infinities)."""
    a = np.concatenate([orc.normal(1000, 51), np.float32([0.0, -0.0, np.inf, 1e38, 1.0])])
    b = np.concatenate([orc.normal(1000, 52), np.float32([-0.0, -0.0, 1.0, 1e38, np.float32(2 ** -24)])])
    got = orc.add(a, b)
    assert np.array_equal(got.view(np.uint32), (a + b).view(np.uint32))


def test_silu_mul_against_fp64_and_limits(orc):
    """gpuSiluMul (naive.nim:2179-2187): x * sigmoid(x) * up.  Pinned by an
    fp64 evaluation, and by its limits: silu(0) = 0; for x >= 20 the fp32
    sigmoid is exactly 1 (the result is x * up, exactly); for x <= -104,
    exp(-x) overflows to inf and the result is a signed zero."""
    g = orc.normal(4000, 53) * np.float32(4)
    u = orc.normal(4000, 54)
    got = orc.silu_mul(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 1e-6
    edge_g = np.float32([0.0, 20.0, 37.5, -104.0, -200.0])
    edge_u = np.float32([3.0, 1.25, -2.0, 5.0, -5.0])
    e = orc.silu_mul(edge_g, edge_u)
    assert e[0] == 0.0
    assert e[1] == np.float32(20.0) * np.float32(1.25) and e[2] == np.float32(37.5) * np.float32(-2.0)
    assert e[3] == 0.0 and e[4] == 0.0
    # the GPU form x * (1/(1+e)) * u and the CPU form x / (1+e) * u differ by
    # at most a couple of ulps: both are the same function
    cpu_form = (g / (np.float32(1) + np.exp(-g, dtype=np.float32)) * u).astype(np.float32)
    assert np.max(np.abs(got - cpu_form) / np.maximum(np.abs(cpu_form), 1e-30)) < 1e-6
