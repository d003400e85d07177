"""GPU parity: causal prefill with fused qkNorm / RoPE / KV-cache write
(hl_attn_prefill, hl_gpu_attention_prefill) against the CPU oracle."""
import numpy as np
import pytest
import torch

from util import TOL_F32, TOL_LOWP, golden, rel_err

pytestmark = pytest.mark.gpu

TDT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def to_dev(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(TDT[dt])


def from_dev(t):
    return t.float().cpu().numpy()


def run_prefill(q, k, v, hq, hkv, d, T, out_dtype=torch.float32, **kw):
    from hippo_leap_amd import attention as A
    out = torch.full(q.shape, float("nan"), dtype=out_dtype, device="cuda")
    a = A.prefill_args(q, k, v, out, hq, hkv, d, T, **kw)
    ws = A.workspace(A.prefill_workspace_bytes(a))
    A.attn_prefill(a, ws)
    torch.cuda.synchronize()
    return out


def oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=None, style=0, wq=None, wk=None, eps=1e-6,
                   heads=None, rows=None, rope_dim=None):
    q, k = q.copy(), k.copy()
    if wq is not None:
        q = orc.qk_norm_cols(q, wq, hq, d, T, eps)
        k = orc.qk_norm_cols(k, wk, hkv, d, T, eps)
    if base is not None:
        rd = rope_dim or d
        th = orc.theta_table(rd, base)
        q = orc.rope_cols(q, hq, d, T, rd, th, 0, style)
        k = orc.rope_cols(k, hkv, d, T, rd, th, 0, style)
    return orc.attention_prefill(q, k, v, hq, hkv, d, T, heads=heads, rows=rows), q, k


@pytest.mark.parametrize("name", ["prefill_f32_halfsplit", "prefill_f32_interleaved"])
def test_prefill_golden_fp32(hl, name):
    g = golden(name)
    hq, hkv, d, T, style = (int(v) for v in g["shape"])
    out = run_prefill(to_dev(g["q"], 0), to_dev(g["k"], 0), to_dev(g["v"], 0), hq, hkv, d, T,
                      apply_rope=True, rope_base=float(g["base"][0]), rope_style=style)
    assert rel_err(from_dev(out), g["expected"]) < TOL_F32 / 10


def test_prefill_reference_dropin(hl, orc):
    """gpuAttentionPrefill signature: already-roped fp32 projections.  At head
    dim 64 the call uses a library-held workspace (the K/V split images):
    the second length grows it, the third runs in the larger one."""
    from hippo_leap_amd import attention as A
    hq, hkv, d = 32, 4, 64
    for T in (300, 700, 65):
        q = orc.normal(hq * d * T, 11 + T).reshape(hq * d, T)
        k = orc.normal(hkv * d * T, 12 + T).reshape(hkv * d, T)
        v = orc.normal(hkv * d * T, 13 + T).reshape(hkv * d, T)
        ref = orc.attention_prefill(q, k, v, hq, hkv, d, T)
        dst = torch.empty(hq * d, T, device="cuda")
        A.gpu_attention_prefill(dst, to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T)
        torch.cuda.synchronize()
        assert rel_err(from_dev(dst), ref) < TOL_F32, T


def test_prefill_c2_full(hl, orc):
    """Config 2: T=512, Hq32/Hkv4, D64 fp32, RoPE 1e4 on q,k, KV cache written."""
    hq, hkv, d, T, max_len = 32, 4, 64, 512, 600
    q = orc.normal(hq * d * T, 21).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 22).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 23).reshape(hkv * d, T)
    ref, qr, kr = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e4)
    kc = torch.full((hkv * d, max_len), 7.0, device="cuda")
    vc = torch.full((hkv * d, max_len), 7.0, device="cuda")
    qd, kd = to_dev(q, 0), to_dev(k, 0)
    out = run_prefill(qd, kd, to_dev(v, 0), hq, hkv, d, T, apply_rope=True, rope_base=1e4,
                      k_cache=kc, v_cache=vc, max_len=max_len, write_back_qk=True)
    err = rel_err(from_dev(out), ref)
    print(f"c2 rel err {err:.3e}")
    assert err < TOL_F32
    # in-place semantics of the reference: q, k hold the roped values
    assert rel_err(from_dev(qd), qr) < 1e-5 and rel_err(from_dev(kd), kr) < 1e-5
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    assert rel_err(kcn[:, :T], kr) < 1e-5
    assert np.array_equal(vcn[:, :T], v)                  # V stored bit-exactly
    assert np.all(kcn[:, T:] == 7.0) and np.all(vcn[:, T:] == 7.0)  # canary untouched


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("T", [1, 2, 31, 33, 63, 65, 127, 130, 257])
def test_prefill_fp32_split_path_lengths(hl, orc, T, d):
    """The fp32 kernel's steps run on fp16 hi/lo splits of the operands (K
    and V split by the prologue per 32-key half tile); partial tiles and
    lengths that are not a multiple of 4 against the fp32 oracle."""
    hq, hkv = 8, 2
    q = orc.normal(hq * d * T, 40 + T).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 41 + T).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 42 + T).reshape(hkv * d, T)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e4)
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T, apply_rope=True,
                      rope_base=1e4)
    err = rel_err(from_dev(out), ref)
    print(f"split path D={d} T={T} rel err {err:.3e}")
    assert err < TOL_F32 / 10


@pytest.mark.parametrize("T", [65, 200])
@pytest.mark.parametrize("hq,hkv,d", [(4, 4, 64), (6, 3, 128), (16, 2, 64), (8, 2, 128), (12, 4, 64)])
def test_prefill_fp32_split_path_gqa(hl, orc, hq, hkv, d, T):
    """GQA groups of 1, 2, 3, 4 and 8 query heads per kv head (workgroups of
    one, two or four heads, with and without the two-way key split) through
    the split-operand fp32 kernel, with the KV cache written."""
    q = orc.normal(hq * d * T, 70 + T).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 71 + T).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 72 + T).reshape(hkv * d, T)
    ref, _, kr = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e4)
    kc = torch.zeros(hkv * d, T, device="cuda")
    vc = torch.zeros(hkv * d, T, device="cuda")
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T, apply_rope=True,
                      rope_base=1e4, k_cache=kc, v_cache=vc, max_len=T)
    assert rel_err(from_dev(out), ref) < TOL_F32 / 10
    assert np.array_equal(from_dev(vc), v)
    assert rel_err(from_dev(kc), kr) < 1e-6


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("style,half_rope", [(0, False), (1, False), (0, True)])
def test_prefill_fp32_split_path_qknorm_rope(hl, orc, d, style, half_rope):
    """fp32 with qkNorm and RoPE (half-split, interleaved, half-split over
    half the head) applied by the prologue before it splits K: the oracle's
    norm and rotation, then attention."""
    hq, hkv, T = 8, 2, 150
    rd = d // 2 if half_rope else d
    q = orc.normal(hq * d * T, 81).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 82).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 83).reshape(hkv * d, T)
    wq, wk = orc.uniform(d, 84, 0.5, 1.5), orc.uniform(d, 85, 0.5, 1.5)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e6, style=style, wq=wq, wk=wk,
                               rope_dim=rd)
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T, apply_rope=True,
                      rope_base=1e6, rope_style=style, rope_dim=rd,
                      q_norm_w=torch.from_numpy(wq).cuda(), k_norm_w=torch.from_numpy(wk).cuda())
    err = rel_err(from_dev(out), ref)
    print(f"fp32 qknorm rope D={d} style={style} rope_dim={rd} rel err {err:.3e}")
    assert err < TOL_F32 / 10


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("style", [0, 1])
def test_prefill_fp32_split_path_start_pos(hl, orc, d, style):
    """fp32 chunk continuing a sequence: RoPE at positions start_pos + t, the
    cache written from column start_pos (earlier and later columns
    untouched), attention over the chunk's own keys."""
    hq, hkv, T, start, max_len = 8, 2, 70, 37, 128
    q, k, v = (orc.normal(h * d * T, 180 + i).reshape(h * d, T) for i, h in enumerate((hq, hkv, hkv)))
    th = orc.theta_table(d, 5e5)
    qr = orc.rope_cols(q, hq, d, T, d, th, start, style)
    kr = orc.rope_cols(k, hkv, d, T, d, th, start, style)
    ref = orc.attention_prefill(qr, kr, v, hq, hkv, d, T)
    kc = torch.full((hkv * d, max_len), 7.0, device="cuda")
    vc = torch.full((hkv * d, max_len), 7.0, device="cuda")
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T, apply_rope=True,
                      rope_base=5e5, rope_style=style, k_cache=kc, v_cache=vc, max_len=max_len,
                      start_pos=start)
    assert rel_err(from_dev(out), ref) < TOL_F32 / 10
    kch, vch = from_dev(kc), from_dev(vc)
    assert np.array_equal(vch[:, start:start + T], v)
    assert rel_err(kch[:, start:start + T], kr) < 1e-6
    assert np.all(kch[:, :start] == 7.0) and np.all(kch[:, start + T:] == 7.0)
    assert np.all(vch[:, :start] == 7.0) and np.all(vch[:, start + T:] == 7.0)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("where", ["k_tile", "v_tile", "q_row", "tiny"])
def test_prefill_fp32_split_path_outliers(hl, orc, where, d):
    """T=300: values of 2^15 and beyond in one K tile, one V tile or one
    query row, and tiny ones, through the scaled fp16 split (each set is
    scaled so that its largest element sits below 2^14).  Against the fp32
    oracle."""
    hq, hkv, T = 8, 2, 300
    q = orc.normal(hq * d * T, 51).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 52).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 53).reshape(hkv * d, T)
    if where == "k_tile":
        k[5, 70:80] = 1e5          # keys 70..79 of kv head 0 (tile 1)
        k[d + 9, 200] = -4e4       # kv head 1, tile 3
        q[5::d, :] = 0.0           # those dims do not reach the scores (a score
        q[9::d, :] = 0.0           # of ~1e4 would leave the softmax ill-conditioned)
    elif where == "v_tile":
        v[3, 130:140] = 5e4        # tile 2 of kv head 0
        v[d + 60, 299] = -1e6      # last key of kv head 1
    elif where == "q_row":
        q[2 * d + 7, 150] = 3e5    # q * scale beyond 2^15 for one row of head 2
    else:
        k[:, 100:110] *= 1e-30
        v[:, 100:110] *= 1e-30
        q[:, 40:50] *= 1e-20
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T)
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T)
    err = rel_err(from_dev(out), ref)
    print(f"outliers {where} D={d} rel err {err:.3e}")
    assert np.isfinite(from_dev(out)).all() and err < TOL_F32


@pytest.mark.parametrize("d", [64, 128])
def test_prefill_fp32_split_path_nan_key(hl, orc, d):
    """A NaN in one V entry at the first key of a 64-key tile: the steps that
    load the tile run fp32 MFMAs, and exactly the rows that see that key come
    out NaN, as in the oracle; the other rows match it.  (Within a tile the
    P V product is a matrix product, so a NaN at a later key of the tile
    also reaches the earlier rows that process the tile: 0 x NaN.)"""
    hq, hkv, T = 8, 2, 200
    q = orc.normal(hq * d * T, 61).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 62).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 63).reshape(hkv * d, T)
    v[5, 128] = np.nan  # kv head 0, key 128 (first key of tile 2)
    with np.errstate(invalid="ignore"):
        ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T)
    out = from_dev(run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T))
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.abs(out[fin] - ref[fin]).max() / np.abs(ref[fin]).max() < TOL_F32


@pytest.mark.parametrize("T", [1, 2, 31, 32, 33, 63, 64, 65, 127, 200])
def test_prefill_fp32_lengths(hl, orc, T):
    hq, hkv, d = 8, 2, 128
    q = orc.normal(hq * d * T, 30 + T).reshape(hq * d, T)
    k = orc.normal(hkv * d * T, 31 + T).reshape(hkv * d, T)
    v = orc.normal(hkv * d * T, 32 + T).reshape(hkv * d, T)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5)
    out = run_prefill(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T, apply_rope=True,
                      rope_base=5e5)
    assert rel_err(from_dev(out), ref) < TOL_F32


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("T", [1, 17, 32, 64, 65, 100, 136, 257])
@pytest.mark.parametrize("hq,hkv,d", [(8, 2, 128), (4, 4, 64), (16, 2, 64), (6, 3, 128)])
def test_prefill_mfma_shapes(hl, orc, dt, T, hq, hkv, d):
    qs = orc.to_storage(orc.normal(hq * d * T, 40 + T), dt)
    ks = orc.to_storage(orc.normal(hkv * d * T, 41 + T), dt)
    vs = orc.to_storage(orc.normal(hkv * d * T, 42 + T), dt)
    q, k, v = (orc.upcast(x, dt).reshape(-1, T) for x in (qs, ks, vs))
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5)
    out = run_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                      apply_rope=True, rope_base=5e5)
    assert rel_err(from_dev(out), ref) < TOL_LOWP


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("style,rd", [(1, 64), (0, 128), (0, 64)])
@pytest.mark.parametrize("T", [150, 152])
def test_prefill_mfma_qknorm_rope_cache(hl, orc, dt, style, rd, T):
    """qkNorm + RoPE + cache write.  Interleaved (any rope_dim) and full-width
    half-split RoPE are applied to Q inside the MFMA kernel; half-split over
    part of the head goes through the prepared-Q layout.  T = 152 (a multiple
    of 8) fetches q through the LDS staging copies, T = 150 element-wise."""
    hq, hkv, d, max_len = 16, 4, 128, 160
    q, k, v = (orc.upcast(orc.to_storage(orc.normal(h * d * T, 50 + i), dt), dt).reshape(-1, T)
               for i, h in enumerate((hq, hkv, hkv)))
    wq, wk = orc.uniform(d, 53, 0.5, 1.5), orc.uniform(d, 54, 0.5, 1.5)
    ref, _, kr = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e6, style=style, wq=wq, wk=wk,
                                rope_dim=rd)
    kc = torch.zeros(hkv * d, max_len, dtype=TDT[dt], device="cuda")
    vc = torch.zeros(hkv * d, max_len, dtype=TDT[dt], device="cuda")
    out = run_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                      apply_rope=True, rope_base=1e6, rope_style=style, rope_dim=rd,
                      q_norm_w=torch.from_numpy(wq).cuda(), k_norm_w=torch.from_numpy(wk).cuda(),
                      k_cache=kc, v_cache=vc, max_len=max_len)
    assert rel_err(from_dev(out), ref) < TOL_LOWP
    # cache: V bit-exact conversion; K within one storage ulp of the oracle's roped K
    assert np.array_equal(from_dev(vc)[:, :T], v)
    assert rel_err(from_dev(kc)[:, :T], kr) < 2 ** -7


@pytest.mark.parametrize("style", [0, 1])
def test_prefill_mfma_start_pos(hl, orc, style):
    """A chunk that continues a sequence: RoPE at positions start_pos + t and
    the cache written from column start_pos; earlier columns untouched."""
    hq, hkv, d, T, start, max_len, dt = 8, 2, 64, 70, 37, 128, 2
    q, k, v = (orc.upcast(orc.to_storage(orc.normal(h * d * T, 80 + i), dt), dt).reshape(-1, T)
               for i, h in enumerate((hq, hkv, hkv)))
    th = orc.theta_table(d, 5e5)
    qr = orc.rope_cols(q, hq, d, T, d, th, start, style)
    kr = orc.rope_cols(k, hkv, d, T, d, th, start, style)
    ref = orc.attention_prefill(qr, kr, v, hq, hkv, d, T)
    kc = torch.full((hkv * d, max_len), 7.0, dtype=TDT[dt], device="cuda")
    vc = torch.full((hkv * d, max_len), 7.0, dtype=TDT[dt], device="cuda")
    out = run_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                      apply_rope=True, rope_base=5e5, rope_style=style, k_cache=kc, v_cache=vc,
                      max_len=max_len, start_pos=start)
    assert rel_err(from_dev(out), ref) < TOL_LOWP
    kch, vch = from_dev(kc), from_dev(vc)
    assert np.array_equal(vch[:, start:start + T], v)
    assert rel_err(kch[:, start:start + T], kr) < 2 ** -7
    assert np.all(kch[:, :start] == 7.0) and np.all(kch[:, start + T:] == 7.0)
    assert np.all(vch[:, :start] == 7.0) and np.all(vch[:, start + T:] == 7.0)


@pytest.mark.parametrize("dt", [1, 2])
def test_prefill_mfma_no_rope_cache_start_pos(hl, orc, dt):
    """D=128 without RoPE or qkNorm (K/V prologue only converts and stores),
    cache written from start_pos, T not a multiple of the tile."""
    hq, hkv, d, T, start, max_len = 8, 2, 128, 77, 19, 128
    q, k, v = (orc.upcast(orc.to_storage(orc.normal(h * d * T, 90 + i), dt), dt).reshape(-1, T)
               for i, h in enumerate((hq, hkv, hkv)))
    ref = orc.attention_prefill(q, k, v, hq, hkv, d, T)
    kc = torch.full((hkv * d, max_len), 5.0, dtype=TDT[dt], device="cuda")
    vc = torch.full((hkv * d, max_len), 5.0, dtype=TDT[dt], device="cuda")
    out = run_prefill(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T, k_cache=kc,
                      v_cache=vc, max_len=max_len, start_pos=start)
    assert rel_err(from_dev(out), ref) < TOL_LOWP
    kch, vch = from_dev(kc), from_dev(vc)
    assert np.array_equal(kch[:, start:start + T], k) and np.array_equal(vch[:, start:start + T], v)
    assert np.all(kch[:, :start] == 5.0) and np.all(kch[:, start + T:] == 5.0)
    assert np.all(vch[:, :start] == 5.0) and np.all(vch[:, start + T:] == 5.0)


def test_prefill_c4_full_size_sampled(hl, orc):
    """Config 4 at full size (T=4096, Hq32/Hkv8, D128, bf16, RoPE 5e5, cache
    write); the oracle checks 4 heads x 48 sampled rows incl. first/last."""
    hq, hkv, d, T, dt = 32, 8, 128, 4096, 2
    gen = torch.Generator(device="cuda").manual_seed(60)
    qd = torch.randn(hq * d, T, generator=gen, device="cuda").to(torch.bfloat16)
    kd = torch.randn(hkv * d, T, generator=gen, device="cuda").to(torch.bfloat16)
    vd = torch.randn(hkv * d, T, generator=gen, device="cuda").to(torch.bfloat16)
    kc = torch.zeros(hkv * d, T, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros(hkv * d, T, dtype=torch.bfloat16, device="cuda")
    out = from_dev(run_prefill(qd, kd, vd, hq, hkv, d, T, apply_rope=True, rope_base=5e5,
                               k_cache=kc, v_cache=vc, max_len=T))
    q, k, v = from_dev(qd), from_dev(kd), from_dev(vd)
    th = orc.theta_table(d, 5e5)
    qr = orc.rope_cols(q, hq, d, T, d, th)
    kr = orc.rope_cols(k, hkv, d, T, d, th)
    # rows 0, 97, 194, ... and the last 5 rows of every 16th near the end (incl. 4095)
    samples = [(0, T, 97), (T - 65, T, 16)]
    for h in (0, 5, 17, 31):
        blk = slice(h * d, (h + 1) * d)
        for r0, r1, rs in samples:
            ref = orc.attention_prefill(qr, kr, v, hq, hkv, d, T, heads=(h, h + 1),
                                        rows=(r0, r1, rs))
            err = rel_err(out[blk, r0:r1:rs], ref[blk, r0:r1:rs])
            print(f"c4 head {h} rows {r0}:{r1}:{rs} rel err {err:.3e}")
            assert err < TOL_LOWP
    assert np.array_equal(from_dev(vc), v)
    assert rel_err(from_dev(kc), kr) < 2 ** -7


@pytest.mark.parametrize("dt", [1, 2])
def test_prefill_lowp_output_is_rne_of_fp32_output(hl, orc, dt):
    """fp16/bf16 output = round-to-nearest-even of the fp32 output, bit for bit."""
    hq, hkv, d, T = 8, 2, 128, 130
    q, k, v = (orc.upcast(orc.to_storage(orc.normal(h * d * T, 70 + i), dt), dt).reshape(-1, T)
               for i, h in enumerate((hq, hkv, hkv)))
    args = (to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T)
    o32 = run_prefill(*args, apply_rope=True, rope_base=5e5)
    olp = run_prefill(*args, out_dtype=TDT[dt], apply_rope=True, rope_base=5e5)
    exp = orc.to_storage(from_dev(o32), dt)
    assert np.array_equal(olp.view(torch.int16).cpu().numpy().view(np.uint16), exp)


@pytest.mark.parametrize("d", [64, 128])
def test_prefill_fp32_split_path_graph_replays(hl, orc, d):
    """The fp32 prefill captured once and replayed on three inputs copied into
    the same buffers (plain; a 1e5 outlier in a K tile; a NaN in a V tile, so
    the split images' flags switch steps to the fp32 MFMAs and back): each
    replay reproduces its eager result bit for bit, with the eager runs of
    the other inputs in between."""
    from hippo_leap_amd import attention as A
    hq, hkv, T = 8, 2, 200
    base = [orc.normal(h * d * T, 90 + i).reshape(h * d, T) for i, h in enumerate((hq, hkv, hkv))]
    outl = [x.copy() for x in base]
    outl[1][3, 70:75] = 1e5
    nan = [x.copy() for x in base]
    nan[2][d + 5, 150] = np.nan
    inputs = {"plain": base, "outlier": outl, "nan": nan}
    qd, kd, vd = (to_dev(x, 0) for x in base)
    out = torch.empty(hq * d, T, device="cuda")
    a = A.prefill_args(qd, kd, vd, out, hq, hkv, d, T, apply_rope=True, rope_base=1e4)
    ws = A.workspace(A.prefill_workspace_bytes(a))
    eager = {}
    for name, src in inputs.items():
        for dst, x in zip((qd, kd, vd), src):
            dst.copy_(to_dev(x, 0))
        A.attn_prefill(a, ws)
        torch.cuda.synchronize()
        eager[name] = from_dev(out).copy()
    with np.errstate(invalid="ignore"):
        ref, _, _ = oracle_prefill(orc, *base, hq, hkv, d, T, base=1e4)
    assert rel_err(eager["plain"], ref) < TOL_F32 / 10
    assert np.isnan(eager["nan"]).any() and not np.isnan(eager["outlier"]).any()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.attn_prefill(a, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        A.attn_prefill(a, ws)
    for name in ("nan", "plain", "outlier", "nan", "plain"):
        for dst, x in zip((qd, kd, vd), inputs[name]):
            dst.copy_(to_dev(x, 0))
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out), eager[name], equal_nan=True), name
