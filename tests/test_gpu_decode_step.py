"""GPU parity: the fused decode step (hl_decode_step) against the two-call
sequence it replaces (hl_rope_store_decode then hl_attn_decode) and against
the CPU oracle (qkNorm -> RoPE -> cache store -> attention,
naive.nim:4697-4700, 3149-3223, 3369-3383).

Bars: cache columns identical to the two-call path, bit for bit; outputs
within 1e-5 relative of it (the fused kernel scores the new column with an
fp32 dot product, the attention kernel with the split hi/lo MFMA, which
carries about 16 significant bits of q for bf16 KV; with fp32 KV the step
runs the same two kernels and matches exactly);
outputs within 1e-4 (fp32 KV) / 2e-3 (fp16/bf16 KV) relative of the oracle."""
import numpy as np
import pytest
import torch

from util import TOL_F32, TOL_LOWP, rel_err
from test_gpu_decode import TDT, dev_bits, make_case

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def cache_bits(t, dt):
    return t.cpu().numpy() if dt == 0 else t.view(torch.int16).cpu().numpy().view(np.uint16)


def run_both(orc, B, hq, hkv, d, max_len, dt, positions, rope_dim, style, norm, splits, seed):
    """Returns (step out, step caches, two-call out, two-call caches, inputs)."""
    from hippo_leap_amd import attention as A
    q, kb, vb = make_case(orc, B, hq, hkv, d, max_len, max_len, dt, seed)
    qa = orc.normal(B * hq * d, seed + 3)
    ka = orc.normal(B * hkv * d, seed + 4)
    va = orc.normal(B * hkv * d, seed + 5)
    wq = orc.uniform(d, seed + 6, 0.5, 1.5) if norm else None
    wk = orc.uniform(d, seed + 7, 0.5, 1.5) if norm else None
    pos_t = torch.tensor(positions, dtype=torch.int32, device="cuda") if len(positions) > 1 else None
    pos0 = positions[0]
    L = max(positions) + 1
    base = 5e5
    outs = []
    for fused in (True, False):
        qd, kd, vd = dev(qa), dev(ka), dev(va)
        kc, vc = dev_bits(kb, dt), dev_bits(vb, dt)
        out = torch.full((B * hq * d,), float("nan"), device="cuda")
        rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, max_len, pos0, base,
                               rope_dim=rope_dim, rope_style=style, positions=pos_t,
                               q_norm_w=dev(wq) if norm else None,
                               k_norm_w=dev(wk) if norm else None, eps=1e-6)
        if fused:
            at = A.decode_args(qd, kc, vc, out, hq, hkv, d, max_len, L, num_splits=splits)
            A.decode_step(rs, at, A.decode_step_workspace(rs, at))
        else:
            lens = (pos_t + 1) if pos_t is not None else None
            at = A.decode_args(qd, kc, vc, out, hq, hkv, d, max_len, L, seq_lens=lens,
                               num_splits=splits)
            A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, max_len, pos0, base,
                                rope_dim=rope_dim, rope_style=style, positions=pos_t,
                                q_norm_w=dev(wq) if norm else None,
                                k_norm_w=dev(wk) if norm else None, eps=1e-6)
            A.attn_decode(at, A.decode_workspace(at))
        torch.cuda.synchronize()
        outs.append((out.cpu().numpy(), cache_bits(kc, dt), cache_bits(vc, dt)))
    return outs, (q, kb, vb, qa, ka, va, wq, wk, base)


def oracle_step(orc, B, hq, hkv, d, max_len, dt, positions, rope_dim, style, inputs):
    _, kb, vb, qa, ka, va, wq, wk, base = inputs
    rd = rope_dim or d
    th = orc.theta_table(rd, base)
    per = hkv * d * max_len
    out = np.empty(B * hq * d, np.float32)
    for b in range(B):
        p = positions[b] if len(positions) > 1 else positions[0]
        qb = qa[b * hq * d:(b + 1) * hq * d]
        kbv = ka[b * hkv * d:(b + 1) * hkv * d]
        if wq is not None:
            qb = orc.qk_norm(qb, wq, hq, d, 1e-6)
            kbv = orc.qk_norm(kbv, wk, hkv, d, 1e-6)
        qb = orc.rope_heads(qb, hq, d, rd, th, p, style)
        kbv = orc.rope_heads(kbv, hkv, d, rd, th, p, style)
        kc = orc.upcast(kb[b * per:(b + 1) * per], dt).reshape(hkv * d, max_len).copy()
        vc = orc.upcast(vb[b * per:(b + 1) * per], dt).reshape(hkv * d, max_len).copy()
        kc[:, p] = orc.upcast(orc.to_storage(kbv, dt), dt)
        vc[:, p] = orc.upcast(orc.to_storage(va[b * hkv * d:(b + 1) * hkv * d], dt), dt)
        out[b * hq * d:(b + 1) * hq * d] = orc.attention_decode(qb, kc.reshape(-1), vc.reshape(-1),
                                                                hq, hkv, d, p + 1, max_len)
    return out


CASES = [
    # B, hq, hkv, d, max_len, positions, rope_dim, style, norm, splits
    (8, 32, 8, 64, 2112, [2048], 0, 0, False, 8),          # the c3 step shape
    (3, 32, 4, 128, 960, [0, 500, 959], 0, 0, True, 4),    # ragged, qkNorm, first/last column
    (2, 40, 2, 64, 512, [31, 32], 32, 1, False, 0),        # G=20: two head chunks, partial interleaved rope
    (1, 16, 16, 128, 4096, [4095], 64, 0, True, 0),        # G=1, long, partial half-split rope
    (2, 8, 2, 64, 256, [63, 64], 0, 0, True, 3),           # new column on a tile edge
    (3, 16, 4, 64, 257, [5, 200, 256], 0, 0, True, 0),     # odd max_len: element-wise loads
    (2, 24, 3, 128, 131, [130, 64], 0, 1, False, 2),       # odd max_len, D128, interleaved
]


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_decode_step_matches_two_calls_and_oracle(hl, orc, dt, case):
    B, hq, hkv, d, max_len, positions, rope_dim, style, norm, splits = CASES[case]
    print(f"decode_step case {case} dt {dt}", flush=True)
    outs, inputs = run_both(orc, B, hq, hkv, d, max_len, dt, positions, rope_dim, style, norm,
                            splits, 1300 + 10 * case)
    (fo, fk, fv), (so, sk, sv) = outs
    assert np.array_equal(fk, sk) and np.array_equal(fv, sv)
    if dt == 0 and splits:
        assert np.array_equal(fo, so)
    else:
        assert rel_err(fo, so) < 1e-5
    ref = oracle_step(orc, B, hq, hkv, d, max_len, dt, positions, rope_dim, style, inputs)
    assert rel_err(fo, ref) < (TOL_F32 if dt == 0 else TOL_LOWP)


SEED_CASES = [
    # B, hq, hkv, d, max_len, positions, splits: the split holding the new
    # column seeds its softmax state with it, so the whole column (written to
    # LDS by every wave) must be visible to the seeding wave
    (2, 24, 3, 128, 160, [31, 32], 1),    # one split, new column last / first of a tile
    (2, 32, 8, 64, 128, [31, 95], 1),
    (3, 32, 4, 128, 256, [31, 127, 200], 0),
]


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("case", range(len(SEED_CASES)))
def test_decode_step_new_column_seed_repeated(hl, orc, dt, case):
    """Regression guard: the fused step matches the two-call path on every
    one of eight repetitions.  A missing barrier before the seeding once let
    the seeding wave read new-column entries the other waves had not written
    yet; the timing-dependent failure showed in the fp8 tiled step case of
    test_gpu_kv_fp8.py (one split, D = 128, new column last in its tile)."""
    B, hq, hkv, d, max_len, positions, splits = SEED_CASES[case]
    print(f"decode_step seed case {case} dt {dt}", flush=True)
    for rep in range(8):
        outs, _ = run_both(orc, B, hq, hkv, d, max_len, dt, positions, 0, 0, False, splits,
                           1500 + 10 * case + rep)
        (fo, fk, fv), (so, sk, sv) = outs
        assert np.array_equal(fk, sk) and np.array_equal(fv, sv)
        assert rel_err(fo, so) < 1e-5, f"repetition {rep}"


def test_decode_step_graph_replay(hl, orc):
    """The step in a HIP graph: replays with eager work in between give the
    eager result every time (the cache column is rewritten with the same bits)."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, dt = 4, 32, 8, 64, 1024, 1
    q, kb, vb = make_case(orc, B, hq, hkv, d, M, M, dt, 1400)
    qd = dev(orc.normal(B * hq * d, 1401))
    kd, vd = dev(orc.normal(B * hkv * d, 1402)), dev(orc.normal(B * hkv * d, 1403))
    kc, vc = dev_bits(kb, dt), dev_bits(vb, dt)
    out = torch.empty(B * hq * d, device="cuda")
    rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, 700, 5e5)
    at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, 701)
    ws = A.decode_step_workspace(rs, at)
    A.decode_step(rs, at, ws)
    torch.cuda.synchronize()
    eager = out.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.decode_step(rs, at, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        A.decode_step(rs, at, ws)
    for _ in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), eager)


@pytest.mark.parametrize("layout", [0, 1])
def test_decode_step_c5_full_shape(hl, orc, layout):
    """Config 5's fused step at full size, as bench.py times it: B=16,
    Hq32/Hkv4, D128, bf16 caches, qkNorm (w ~ U(0.5, 1.5) seeded, eps 1e-6)
    then RoPE theta 1e6 at position 32768 (angles up to 3.3e4 rad), the cache
    write, then attention over 32769 columns (naive.nim:2887-2926, 3046-3086,
    3149-3223, 3292-3383).  Column-major (max_len 32769) and tiled (32800)
    caches.  The oracle checks sequences 0 and 15 in full: the written
    column within one bf16 ulp of the oracle's rounded value (the device
    and glibc sincosf differ by a few fp32 ulps, which can move an RNE
    rounding by one step) and the outputs within 2e-3.  Every sequence's
    written column equals the two-call path's bit for bit."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, pos, dt = 16, 32, 4, 128, 32768, 2
    M = 32769 if layout == 0 else 32800
    print(f"c5 full step layout {layout}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(3100 + layout)
    per = hkv * d * M
    kc0 = torch.randn(B * per, generator=gen, device="cuda").to(torch.bfloat16)
    vc0 = torch.randn(B * per, generator=gen, device="cuda").to(torch.bfloat16)
    host_k = {b: kc0[b * per:(b + 1) * per].view(torch.int16).cpu().numpy().view(np.uint16)
              for b in (0, B - 1)}
    host_v = {b: vc0[b * per:(b + 1) * per].view(torch.int16).cpu().numpy().view(np.uint16)
              for b in (0, B - 1)}
    qa, ka, va = orc.normal(B * hq * d, 3101), orc.normal(B * hkv * d, 3102), orc.normal(B * hkv * d, 3103)
    wq, wk = orc.uniform(d, 3104, 0.5, 1.5), orc.uniform(d, 3105, 0.5, 1.5)
    base = 1e6

    def new_column(cache):
        c = cache if layout == 0 else A.kv_from_tiled(cache, hkv, d, M)
        return c.view(B, hkv * d, M)[:, :, pos].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    results = []
    for fused in (True, False):
        kc = kc0.clone() if layout == 0 else A.kv_to_tiled(kc0, hkv, d, M)
        vc = vc0.clone() if layout == 0 else A.kv_to_tiled(vc0, hkv, d, M)
        qd, kd, vd = dev(qa), dev(ka), dev(va)
        out = torch.full((B * hq * d,), float("nan"), device="cuda")
        rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, pos, base,
                               q_norm_w=dev(wq), k_norm_w=dev(wk), eps=1e-6, kv_layout=layout)
        at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, pos + 1, kv_layout=layout)
        if fused:
            A.decode_step(rs, at, A.decode_step_workspace(rs, at))
        else:
            A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, M, pos, base,
                                q_norm_w=dev(wq), k_norm_w=dev(wk), eps=1e-6, kv_layout=layout)
            A.attn_decode(at, A.decode_workspace(at))
        torch.cuda.synchronize()
        results.append((out.cpu().numpy(), new_column(kc), new_column(vc)))
        del kc, vc
    (fo, fk, fv), (so, sk, sv) = results
    assert np.array_equal(fk, sk) and np.array_equal(fv, sv)
    assert rel_err(fo, so) < 1e-5

    th = orc.theta_table(d, base)
    for b in (0, B - 1):
        qb = orc.rope_heads(orc.qk_norm(qa[b * hq * d:(b + 1) * hq * d], wq, hq, d, 1e-6),
                            hq, d, d, th, pos)
        kb = orc.rope_heads(orc.qk_norm(ka[b * hkv * d:(b + 1) * hkv * d], wk, hkv, d, 1e-6),
                            hkv, d, d, th, pos)
        kcol = orc.to_storage(kb, dt)
        vcol = orc.to_storage(va[b * hkv * d:(b + 1) * hkv * d], dt)
        assert np.array_equal(fv[b], vcol)
        ulps = np.abs(fk[b].astype(np.int32) - kcol.astype(np.int32))
        assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01, f"seq {b}: k column off by {ulps.max()} ulp"
        kf = orc.upcast(host_k[b], dt).reshape(hkv * d, M).copy()
        vf = orc.upcast(host_v[b], dt).reshape(hkv * d, M).copy()
        kf[:, pos] = orc.upcast(kcol, dt)
        vf[:, pos] = orc.upcast(vcol, dt)
        ref = orc.attention_decode(qb, kf.reshape(-1), vf.reshape(-1), hq, hkv, d, pos + 1, M)
        err = rel_err(fo[b * hq * d:(b + 1) * hq * d], ref)
        print(f"c5 step layout {layout} seq {b} rel err {err:.3e}", flush=True)
        assert err < TOL_LOWP
