"""GPU parity: split-K decode attention (hl_attn_decode / hl_gpu_attention_decode)
against the CPU oracle on the same seeded inputs and stored bits.

Bars: 1e-4 relative for fp32 KV, 2e-3 for fp16/bf16 (north star), metric
max|gpu - ref| / max|ref| per output tensor.
"""
import numpy as np
import pytest
import torch

from util import TOL_F32, TOL_LOWP, golden, rel_err

pytestmark = pytest.mark.gpu

TDT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def dev_bits(bits, dt):
    """Stored host bits -> device tensor of the storage dtype."""
    if dt == 0:
        return torch.from_numpy(np.ascontiguousarray(bits, np.float32)).cuda()
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).cuda().view(TDT[dt])


def run_decode(q, kc, vc, B, hq, hkv, d, L, max_len, seq_lens=None, num_splits=0, stride=0):
    from hippo_leap_amd import attention as A
    out = torch.full((B * hq * d,), float("nan"), device="cuda")
    a = A.decode_args(q, kc, vc, out, hq, hkv, d, max_len, L, seq_lens=seq_lens,
                      cache_batch_stride=stride, num_splits=num_splits)
    ws = A.decode_workspace(a)
    A.attn_decode(a, ws)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def make_case(orc, B, hq, hkv, d, L, max_len, dt, seed, dist="uniform"):
    n = B * hkv * d * max_len
    gen = orc.uniform if dist == "uniform" else orc.normal
    q = gen(B * hq * d, seed)
    kb = orc.to_storage(gen(n, seed + 1), dt)
    vb = orc.to_storage(gen(n, seed + 2), dt)
    return q, kb, vb


def oracle_decode(orc, q, kb, vb, B, hq, hkv, d, lens, max_len, dt, seqs=None):
    per = hkv * d * max_len
    out = np.full(B * hq * d, np.nan, np.float32)
    for b in (range(B) if seqs is None else seqs):
        kc = orc.upcast(kb[b * per:(b + 1) * per], dt)
        vc = orc.upcast(vb[b * per:(b + 1) * per], dt)
        out[b * hq * d:(b + 1) * hq * d] = orc.attention_decode(
            q[b * hq * d:(b + 1) * hq * d], kc, vc, hq, hkv, d, lens[b], max_len)
    return out


@pytest.mark.parametrize("name", ["decode_f32", "decode_f16", "decode_bf16"])
def test_decode_golden(hl, name):
    g = golden(name)
    hq, hkv, d, L, max_len, dt = (int(v) for v in g["shape"])
    out = run_decode(torch.from_numpy(g["q"]).cuda(), dev_bits(g["k_cache"], dt),
                     dev_bits(g["v_cache"], dt), 1, hq, hkv, d, L, max_len)
    assert rel_err(out, g["expected"]) < (TOL_F32 if dt == 0 else TOL_LOWP) / 10


def test_decode_c1_reference_dropin(hl, orc):
    """Config 1: TinyLlama shape through the gpuAttentionDecode signature."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, L, max_len = 32, 4, 64, 512, 512
    q, kb, vb = make_case(orc, 1, hq, hkv, d, L, max_len, 0, 101)
    ref = orc.attention_decode(q, kb, vb, hq, hkv, d, L, max_len)
    dst = torch.empty(hq * d, device="cuda")
    A.gpu_attention_decode(dst, torch.from_numpy(q).cuda(), torch.from_numpy(kb).cuda(),
                           torch.from_numpy(vb).cuda(), hq, hkv, d, L, max_len)
    torch.cuda.synchronize()
    err = rel_err(dst.cpu().numpy(), ref)
    print(f"c1 rel err {err:.3e}")
    assert err < TOL_F32


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("L", [1, 2, 31, 32, 33, 127, 128, 129, 255, 256, 257, 1000])
def test_decode_lengths(hl, orc, dt, L):
    B, hq, hkv, d, max_len = 2, 8, 2, 64, 1024
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, max_len, dt, 200 + L)
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, max_len, dt)
    out = run_decode(torch.from_numpy(q).cuda(), dev_bits(kb, dt), dev_bits(vb, dt), B, hq, hkv,
                     d, L, max_len)
    assert rel_err(out, ref) < (TOL_F32 if dt == 0 else TOL_LOWP)


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 64), (32, 4, 128), (16, 16, 128), (40, 2, 64),
                                      (8, 8, 64)])
def test_decode_shapes(hl, orc, dt, hq, hkv, d):
    B, L, max_len = 3, 777, 800
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, max_len, dt, 300 + hq + d, "normal")
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, max_len, dt)
    out = run_decode(torch.from_numpy(q).cuda(), dev_bits(kb, dt), dev_bits(vb, dt), B, hq, hkv,
                     d, L, max_len)
    assert rel_err(out, ref) < (TOL_F32 if dt == 0 else TOL_LOWP)


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_decode_split_invariance(hl, orc, dt):
    """Any split count gives the same result within fp32 rounding."""
    B, hq, hkv, d, L, max_len = 2, 16, 4, 128, 1500, 1536
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, max_len, dt, 400)
    qd, kd, vd = torch.from_numpy(q).cuda(), dev_bits(kb, dt), dev_bits(vb, dt)
    base = run_decode(qd, kd, vd, B, hq, hkv, d, L, max_len, num_splits=1)
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, max_len, dt)
    assert rel_err(base, ref) < (TOL_F32 if dt == 0 else TOL_LOWP)
    for ns in (2, 3, 7, 12):
        assert rel_err(run_decode(qd, kd, vd, B, hq, hkv, d, L, max_len, num_splits=ns), base) < 1e-5


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_decode_ragged_lengths_and_stride(hl, orc, dt):
    """Per-sequence lengths (device array) and a padded batch stride."""
    B, hq, hkv, d, max_len = 4, 16, 4, 64, 600
    lens = [600, 1, 333, 129]
    per = hkv * d * max_len
    stride = per + 64
    q, kb, vb = make_case(orc, B, hq, hkv, d, max_len, max_len, dt, 500)
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, lens, max_len, dt)
    # lay the caches out with the padded stride; the pad holds NaN/garbage bits
    def strided(bits):
        if dt == 0:
            buf = np.full(B * stride, np.nan, np.float32)
        else:
            buf = np.full(B * stride, 0x7E00, np.uint16)
        for b in range(B):
            buf[b * stride:b * stride + per] = bits[b * per:(b + 1) * per]
        return buf
    sl = torch.tensor(lens, dtype=torch.int32, device="cuda")
    out = run_decode(torch.from_numpy(q).cuda(), dev_bits(strided(kb), dt),
                     dev_bits(strided(vb), dt), B, hq, hkv, d, max(lens), max_len, seq_lens=sl,
                     stride=stride)
    assert rel_err(out, ref) < (TOL_F32 if dt == 0 else TOL_LOWP)


@pytest.mark.parametrize("dt", [1, 2])
def test_decode_nan_beyond_length_is_ignored(hl, orc, dt):
    """Cache columns >= L hold NaN bits: the masked tail must not leak."""
    B, hq, hkv, d, L, max_len = 1, 8, 2, 128, 70, 96
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, max_len, dt, 600)
    kb2, vb2 = kb.reshape(hkv * d, max_len).copy(), vb.reshape(hkv * d, max_len).copy()
    kb2[:, L:] = 0x7E00
    vb2[:, L:] = 0x7E00
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L], max_len, dt)
    out = run_decode(torch.from_numpy(q).cuda(), dev_bits(kb2.reshape(-1), dt),
                     dev_bits(vb2.reshape(-1), dt), B, hq, hkv, d, L, max_len)
    assert rel_err(out, ref) < TOL_LOWP


def test_decode_c3_full_size(hl, orc):
    """Config 3 at full size: B=8, Hq32/Hkv8, D64, L=2049, fp16 KV ~ N(0, 0.5)."""
    B, hq, hkv, d, L, max_len, dt = 8, 32, 8, 64, 2049, 2049, 1
    q = orc.normal(B * hq * d, 700, 0, 0.5)
    n = B * hkv * d * max_len
    kb = orc.to_storage(orc.normal(n, 701, 0, 0.5), dt)
    vb = orc.to_storage(orc.normal(n, 702, 0, 0.5), dt)
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, max_len, dt)
    out = run_decode(torch.from_numpy(q).cuda(), dev_bits(kb, dt), dev_bits(vb, dt), B, hq, hkv,
                     d, L, max_len)
    err = rel_err(out, ref)
    print(f"c3 rel err {err:.3e}")
    assert err < TOL_LOWP


def test_decode_c5_full_size_sampled(hl, orc):
    """Config 5 attention at full size (B=16, L=32769, bf16, D128, G=8); the
    oracle checks sequences 0 and 15, all heads; the rest by split invariance."""
    B, hq, hkv, d, L, max_len, dt = 16, 32, 4, 128, 32769, 32769, 2
    gen = torch.Generator(device="cuda").manual_seed(800)
    kc = torch.randn(B * hkv * d * max_len, generator=gen, device="cuda").to(torch.bfloat16)
    vc = torch.randn(B * hkv * d * max_len, generator=gen, device="cuda").to(torch.bfloat16)
    q = torch.randn(B * hq * d, generator=gen, device="cuda")
    out = run_decode(q, kc, vc, B, hq, hkv, d, L, max_len)
    per = hkv * d * max_len
    for b in (0, B - 1):
        kb = kc[b * per:(b + 1) * per].view(torch.int16).cpu().numpy().view(np.uint16)
        vb = vc[b * per:(b + 1) * per].view(torch.int16).cpu().numpy().view(np.uint16)
        ref = orc.attention_decode(q[b * hq * d:(b + 1) * hq * d].cpu().numpy(),
                                   orc.upcast(kb, dt), orc.upcast(vb, dt), hq, hkv, d, L, max_len)
        err = rel_err(out[b * hq * d:(b + 1) * hq * d], ref)
        print(f"c5 seq {b} rel err {err:.3e}")
        assert err < TOL_LOWP
    out1 = run_decode(q, kc, vc, B, hq, hkv, d, L, max_len, num_splits=5)
    assert rel_err(out1, out) < 1e-5


def test_decode_reference_dropin_matches_batched(hl, orc):
    from hippo_leap_amd import attention as A
    hq, hkv, d, L, max_len = 32, 8, 128, 300, 301
    q, kb, vb = make_case(orc, 1, hq, hkv, d, L, max_len, 0, 900)
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, kb, vb))
    dst = torch.empty(hq * d, device="cuda")
    A.gpu_attention_decode(dst, qd, kd, vd, hq, hkv, d, L, max_len)
    torch.cuda.synchronize()
    assert rel_err(dst.cpu().numpy(), run_decode(qd, kd, vd, 1, hq, hkv, d, L, max_len)) < 1e-6


@pytest.mark.parametrize("dt,hq,hkv,d", [(0, 16, 4, 64), (2, 16, 4, 64), (1, 32, 2, 128)])
def test_decode_workspace_reuse_and_graph_replay(hl, orc, dt, hq, hkv, d):
    """The fused split merge keeps arrival counters in the workspace: after
    hl_attn_decode_workspace_init (the partials may hold garbage) every call
    leaves them zero, so reuse with other split counts and graph replays stay
    correct.  (32, 2, 128): 16 heads x 128 dims per workgroup, so the last
    arrival folds several elements per thread."""
    from hippo_leap_amd import attention as A
    B, L, max_len = 3, 900, 960
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, max_len, dt, 1000)
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, max_len, dt)
    qd, kd, vd = torch.from_numpy(q).cuda(), dev_bits(kb, dt), dev_bits(vb, dt)
    out = torch.full((B * hq * d,), float("nan"), device="cuda")
    args = {ns: A.decode_args(qd, kd, vd, out, hq, hkv, d, max_len, L, num_splits=ns)
            for ns in (5, 11, 0, 16, 2)}
    nbytes = max(A.decode_workspace_bytes(a) for a in args.values())
    ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")
    hl.hl_attn_decode_workspace_init(ws.data_ptr(), nbytes, None)
    torch.cuda.synchronize()
    assert int(ws.sum()) == 0
    tol = TOL_F32 if dt == 0 else TOL_LOWP
    for ns in (5, 11, 0, 16, 2, 5):
        out.fill_(float("nan"))
        A.attn_decode(args[ns], ws)
        torch.cuda.synchronize()
        assert rel_err(out.cpu().numpy(), ref) < tol, ns
        assert int(ws[:B * hkv * 4].count_nonzero()) == 0, ns  # the counters are zero again
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.attn_decode(args[11], ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        A.attn_decode(args[11], ws)
    for _ in range(4):
        out.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert rel_err(out.cpu().numpy(), ref) < tol


def test_decode_dropin_refuses_to_grow_under_capture(hl, orc):
    """hl_gpu_attention_decode owns one workspace per device and grows it
    (hipMalloc + device sync) when a call needs more.  Under stream capture
    that call returns HL_ECAPTURE instead: the capture stays valid, and after
    one eager call of the shape the same call captures and replays."""
    import ctypes
    from hippo_leap_amd import _lib, attention as A
    # 512 query heads over 8 kv heads, D = 128, L = 8192: a split-K workspace
    # of several MB, larger than any other test's drop-in call needs.
    hq, hkv, d, L, max_len = 512, 8, 128, 8192, 8192
    q, kb, vb = make_case(orc, 1, hq, hkv, d, L, max_len, 0, 1200)
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, kb, vb))
    dst = torch.full((hq * d,), float("nan"), device="cuda")
    side = torch.cuda.Stream()
    args = (dst.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hq, hkv, d, L, max_len)
    g = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=side):
        dst.fill_(float("nan"))
        rc = hl.hl_gpu_attention_decode(*args, ctypes.c_void_p(side.cuda_stream))
    assert rc == _lib.HL_ECAPTURE, rc
    assert "capture" in hl.hl_last_error().decode()
    g.replay()  # the capture (the fill alone) is still a valid graph
    torch.cuda.synchronize()
    assert torch.isnan(dst).all()
    A.gpu_attention_decode(dst, qd, kd, vd, hq, hkv, d, L, max_len)  # eager: grows the workspace
    torch.cuda.synchronize()
    ref = dst.cpu().numpy().copy()
    sub = orc.attention_decode(q[:16 * d], kb[:d * max_len], vb[:d * max_len], 16, 1, d, L, max_len)
    assert rel_err(ref[:16 * d], sub) < TOL_F32  # heads 0..15 (kv head 0) against the oracle
    g2 = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g2, stream=side):
        assert hl.hl_gpu_attention_decode(*args, ctypes.c_void_p(side.cuda_stream)) == _lib.HL_OK
    for _ in range(3):
        dst.fill_(float("nan"))
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dst.cpu().numpy(), ref)


def test_decode_dropin_shape_changes_share_library_workspace(hl, orc):
    """The drop-in keeps one library workspace per device: a call with more
    kv heads (a longer arrival-counter region) after calls whose partials
    covered that region must still merge correctly, and so must the small
    shape after it."""
    from hippo_leap_amd import attention as A
    d, L, max_len = 64, 900, 960
    for hq, hkv in ((16, 2), (128, 128), (16, 2), (128, 128)):
        q, kb, vb = make_case(orc, 1, hq, hkv, d, L, max_len, 0, 1100 + hkv)
        dst = torch.full((hq * d,), float("nan"), device="cuda")
        A.gpu_attention_decode(dst, *(torch.from_numpy(x).cuda() for x in (q, kb, vb)), hq, hkv,
                               d, L, max_len)
        torch.cuda.synchronize()
        ref = oracle_decode(orc, q, kb, vb, 1, hq, hkv, d, [L], max_len, 0)
        assert rel_err(dst.cpu().numpy(), ref) < TOL_F32, (hq, hkv)
