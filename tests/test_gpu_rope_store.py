"""GPU parity: qkNorm, RoPE and KV-cache store kernels, through both the
reference-signature drop-ins and the fused batched entry point."""
import numpy as np
import pytest
import torch

from util import golden, rel_err

pytestmark = pytest.mark.gpu

TDT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}
ROPE_TOL = 2e-6  # device cosf/sinf vs glibc: a few ulps on |x| ~ 1 values


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


def host(t):
    return t.float().cpu().numpy()


def bits_of(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_qk_norm_dropins(hl, orc):
    from hippo_leap_amd import attention as A
    H, D, T, eps = 8, 128, 37, 1e-6
    w = orc.uniform(D, 1, 0.5, 1.5)
    x = orc.normal(H * D, 2, 0, 3)
    xd = dev(x)
    A.gpu_qk_norm(xd, dev(w), H, D, eps)
    torch.cuda.synchronize()
    assert rel_err(host(xd), orc.qk_norm(x, w, H, D, eps)) < 1e-6
    xc = orc.normal(H * D * T, 3).reshape(H * D, T)
    xcd = dev(xc)
    A.gpu_qk_norm_prefill(xcd, dev(w), H, D, T, eps)
    torch.cuda.synchronize()
    assert rel_err(host(xcd), orc.qk_norm_cols(xc, w, H, D, T, eps)) < 1e-6


@pytest.mark.parametrize("rd", [64, 32])
def test_rope_dropins(hl, orc, rd):
    from hippo_leap_amd import attention as A
    H, D, T, base = 4, 64, 45, 1e4
    th = orc.theta_table(rd, base)
    x = orc.normal(H * D, 4)
    xd = dev(x)
    A.gpu_rope_at_pos(xd, H, D, rd, base, 123, 1)
    torch.cuda.synchronize()
    assert rel_err(host(xd), orc.rope_heads(x, H, D, rd, th, 123)) < ROPE_TOL
    xc = orc.normal(H * D * T, 5).reshape(H * D, T)
    xcd = dev(xc)
    A.gpu_rope_at_pos(xcd, H, D, rd, base, 999, T)  # prefill: column p at position p
    torch.cuda.synchronize()
    assert rel_err(host(xcd), orc.rope_cols(xc, H, D, T, rd, th, 0)) < ROPE_TOL
    A.set_rope_theta(rd, base)
    xcd = dev(xc)
    A.gpu_rope_at_pos_theta(xcd, H, D, rd, 50, T)  # column p at position 50 + p
    torch.cuda.synchronize()
    assert rel_err(host(xcd), orc.rope_cols(xc, H, D, T, rd, th, 50)) < ROPE_TOL
    q, k = orc.normal(H * D, 6), orc.normal(2 * D, 7)
    qd, kd = dev(q), dev(k)
    A.gpu_rope_qk_decode(qd, kd, H, 2, D, rd, base, 77)
    torch.cuda.synchronize()
    assert rel_err(host(qd), orc.rope_heads(q, H, D, rd, th, 77)) < ROPE_TOL
    assert rel_err(host(kd), orc.rope_heads(k, 2, D, rd, th, 77)) < ROPE_TOL


def test_fused_rope_store_kv_dropin(hl, orc):
    from hippo_leap_amd import attention as A
    hq, hkv, D, rd, M, pos, base = 32, 4, 64, 64, 512, 300, 1e4
    A.set_rope_theta(rd, base)
    th = orc.theta_table(rd, base)
    q, k, v = orc.normal(hq * D, 8), orc.normal(hkv * D, 9), orc.normal(hkv * D, 10)
    kc = torch.full((hkv * D, M), 3.0, device="cuda")
    vc = torch.full((hkv * D, M), 3.0, device="cuda")
    qd, kd, vd = dev(q), dev(k), dev(v)
    A.gpu_fused_rope_store_kv(qd, kd, vd, kc, vc, hq, hkv, D, rd, hkv * D, M, pos)
    torch.cuda.synchronize()
    kr = orc.rope_heads(k, hkv, D, rd, th, pos)
    assert rel_err(host(qd), orc.rope_heads(q, hq, D, rd, th, pos)) < ROPE_TOL
    assert rel_err(host(kd), kr) < ROPE_TOL
    kcn, vcn = host(kc), host(vc)
    assert np.array_equal(kcn[:, pos], host(kd))  # cache holds the rotated k, bit for bit
    assert np.array_equal(vcn[:, pos], v)
    mask = np.ones(M, bool)
    mask[pos] = False
    assert np.all(kcn[:, mask] == 3.0) and np.all(vcn[:, mask] == 3.0)


def test_store_kv_dropins(hl, orc):
    from hippo_leap_amd import attention as A
    rows, cols, M, start = 256, 37, 100, 20
    src, src2 = orc.normal(rows * cols, 11), orc.normal(rows * cols, 12)
    c = torch.zeros(rows, M, device="cuda")
    A.gpu_store_kv(c, dev(src), rows, cols, M, start)
    torch.cuda.synchronize()
    ref = np.zeros((rows, M), np.float32)
    orc.store_kv(ref, 0, src, rows, cols, M, start)
    assert np.array_equal(host(c), ref)
    c1, c2 = torch.zeros(rows, M, device="cuda"), torch.zeros(rows, M, device="cuda")
    A.gpu_store_kv_pair(c1, dev(src), c2, dev(src2), rows, cols, M, start)
    torch.cuda.synchronize()
    ref2 = np.zeros((rows, M), np.float32)
    orc.store_kv(ref2, 0, src2, rows, cols, M, start)
    assert np.array_equal(host(c1), ref) and np.array_equal(host(c2), ref2)


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("style", [0, 1])
def test_rope_store_decode_batched(hl, orc, dt, style):
    from hippo_leap_amd import attention as A
    B, hq, hkv, D, M, base, eps = 3, 16, 4, 128, 64, 1e6, 1e-6
    positions = np.array([0, 31, 63], np.int32)
    th = orc.theta_table(D, base)
    q, k, v = orc.normal(B * hq * D, 13), orc.normal(B * hkv * D, 14), orc.normal(B * hkv * D, 15)
    wq, wk = orc.uniform(D, 16, 0.5, 1.5), orc.uniform(D, 17, 0.5, 1.5)
    kc = torch.zeros(B * hkv * D * M, dtype=TDT[dt], device="cuda")
    vc = torch.zeros(B * hkv * D * M, dtype=TDT[dt], device="cuda")
    qd, kd, vd = dev(q), dev(k), dev(v)
    A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, D, M, 0, base, rope_style=style,
                        positions=torch.from_numpy(positions).cuda(), q_norm_w=dev(wq),
                        k_norm_w=dev(wk), eps=eps)
    torch.cuda.synchronize()
    kc_h = (host(kc) if dt == 0 else bits_of(kc)).reshape(B, hkv * D, M)
    vc_h = (host(vc) if dt == 0 else bits_of(vc)).reshape(B, hkv * D, M)
    for b in range(B):
        p = int(positions[b])
        qb = orc.rope_heads(orc.qk_norm(q[b * hq * D:(b + 1) * hq * D], wq, hq, D, eps), hq, D, D,
                            th, p, style)
        kb = orc.rope_heads(orc.qk_norm(k[b * hkv * D:(b + 1) * hkv * D], wk, hkv, D, eps), hkv, D,
                            D, th, p, style)
        assert rel_err(host(qd)[b * hq * D:(b + 1) * hq * D], qb) < ROPE_TOL * 4
        kgpu = host(kd)[b * hkv * D:(b + 1) * hkv * D]
        assert rel_err(kgpu, kb) < ROPE_TOL * 4
        # the cache column is the RNE conversion of the kernel's own rotated k, exactly
        assert np.array_equal(kc_h[b][:, p], orc.to_storage(kgpu, dt))
        assert np.array_equal(vc_h[b][:, p], orc.to_storage(v[b * hkv * D:(b + 1) * hkv * D], dt))
        others = np.delete(np.arange(M), p)
        assert np.all(kc_h[b][:, others] == 0) and np.all(vc_h[b][:, others] == 0)


@pytest.mark.parametrize("name", ["decode_step_bf16_qknorm", "decode_step_f16_qknorm"])
def test_decode_step_golden(hl, orc, name):
    """qkNorm -> RoPE -> store -> attention, one new token (config-5 style)."""
    from hippo_leap_amd import attention as A
    from test_gpu_decode import dev_bits
    g = golden(name)
    hq, hkv, d, prev, M, dt = (int(v) for v in g["shape"])
    qd, kd, vd = dev(g["q"]), dev(g["k"]), dev(g["v"])
    kc, vc = dev_bits(g["k_cache"], dt), dev_bits(g["v_cache"], dt)
    A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, M, prev, float(g["base"][0]),
                        q_norm_w=dev(g["wq"]), k_norm_w=dev(g["wk"]), eps=float(g["eps"][0]))
    out = torch.empty(hq * d, device="cuda")
    a = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, prev + 1)
    A.attn_decode(a, A.decode_workspace(a))
    torch.cuda.synchronize()
    assert rel_err(host(out), g["expected"]) < 2e-4


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_kv_cache_to_f32_kat(hl, orc, dt):
    """Device decode of stored bits; fp16 includes the reference halfToFloat KAT
    (tests/test_quant.nim:5-15): 0x0000, 0x3C00, 0xBC00, 0x4000, 0x3800, +-Inf, NaN."""
    from hippo_leap_amd import attention as A
    if dt == 1:
        bits = np.array([0x0000, 0x3C00, 0xBC00, 0x4000, 0x3800, 0x7C00, 0xFC00, 0x7C01] +
                        list(range(0, 65536, 97)), np.uint16)
    elif dt == 2:
        bits = np.arange(0, 65536, 13, dtype=np.uint16)
    else:
        bits = orc.normal(4096, 18)
    from test_gpu_decode import dev_bits
    n = bits.size
    out = host(A.kv_cache_to_f32(dev_bits(bits, dt), 1, n, 0, n))[0]
    ref = orc.upcast(bits, dt)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan], ref[~nan])
    if dt == 1:
        assert list(out[:7]) == [0.0, 1.0, -1.0, 2.0, 0.5, np.inf, -np.inf] and np.isnan(out[7])


@pytest.mark.parametrize("pos", [8191, 32768, 131071])
def test_rope_dropins_large_positions(hl, orc, pos):
    """RoPE at long-context positions (angles up to 1.3e5 rad, where the
    argument reduction of sincosf matters), theta 1e6 and 5e5, against the
    oracle's glibc cosf/sinf of the same fp32 angle.  The theta table is
    installed first: hl_gpu_rope_qk_decode then uses it and ignores its
    rope_base argument, as ropeQKDecodeKernel does (naive.nim:3046-3086)."""
    from hippo_leap_amd import attention as A
    H, D = 8, 128
    for base in (1e6, 5e5):
        th = orc.theta_table(D, base)
        A.set_rope_theta(D, base)
        q, k = orc.normal(H * D, 40 + pos % 7), orc.normal(2 * D, 41 + pos % 5)
        qd, kd = dev(q), dev(k)
        A.gpu_rope_qk_decode(qd, kd, H, 2, D, D, base, pos)
        torch.cuda.synchronize()
        assert rel_err(host(qd), orc.rope_heads(q, H, D, D, th, pos)) < ROPE_TOL
        assert rel_err(host(kd), orc.rope_heads(k, 2, D, D, th, pos)) < ROPE_TOL
        xd = dev(q)
        A.gpu_rope_at_pos(xd, H, D, D, base, pos, 1)
        torch.cuda.synchronize()
        assert rel_err(host(xd), orc.rope_heads(q, H, D, D, th, pos)) < ROPE_TOL
        T = 16
        xc = orc.normal(H * D * T, 42).reshape(H * D, T)
        xcd = dev(xc)
        A.gpu_rope_at_pos_theta(xcd, H, D, D, pos - T, T)  # columns at pos-16 .. pos-1
        torch.cuda.synchronize()
        assert rel_err(host(xcd), orc.rope_cols(xc, H, D, T, D, th, pos - T)) < ROPE_TOL
