"""GPU parity of fp8 (OCP e4m3) KV caches, an extension of the reference
(whose caches are fp32): caches in the tiled layout (HL_KV_TILED32) holding
e4m3 bytes.

- Decode attention against the oracle on the same stored bytes (upcast
  exactly): 2e-3 relative, the fp16/bf16 bar.
- The fused decode step and the stand-alone rope/store write the new column
  as the e4m3 encoding of the values the fp32 path computes, bit for bit,
  and the step's output matches the two-call path and the oracle.
- Prefill writes the e4m3 encoding of the fp32 cache values bit for bit.
- The encoding is pinned against torch's float8_e4m3fn cast in
  tests/test_oracle.py."""
import numpy as np
import pytest
import torch

from util import TOL_LOWP, rel_err
from test_gpu_decode import oracle_decode

pytestmark = pytest.mark.gpu
FP8, TILED = 3, 1


def tiled(t, hkv, d, max_len):
    from hippo_leap_amd import attention as A
    return A.kv_to_tiled(t, hkv, d, max_len)


def untiled(t, hkv, d, max_len):
    from hippo_leap_amd import attention as A
    return A.kv_from_tiled(t, hkv, d, max_len)


def fp8_case(orc, B, hq, hkv, d, max_len, seed, std=1.0):
    n = B * hkv * d * max_len
    q = orc.normal(B * hq * d, seed)
    kb = orc.to_storage(orc.normal(n, seed + 1, 0.0, std), FP8)
    vb = orc.to_storage(orc.normal(n, seed + 2, 0.0, std), FP8)
    return q, kb, vb


DECODE_CASES = [
    # B, hq, hkv, d, max_len, L, splits, ragged
    (8, 32, 8, 64, 2080, 2049, 0, False),    # c3 shape
    (2, 32, 4, 128, 4096, 4000, 0, False),   # c5 family: prefetching kernel
    (3, 16, 2, 128, 512, 500, 3, True),      # ragged lengths, explicit splits
    (1, 8, 8, 64, 64, 33, 1, False),         # one split, partial tile
    (2, 40, 2, 64, 256, 256, 0, False),      # two head chunks
]


@pytest.mark.parametrize("case", range(len(DECODE_CASES)))
def test_decode_fp8_matches_oracle(hl, orc, case):
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, L, splits, ragged = DECODE_CASES[case]
    print(f"decode fp8 case {case}", flush=True)
    q, kb, vb = fp8_case(orc, B, hq, hkv, d, M, 5100 + 10 * case)
    k = tiled(torch.from_numpy(kb).cuda(), hkv, d, M)
    v = tiled(torch.from_numpy(vb).cuda(), hkv, d, M)
    lens = [L - 37 * b for b in range(B)] if ragged else [L] * B
    lt = torch.tensor(lens, dtype=torch.int32, device="cuda") if ragged else None
    out = torch.full((B * hq * d,), float("nan"), device="cuda")
    a = A.decode_args(torch.from_numpy(q).cuda(), k, v, out, hq, hkv, d, M, L, seq_lens=lt,
                      num_splits=splits, kv_layout=TILED)
    assert a.kv_dtype == FP8
    A.attn_decode(a, A.decode_workspace(a))
    torch.cuda.synchronize()
    ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, lens, M, FP8)
    assert rel_err(out.cpu().numpy(), ref) < TOL_LOWP


STEP_CASES = [
    # B, hq, hkv, d, max_len, positions, norm
    (8, 32, 8, 64, 2080, [2048], False),
    (3, 32, 4, 128, 992, [0, 500, 991], True),
    (2, 24, 3, 128, 160, [31, 32], False),
]


@pytest.mark.parametrize("case", range(len(STEP_CASES)))
def test_decode_step_fp8(hl, orc, case):
    """Fused step vs two calls (rope_store + attention) on fp8 caches: same
    cache bytes, outputs within 1e-5; the new column equals the e4m3 encoding
    of the fp32 path's column; the output matches the oracle."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, positions, norm = STEP_CASES[case]
    print(f"step fp8 case {case}", flush=True)
    q, kb, vb = fp8_case(orc, B, hq, hkv, d, M, 5200 + 10 * case)
    qa, ka, va = (orc.normal(B * h * d, 5201 + 10 * case + i) for i, h in enumerate((hq, hkv, hkv)))
    wq = torch.from_numpy(orc.uniform(d, 5205, 0.5, 1.5)).cuda() if norm else None
    wk = torch.from_numpy(orc.uniform(d, 5206, 0.5, 1.5)).cuda() if norm else None
    pos_t = torch.tensor(positions, dtype=torch.int32, device="cuda") if len(positions) > 1 else None
    L = max(positions) + 1
    res = {}
    for mode in ("fused", "two", "f32"):
        if mode == "f32":   # fp32 column-major caches: the exact column values
            kc = torch.from_numpy(orc.upcast(kb, FP8)).cuda()
            vc = torch.from_numpy(orc.upcast(vb, FP8)).cuda()
            lay = 0
        else:
            kc = tiled(torch.from_numpy(kb).cuda(), hkv, d, M)
            vc = tiled(torch.from_numpy(vb).cuda(), hkv, d, M)
            lay = TILED
        qd = torch.from_numpy(qa).cuda()
        kd, vd = torch.from_numpy(ka).cuda(), torch.from_numpy(va).cuda()
        out = torch.full((B * hq * d,), float("nan"), device="cuda")
        kw = dict(rope_dim=0, rope_style=0, positions=pos_t, q_norm_w=wq, k_norm_w=wk)
        if mode == "fused":
            rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5,
                                   kv_layout=lay, **kw)
            at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, L, kv_layout=lay)
            A.decode_step(rs, at, A.decode_step_workspace(rs, at))
        else:
            A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5,
                                kv_layout=lay, **kw)
            if mode == "two":
                lens = (pos_t + 1) if pos_t is not None else None
                at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, L, seq_lens=lens, kv_layout=lay)
                A.attn_decode(at, A.decode_workspace(at))
        torch.cuda.synchronize()
        if lay:
            kc, vc = untiled(kc, hkv, d, M), untiled(vc, hkv, d, M)
        res[mode] = (out.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), qd.cpu().numpy())
    fo, fk, fv, fq = res["fused"]
    so, sk, sv, _ = res["two"]
    _, ck, cv, _ = res["f32"]
    assert np.array_equal(fk, sk) and np.array_equal(fv, sv)
    assert np.array_equal(fk, orc.to_storage(ck, FP8)) and np.array_equal(fv, orc.to_storage(cv, FP8))
    assert rel_err(fo, so) < 1e-5
    # oracle: attention over the fp8 cache written by the step, with the roped q
    # of the two-call path (rope_store writes q back in place)
    qr = res["two"][3]
    lens = [p + 1 for p in positions] * (B if len(positions) == 1 else 1)
    ref = oracle_decode(orc, qr, fk.reshape(-1), fv.reshape(-1), B, hq, hkv, d, lens, M, FP8)
    assert rel_err(fo, ref) < TOL_LOWP


PREFILL_CASES = [
    # hq, hkv, d, T, io dtype, start_pos, rope style
    (32, 8, 128, 300, torch.bfloat16, 0, 0),   # K/V prologue kernel (c4 family)
    (16, 4, 128, 150, torch.float16, 5, 1),    # start_pos % 8 != 0
    (16, 2, 64, 100, torch.bfloat16, 40, 0),   # general prologue
    (8, 2, 64, 77, torch.float32, 3, 1),       # fp32 activations
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_prefill_fp8_cache_write(hl, orc, case):
    """fp8 tiled caches hold exactly the e4m3 encoding of what an fp32
    column-major cache receives from the same prefill; outputs identical."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, io, start, style = PREFILL_CASES[case]
    print(f"prefill fp8 case {case}", flush=True)
    M = (start + T + 31) // 32 * 32 + 32
    q, k, v = (torch.from_numpy(orc.normal(h * d * T, 5300 + 3 * case + i)).reshape(h * d, T)
               .cuda().to(io) for i, h in enumerate((hq, hkv, hkv)))
    init = orc.to_storage(orc.normal(hkv * d * M, 5350 + case), FP8)
    res = {}
    for mode in ("f32", "fp8"):
        if mode == "f32":
            kc = torch.from_numpy(orc.upcast(init, FP8)).cuda().reshape(hkv * d, M)
            vc = kc.clone()
            lay = 0
        else:
            kc = tiled(torch.from_numpy(init).cuda(), hkv, d, M).reshape(hkv * d, M)
            vc = kc.clone()
            lay = TILED
        out = torch.full((hq * d, T), float("nan"), device="cuda")
        a = A.prefill_args(q, k, v, out, hq, hkv, d, T, rope_base=5e5, apply_rope=True,
                           rope_style=style, k_cache=kc, v_cache=vc, max_len=M, start_pos=start,
                           kv_layout=lay)
        A.attn_prefill(a, A.workspace(A.prefill_workspace_bytes(a)))
        torch.cuda.synchronize()
        if lay:
            kc, vc = untiled(kc, hkv, d, M), untiled(vc, hkv, d, M)
        res[mode] = (out.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy())
    assert np.array_equal(res["f32"][0], res["fp8"][0])
    assert np.array_equal(res["fp8"][1], orc.to_storage(res["f32"][1], FP8))
    assert np.array_equal(res["fp8"][2], orc.to_storage(res["f32"][2], FP8))


def test_fp8_needs_tiled_layout(hl, orc):
    from hippo_leap_amd import attention as A
    from hippo_leap_amd._lib import HLError
    kc = torch.zeros(8 * 64 * 64, dtype=torch.uint8, device="cuda")
    out = torch.empty(32 * 64, device="cuda")
    a = A.decode_args(torch.zeros(32 * 64, device="cuda"), kc, kc.clone(), out, 32, 8, 64, 64, 10)
    with pytest.raises(HLError):
        A.attn_decode(a, A.decode_workspace(a))
