"""GPU parity of the tiled KV-cache layout (HL_KV_TILED32: per kv head,
max_len/32 tiles of [D][32]) against the reference column-major layout.

Every entry point that reads or writes a cache is run twice on the same
values, once per layout (the tiled cache made from the column-major one on
the host side of the test).  Only addresses differ between the two runs, so
the bar is bit-exact: identical outputs, and tiled caches identical to the
column-major caches converted.  The column-major path itself is pinned to
the CPU oracle by the other GPU tests; one case here also checks the oracle
directly."""
import numpy as np
import pytest
import torch

from util import TOL_LOWP, rel_err
from test_gpu_decode import dev_bits, make_case, oracle_decode

pytestmark = pytest.mark.gpu

TILED = 1


def tiled(t, hkv, d, max_len):
    from hippo_leap_amd import attention as A
    return A.kv_to_tiled(t, hkv, d, max_len)


def bits(t):
    return t.view(torch.int16).cpu().numpy()


DECODE_CASES = [
    # B, hq, hkv, d, max_len, L, dt, splits, ragged
    (8, 32, 8, 64, 2080, 2049, 1, 0, False),     # c3 shape (max_len rounded to 32)
    (2, 32, 4, 128, 4096, 4000, 2, 0, False),    # c5 family: pipelined kernel
    (3, 16, 2, 128, 512, 500, 1, 3, True),       # ragged lengths, explicit splits
    (1, 8, 8, 64, 64, 33, 2, 1, False),          # one split, partial last tile
    (2, 40, 2, 64, 256, 256, 2, 0, False),       # G = 20: two head chunks, full cache
]


@pytest.mark.parametrize("case", range(len(DECODE_CASES)))
def test_decode_tiled_matches_colmajor(hl, orc, case):
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, L, dt, splits, ragged = DECODE_CASES[case]
    print(f"decode tiled case {case}", flush=True)
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, M, dt, 2100 + case)
    qd = torch.from_numpy(q).cuda()
    kc, vc = dev_bits(kb, dt), dev_bits(vb, dt)
    lens = None
    if ragged:
        lens = torch.tensor([L - 37 * b for b in range(B)], dtype=torch.int32, device="cuda")
    outs = []
    for layout in (0, TILED):
        k = kc if layout == 0 else tiled(kc, hkv, d, M)
        v = vc if layout == 0 else tiled(vc, hkv, d, M)
        out = torch.full((B * hq * d,), float("nan"), device="cuda")
        a = A.decode_args(qd, k, v, out, hq, hkv, d, M, L, seq_lens=lens, num_splits=splits,
                          kv_layout=layout)
        A.attn_decode(a, A.decode_workspace(a))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    if case == 0:
        ref = oracle_decode(orc, q, kb, vb, B, hq, hkv, d, [L] * B, M, dt)
        assert rel_err(outs[1], ref) < TOL_LOWP


def test_decode_tiled_batch_stride(hl, orc):
    """Sequences further apart than one cache (a multiple of 8 elements)."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, L, dt = 3, 16, 4, 64, 320, 300, 1
    per = hkv * d * M
    stride = per + 64
    q, kb, vb = make_case(orc, B, hq, hkv, d, L, M, dt, 2200)
    kc, vc = dev_bits(kb, dt).view(B, per), dev_bits(vb, dt).view(B, per)
    outs = []
    for layout in (0, TILED):
        ks = torch.zeros(B, stride, dtype=kc.dtype, device="cuda")
        vs = torch.zeros(B, stride, dtype=kc.dtype, device="cuda")
        ks[:, :per] = kc if layout == 0 else tiled(kc, hkv, d, M)
        vs[:, :per] = vc if layout == 0 else tiled(vc, hkv, d, M)
        out = torch.empty(B * hq * d, device="cuda")
        a = A.decode_args(torch.from_numpy(q).cuda(), ks, vs, out, hq, hkv, d, M, L,
                          cache_batch_stride=stride, kv_layout=layout)
        A.attn_decode(a, A.decode_workspace(a))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


STEP_CASES = [
    # B, hq, hkv, d, max_len, positions, rope_dim, style, norm
    (8, 32, 8, 64, 2080, [2048], 0, 0, False),        # c3 step
    (3, 32, 4, 128, 992, [0, 500, 991], 0, 0, True),  # ragged, qkNorm, first/last column
    (2, 24, 3, 128, 160, [31, 32], 0, 1, False),      # new column on a tile edge, interleaved
]


@pytest.mark.parametrize("dt", [1, 2])
@pytest.mark.parametrize("case", range(len(STEP_CASES)))
def test_decode_step_and_rope_store_tiled(hl, orc, dt, case):
    """The fused step and the stand-alone rope/store write the new column
    into the tiled cache at the same place the conversion puts it, and the
    step's output equals the column-major step's."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, positions, rope_dim, style, norm = STEP_CASES[case]
    print(f"step tiled case {case} dt {dt}", flush=True)
    q, kb, vb = make_case(orc, B, hq, hkv, d, M, M, dt, 2300 + 10 * case)
    qa = orc.normal(B * hq * d, 2301 + case)
    ka, va = orc.normal(B * hkv * d, 2302 + case), orc.normal(B * hkv * d, 2303 + case)
    wq = torch.from_numpy(orc.uniform(d, 2304, 0.5, 1.5)).cuda() if norm else None
    wk = torch.from_numpy(orc.uniform(d, 2305, 0.5, 1.5)).cuda() if norm else None
    pos_t = torch.tensor(positions, dtype=torch.int32, device="cuda") if len(positions) > 1 else None
    L = max(positions) + 1
    res = {}
    for fused in (True, False):
        for layout in (0, TILED):
            kc, vc = dev_bits(kb, dt), dev_bits(vb, dt)
            if layout:
                kc, vc = tiled(kc, hkv, d, M), tiled(vc, hkv, d, M)
            qd = torch.from_numpy(qa).cuda()
            kd, vd = torch.from_numpy(ka).cuda(), torch.from_numpy(va).cuda()
            out = torch.full((B * hq * d,), float("nan"), device="cuda")
            rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5,
                                   rope_dim=rope_dim, rope_style=style, positions=pos_t,
                                   q_norm_w=wq, k_norm_w=wk, kv_layout=layout)
            if fused:
                at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, L, kv_layout=layout)
                A.decode_step(rs, at, A.decode_step_workspace(rs, at))
            else:
                A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5,
                                    rope_dim=rope_dim, rope_style=style, positions=pos_t,
                                    q_norm_w=wq, k_norm_w=wk, kv_layout=layout)
            torch.cuda.synchronize()
            if layout:
                kc, vc = A.kv_from_tiled(kc, hkv, d, M), A.kv_from_tiled(vc, hkv, d, M)
            res[fused, layout] = (out.cpu().numpy(), bits(kc), bits(vc))
    for fused in (True, False):
        assert np.array_equal(res[fused, 0][1], res[fused, TILED][1])
        assert np.array_equal(res[fused, 0][2], res[fused, TILED][2])
    assert np.array_equal(res[True, 0][0], res[True, TILED][0])


PREFILL_CASES = [
    # hq, hkv, d, T, io_dt, kv_dt, start_pos, rope style
    (32, 8, 128, 300, 2, 2, 0, 0),      # c4 family: K/V prologue kernel, half-split
    (16, 4, 128, 150, 1, 1, 5, 1),      # start_pos % 8 != 0: 8-column runs cross tiles
    (16, 2, 64, 100, 2, 1, 40, 0),      # head dim 64: general prologue, mixed dtypes
    (8, 2, 64, 77, 0, 2, 3, 1),         # fp32 activations, bf16 cache
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_prefill_cache_write_tiled(hl, orc, case):
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, io, kvd, start, style = PREFILL_CASES[case]
    print(f"prefill tiled case {case}", flush=True)
    TDT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}
    M = (start + T + 31) // 32 * 32 + 32
    q, k, v = (torch.from_numpy(orc.normal(h * d * T, 2400 + 3 * case + i)).reshape(h * d, T)
               .cuda().to(TDT[io]) for i, h in enumerate((hq, hkv, hkv)))
    init_k = torch.from_numpy(orc.normal(hkv * d * M, 2450 + case)).cuda().to(TDT[kvd]).reshape(hkv * d, M)
    init_v = torch.from_numpy(orc.normal(hkv * d * M, 2460 + case)).cuda().to(TDT[kvd]).reshape(hkv * d, M)
    res = []
    for layout in (0, TILED):
        kc = init_k.clone() if layout == 0 else tiled(init_k, hkv, d, M)
        vc = init_v.clone() if layout == 0 else tiled(init_v, hkv, d, M)
        out = torch.full((hq * d, T), float("nan"), device="cuda")
        a = A.prefill_args(q, k, v, out, hq, hkv, d, T, rope_base=5e5, apply_rope=True,
                           rope_style=style, k_cache=kc, v_cache=vc, max_len=M, start_pos=start,
                           kv_layout=layout)
        A.attn_prefill(a, A.workspace(A.prefill_workspace_bytes(a)))
        torch.cuda.synchronize()
        if layout:
            kc, vc = A.kv_from_tiled(kc, hkv, d, M), A.kv_from_tiled(vc, hkv, d, M)
        res.append((out.cpu().numpy(), bits(kc), bits(vc)))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])   # written columns and untouched ones alike
    assert np.array_equal(res[0][2], res[1][2])
