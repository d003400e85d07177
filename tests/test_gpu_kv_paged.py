"""GPU parity of the paged KV-cache layout (HL_KV_PAGED32: pools of
32-position pages [Hkv][D][32] addressed through a per-sequence block table)
against the reference column-major layout, an extension of the reference
(whose caches are one contiguous block per sequence).

Every entry point that reads or writes a cache runs twice on the same
values: once column-major, once paged through a shuffled block table (the
pool made from the column-major caches on the host side of the test).  Only
addresses differ, so the bar is bit-exact: identical outputs, and pools
identical to the column-major caches converted."""
import numpy as np
import pytest
import torch

from test_gpu_decode import dev_bits, make_case

pytestmark = pytest.mark.gpu
PAGED = 2


def table_for(B, max_len, seed, spare=5):
    """A shuffled block table [B, max_len/32] over B*max_len/32 + spare pages."""
    nt = max_len // 32
    n_pages = B * nt + spare
    perm = np.random.default_rng(seed).permutation(n_pages)[:B * nt]
    return torch.from_numpy(perm.reshape(B, nt).astype(np.int32)).cuda(), n_pages


def paged(t, hkv, d, M, table, n_pages):
    from hippo_leap_amd import attention as A
    return A.kv_to_paged(t, hkv, d, M, table, n_pages)


def unpaged(pool, hkv, d, M, table):
    from hippo_leap_amd import attention as A
    return A.kv_from_paged(pool, hkv, d, M, table)


def bits(t):
    return t.view(torch.uint8).cpu().numpy() if t.element_size() == 1 else t.view(torch.int16).cpu().numpy()


DECODE_CASES = [
    # B, hq, hkv, d, max_len, L, dt, splits, ragged
    (8, 32, 8, 64, 2080, 2049, 1, 0, False),     # c3 shape
    (2, 32, 4, 128, 4096, 4000, 2, 0, False),    # c5 family: prefetching kernel
    (3, 16, 2, 128, 512, 500, 1, 3, True),       # ragged lengths, explicit splits
    (1, 8, 8, 64, 64, 33, 2, 1, False),          # one split, partial last tile
    (2, 40, 2, 64, 256, 256, 2, 0, False),       # two head chunks
    (1, 8, 1, 64, 40000, 40000, 2, 1, False),    # one split asked, > 32768 columns: plan splits
    (4, 16, 4, 128, 1024, 1000, 3, 0, True),     # fp8 pool, ragged
]


@pytest.mark.parametrize("case", range(len(DECODE_CASES)))
def test_decode_paged_matches_colmajor(hl, orc, case):
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, L, dt, splits, ragged = DECODE_CASES[case]
    print(f"decode paged case {case}", flush=True)
    if dt == 3:
        q = orc.uniform(B * hq * d, 6000 + case)
        n = B * hkv * d * M
        kc = torch.from_numpy(orc.to_storage(orc.normal(n, 6001 + case), 3)).cuda()
        vc = torch.from_numpy(orc.to_storage(orc.normal(n, 6002 + case), 3)).cuda()
    else:
        q, kb, vb = make_case(orc, B, hq, hkv, d, L, M, dt, 6000 + case)
        kc, vc = dev_bits(kb, dt), dev_bits(vb, dt)
    table, n_pages = table_for(B, M, 6100 + case)
    lens = None
    if ragged:
        lens = torch.tensor([L - 37 * b for b in range(B)], dtype=torch.int32, device="cuda")
    outs = []
    for layout in (1 if dt == 3 else 0, PAGED):   # fp8 has no column-major form: tiled stands in
        if layout == PAGED:
            k, v, tb = paged(kc, hkv, d, M, table, n_pages), paged(vc, hkv, d, M, table, n_pages), table
        elif layout == 1:
            k, v, tb = A.kv_to_tiled(kc, hkv, d, M), A.kv_to_tiled(vc, hkv, d, M), None
        else:
            k, v, tb = kc, vc, None
        out = torch.full((B * hq * d,), float("nan"), device="cuda")
        ns = 2 if (layout != PAGED and L > 32768) else splits  # what the paged plan must choose
        a = A.decode_args(torch.from_numpy(q).cuda(), k, v, out, hq, hkv, d, M, L, seq_lens=lens,
                          num_splits=ns, kv_layout=layout, block_table=tb)
        A.attn_decode(a, A.decode_workspace(a))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


STEP_CASES = [
    # B, hq, hkv, d, max_len, positions, style, norm, dt
    (8, 32, 8, 64, 2080, [2048], 0, False, 1),
    (3, 32, 4, 128, 992, [0, 500, 991], 0, True, 2),
    (2, 24, 3, 128, 160, [31, 32], 1, False, 3),
]


@pytest.mark.parametrize("case", range(len(STEP_CASES)))
def test_decode_step_and_rope_store_paged(hl, orc, case):
    """The fused step and the stand-alone rope/store write the new column at
    the page the table names; outputs equal the tiled layout's."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M, positions, style, norm, dt = STEP_CASES[case]
    print(f"step paged case {case}", flush=True)
    n = B * hkv * d * M
    if dt == 3:
        kb, vb = (orc.to_storage(orc.normal(n, 6200 + 10 * case + i), 3) for i in (1, 2))
        mk = lambda x: torch.from_numpy(x).cuda()
    else:
        _, kb, vb = make_case(orc, B, hq, hkv, d, M, M, dt, 6200 + 10 * case)
        mk = lambda x: dev_bits(x, dt)
    qa = orc.normal(B * hq * d, 6201 + case)
    ka, va = orc.normal(B * hkv * d, 6202 + case), orc.normal(B * hkv * d, 6203 + case)
    wq = torch.from_numpy(orc.uniform(d, 6204, 0.5, 1.5)).cuda() if norm else None
    wk = torch.from_numpy(orc.uniform(d, 6205, 0.5, 1.5)).cuda() if norm else None
    pos_t = torch.tensor(positions, dtype=torch.int32, device="cuda") if len(positions) > 1 else None
    L = max(positions) + 1
    table, n_pages = table_for(B, M, 6300 + case)
    res = {}
    for fused in (True, False):
        for layout in (1, PAGED):
            kc, vc = mk(kb), mk(vb)
            if layout == PAGED:
                kc, vc, tb = paged(kc, hkv, d, M, table, n_pages), paged(vc, hkv, d, M, table, n_pages), table
            else:
                kc, vc, tb = A.kv_to_tiled(kc, hkv, d, M), A.kv_to_tiled(vc, hkv, d, M), None
            qd = torch.from_numpy(qa).cuda()
            kd, vd = torch.from_numpy(ka).cuda(), torch.from_numpy(va).cuda()
            out = torch.full((B * hq * d,), float("nan"), device="cuda")
            kw = dict(rope_style=style, positions=pos_t, q_norm_w=wq, k_norm_w=wk, kv_layout=layout,
                      block_table=tb)
            if fused:
                rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5, **kw)
                at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, L, kv_layout=layout, block_table=tb)
                A.decode_step(rs, at, A.decode_step_workspace(rs, at))
            else:
                A.rope_store_decode(qd, kd, vd, kc, vc, hq, hkv, d, M, positions[0], 5e5, **kw)
            torch.cuda.synchronize()
            if layout == PAGED:
                kc, vc = unpaged(kc, hkv, d, M, table), unpaged(vc, hkv, d, M, table)
            else:
                kc, vc = A.kv_from_tiled(kc, hkv, d, M), A.kv_from_tiled(vc, hkv, d, M)
            res[fused, layout] = (out.cpu().numpy(), bits(kc), bits(vc))
    for fused in (True, False):
        assert np.array_equal(res[fused, 1][1], res[fused, PAGED][1])
        assert np.array_equal(res[fused, 1][2], res[fused, PAGED][2])
    assert np.array_equal(res[True, 1][0], res[True, PAGED][0])


PREFILL_CASES = [
    # hq, hkv, d, T, io dtype, kv dtype, start_pos, rope style
    (32, 8, 128, 300, torch.bfloat16, torch.bfloat16, 0, 0),   # K/V prologue kernel (c4 family)
    (16, 4, 128, 150, torch.float16, torch.float16, 5, 1),     # start_pos % 8 != 0
    (16, 2, 64, 100, torch.bfloat16, torch.float16, 40, 0),    # general prologue
    (8, 2, 64, 77, torch.float32, torch.bfloat16, 3, 1),       # fp32 activations
    (32, 8, 128, 200, torch.bfloat16, "fp8", 70, 0),           # fp8 pool
]


@pytest.mark.parametrize("case", range(len(PREFILL_CASES)))
def test_prefill_cache_write_paged(hl, orc, case):
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, io, kvd, start, style = PREFILL_CASES[case]
    print(f"prefill paged case {case}", flush=True)
    M = (start + T + 31) // 32 * 32 + 32
    q, k, v = (torch.from_numpy(orc.normal(h * d * T, 6400 + 3 * case + i)).reshape(h * d, T)
               .cuda().to(io) for i, h in enumerate((hq, hkv, hkv)))
    if kvd == "fp8":
        init_k = torch.from_numpy(orc.to_storage(orc.normal(hkv * d * M, 6450 + case), 3)).cuda()
        init_v = torch.from_numpy(orc.to_storage(orc.normal(hkv * d * M, 6460 + case), 3)).cuda()
    else:
        init_k = torch.from_numpy(orc.normal(hkv * d * M, 6450 + case)).cuda().to(kvd)
        init_v = torch.from_numpy(orc.normal(hkv * d * M, 6460 + case)).cuda().to(kvd)
    table, n_pages = table_for(1, M, 6500 + case)
    res = []
    for layout in (1, PAGED):
        if layout == PAGED:
            kc, vc, tb = paged(init_k, hkv, d, M, table, n_pages), paged(init_v, hkv, d, M, table, n_pages), table[0]
        else:
            kc, vc, tb = A.kv_to_tiled(init_k, hkv, d, M), A.kv_to_tiled(init_v, hkv, d, M), None
        out = torch.full((hq * d, T), float("nan"), device="cuda")
        a = A.prefill_args(q, k, v, out, hq, hkv, d, T, rope_base=5e5, apply_rope=True,
                           rope_style=style, k_cache=kc, v_cache=vc, max_len=M, start_pos=start,
                           kv_layout=layout, block_table=tb)
        A.attn_prefill(a, A.workspace(A.prefill_workspace_bytes(a)))
        torch.cuda.synchronize()
        if layout == PAGED:
            kc, vc = unpaged(kc, hkv, d, M, table), unpaged(vc, hkv, d, M, table)
        else:
            kc, vc = A.kv_from_tiled(kc, hkv, d, M), A.kv_from_tiled(vc, hkv, d, M)
        res.append((out.cpu().numpy(), bits(kc), bits(vc)))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])
    assert np.array_equal(res[0][2], res[1][2])


def test_decode_step_paged_fp8_graph_replay(hl, orc):
    """The fused step on a paged fp8 cache inside a HIP graph: replays with
    eager work in between give the eager result every time."""
    from hippo_leap_amd import attention as A
    B, hq, hkv, d, M = 4, 32, 4, 128, 2048
    n = B * hkv * d * M
    kb = torch.from_numpy(orc.to_storage(orc.normal(n, 6601), 3)).cuda()
    vb = torch.from_numpy(orc.to_storage(orc.normal(n, 6602), 3)).cuda()
    table, n_pages = table_for(B, M, 6603)
    kc, vc = paged(kb, hkv, d, M, table, n_pages), paged(vb, hkv, d, M, table, n_pages)
    qd = torch.from_numpy(orc.normal(B * hq * d, 6604)).cuda()
    kd = torch.from_numpy(orc.normal(B * hkv * d, 6605)).cuda()
    vd = torch.from_numpy(orc.normal(B * hkv * d, 6606)).cuda()
    out = torch.empty(B * hq * d, device="cuda")
    rs = A.rope_store_args(qd, kd, vd, kc, vc, hq, hkv, d, M, 1500, 1e6, kv_layout=PAGED,
                           block_table=table)
    at = A.decode_args(qd, kc, vc, out, hq, hkv, d, M, 1501, kv_layout=PAGED, block_table=table)
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
