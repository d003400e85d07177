"""GPU parity of the quantized decode GEMV (hl_gpu_linear_col_quant, the
drop-in for gpuLinearColQuant, backends/naive.nim:1580-1592) against the
oracle's restatement of quant.nim's dequantisers (pinned in
tests/test_oracle.py) followed by an fp64 product: every type the
reference dispatches (F16, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K,
IQ4_NL), dword-aligned rows and the byte-load path (row sizes not a
multiple of 4), the direct and LDS-staged kernels, one to four rows per
wave.  Bar: 1e-4 relative (fp32)."""
import numpy as np
import pytest
import torch

from gguf_pack import random_rows
from util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu

CASES = [
    # qtype, rows, k
    (1, 300, 512), (1, 2048, 4096),
    (8, 300, 4096), (8, 4096, 4096), (8, 17, 1120),     # K % 64 != 0: byte loads
    (12, 300, 4096), (12, 4096, 4096), (12, 1024, 14336), (12, 5, 256),
    (14, 300, 4096), (14, 2048, 4096), (14, 33, 768),   # K % 512 != 0: byte loads
    # four rows per wave (M >= 8192)
    (1, 8193, 64), (8, 8195, 256), (12, 8200, 512), (14, 8199, 512),
    # the other types of the reference's dispatcher (LDS-staged kernel;
    # Q5_K also direct), F16 rows of any length
    (6, 300, 4096), (6, 33, 96), (7, 300, 4096), (7, 2100, 1024), (20, 300, 4096), (20, 17, 160),
    (10, 300, 4096), (10, 9, 768), (11, 300, 4096), (11, 2100, 512),
    (13, 300, 4096), (13, 4096, 4096), (13, 8200, 1024), (13, 5, 256),
    (1, 300, 100), (1, 70, 1), (1, 2050, 4100),
    # one row; long rows (many steps per wave with the four-way split)
    (1, 1, 4096), (6, 1, 4096), (8, 1, 32), (10, 1, 256), (11, 1, 4096), (12, 1, 4096),
    (13, 1, 512), (14, 1, 4096), (20, 1, 32), (7, 3, 64),
    (14, 2048, 14336), (10, 700, 14336), (11, 300, 14336), (6, 4096, 14336), (20, 2100, 14336),
    # K between one and four wave steps
    (1, 300, 1024), (8, 2100, 1024), (14, 700, 2048), (12, 9000, 4096),
]

# (qtype, rows, k, byte offset of w, float offset of x): a 2-byte weight
# offset flips the parity of every Q8_0 / Q6_K block start; an odd byte
# offset or an x that is not 16-byte aligned takes the LDS-staged kernel.
OFFSET_CASES = [
    (1, 300, 512, 0, 1), (1, 300, 544, 2, 0), (1, 300, 512, 16, 0),
    (8, 300, 1024, 2, 0), (8, 3000, 1056, 2, 0), (8, 300, 1024, 1, 0), (8, 300, 1024, 0, 3),
    (12, 300, 1024, 4, 0), (12, 300, 1024, 16, 0), (12, 2500, 1024, 0, 2),
    (14, 300, 1024, 2, 0), (14, 9000, 768, 2, 0), (14, 300, 1024, 3, 0), (14, 300, 768, 0, 1),
    (13, 300, 1024, 8, 0), (13, 300, 1024, 0, 1), (6, 300, 1024, 1, 0), (11, 300, 1024, 2, 3),
    (20, 300, 1024, 3, 1), (10, 300, 1024, 2, 0), (7, 300, 1024, 1, 2),
    (6, 300, 1024, 2, 0), (20, 300, 1056, 2, 0), (7, 300, 1024, 2, 0), (6, 8195, 96, 2, 0),
    (20, 8200, 544, 0, 0), (7, 8193, 160, 2, 0),
    (10, 300, 1024, 4, 0), (10, 8200, 768, 0, 0), (11, 300, 1280, 2, 0), (11, 8200, 768, 0, 0),
    (11, 300, 1024, 1, 0),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_linear_col_quant_matches_oracle(hl, orc, case):
    from hippo_leap_amd import attention as A
    qt, M, K = CASES[case]
    print(f"quant GEMV case {case}: type {qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(7000 + case)
    raw = random_rows(rng, qt, M, K)
    x = orc.normal(K, 7100 + case)
    y = torch.full((M,), float("nan"), device="cuda")
    A.gpu_linear_col_quant(y, torch.from_numpy(x).cuda(), torch.from_numpy(raw).cuda(), K, M, qt)
    torch.cuda.synchronize()
    W = orc.dequant_rows(qt, raw, M, K).astype(np.float64)
    assert rel_err(y.cpu().numpy(), W @ x.astype(np.float64)) < TOL_F32


@pytest.mark.parametrize("case", range(len(OFFSET_CASES)))
def test_linear_col_quant_offsets(hl, orc, case):
    from hippo_leap_amd import attention as A
    qt, M, K, wo, xo = OFFSET_CASES[case]
    print(f"quant GEMV offset case {case}: type {qt} M={M} K={K} w+{wo} x+{xo}", flush=True)
    rng = np.random.default_rng(7200 + case)
    raw = random_rows(rng, qt, M, K)
    x = orc.normal(K, 7300 + case)
    wbuf = torch.zeros(raw.size + 16, dtype=torch.uint8, device="cuda")
    wbuf[wo:wo + raw.size] = torch.from_numpy(raw).cuda()
    xbuf = torch.zeros(K + 4, device="cuda")
    xbuf[xo:xo + K] = torch.from_numpy(x).cuda()
    y = torch.full((M,), float("nan"), device="cuda")
    A.gpu_linear_col_quant(y, xbuf[xo:], wbuf[wo:], K, M, qt)
    torch.cuda.synchronize()
    W = orc.dequant_rows(qt, raw, M, K).astype(np.float64)
    assert rel_err(y.cpu().numpy(), W @ x.astype(np.float64)) < TOL_F32


@pytest.mark.parametrize("qt", [14, 6])
def test_linear_col_quant_tall(hl, orc, qt):
    """Output-head shapes (65536+ rows): each row in one wave, all four
    steps in it.  64 random rows repeated 1024 times."""
    from hippo_leap_amd import attention as A
    K, base, reps = 4096, 64, 1024
    M = base * reps
    print(f"quant GEMV tall: type {qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(7300 + qt)
    raw = random_rows(rng, qt, base, K)
    x = orc.normal(K, 7301)
    y = torch.full((M,), float("nan"), device="cuda")
    A.gpu_linear_col_quant(y, torch.from_numpy(x).cuda(), torch.from_numpy(np.tile(raw, reps)).cuda(), K, M, qt)
    torch.cuda.synchronize()
    ref = np.tile(orc.dequant_rows(qt, raw, base, K).astype(np.float64) @ x.astype(np.float64), reps)
    assert rel_err(y.cpu().numpy(), ref) < TOL_F32


def test_linear_col_quant_errors(hl):
    from hippo_leap_amd import attention as A
    from hippo_leap_amd._lib import HLError
    x = torch.zeros(512, device="cuda")
    y = torch.zeros(8, device="cuda")
    w = torch.zeros(8 * 512, dtype=torch.uint8, device="cuda")
    with pytest.raises(HLError, match="unsupported quant type"):
        A.gpu_linear_col_quant(y, x, w, 512, 8, 9)  # Q8_1: not in the reference dispatcher
    with pytest.raises(HLError, match="q4_K row size must be multiple of 256"):
        A.gpu_linear_col_quant(y, x, w, 300, 8, 12)
    for qt, name, qk in ((6, "q5_0", 32), (7, "q5_1", 32), (10, "q2_K", 256), (11, "q3_K", 256),
                         (13, "q5_K", 256), (20, "iq4_nl", 32)):
        with pytest.raises(HLError, match=f"{name} row size must be multiple of {qk}"):
            A.gpu_linear_col_quant(y, x, w, 300, 8, qt)


@pytest.mark.parametrize("qt,M,K", [(12, 4096, 4096), (14, 300, 1024), (11, 700, 512), (8, 9000, 256)])
def test_linear_col_quant_graph_replay(hl, orc, qt, M, K):
    """Captured in a HIP graph and replayed with new x written eagerly in
    between: every replay matches an eager call on the same inputs."""
    from hippo_leap_amd import attention as A
    print(f"quant GEMV graph replay: type {qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(7400 + qt)
    w = torch.from_numpy(random_rows(rng, qt, M, K)).cuda()
    x = torch.from_numpy(orc.normal(K, 7500 + qt)).cuda()
    y = torch.zeros(M, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.gpu_linear_col_quant(y, x, w, K, M, qt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.gpu_linear_col_quant(y, x, w, K, M, qt)
    ref = torch.empty(M, device="cuda")
    for i in range(4):
        x.copy_(torch.from_numpy(orc.normal(K, 7600 + 10 * qt + i)).cuda())
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        A.gpu_linear_col_quant(ref, x, w, K, M, qt)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"


FUSED = [(12, 14336, 4096), (12, 300, 512), (11, 700, 1024), (13, 2100, 2048), (8, 4096, 4096),
         (14, 900, 768), (1, 300, 512), (20, 333, 1024), (6, 64, 256), (10, 500, 512),
         # four to seven steps per row: each row's blocks split over two waves
         (14, 2000, 4096), (11, 701, 6144), (10, 333, 4096), (1, 300, 2048),
         # a Q4_K pair of 2^24 weights per matrix: the matrix-core pair kernel
         (12, 8192, 2048)]


@pytest.mark.parametrize("qt,M,K", FUSED)
def test_fused_gate_up_silu_and_kv(hl, orc, qt, M, K):
    """gpuFusedGateUpSiluQ4K/Q3K and gpuFusedKVLinearQ4K (naive.nim:1905-1920,
    1693-1708, 1799-1814) for every type: silu(G x) * (U x) and (K x, V x) in
    one launch against the oracle's dequantised rows."""
    from hippo_leap_amd import attention as A
    print(f"fused pair: type {qt} M={M} K={K}", flush=True)
    rng = np.random.default_rng(7700 + qt)
    ga, ub = random_rows(rng, qt, M, K), random_rows(rng, qt, M, K)
    x = orc.normal(K, 7800 + qt)
    G = orc.dequant_rows(qt, ga, M, K).astype(np.float64) @ x.astype(np.float64)
    U = orc.dequant_rows(qt, ub, M, K).astype(np.float64) @ x.astype(np.float64)
    xd = torch.from_numpy(x).cuda()
    gd, ud = torch.from_numpy(ga).cuda(), torch.from_numpy(ub).cuda()
    y = torch.full((M,), float("nan"), device="cuda")
    A.gpu_fused_gate_up_silu_quant(y, xd, gd, ud, K, M, qt)
    y2 = torch.full((M,), float("nan"), device="cuda")
    A.gpu_fused_kv_linear_quant(y, y2, xd, gd, ud, K, M, qt, qt)  # y reused: fused result checked below
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), G) < TOL_F32 and rel_err(y2.cpu().numpy(), U) < TOL_F32
    A.gpu_fused_gate_up_silu_quant(y, xd, gd, ud, K, M, qt)
    torch.cuda.synchronize()
    with np.errstate(over="ignore"):
        ref = G / (1 + np.exp(-G)) * U
    assert rel_err(y.cpu().numpy(), ref) < TOL_F32


def test_fused_kv_mixed_types_and_alignment(hl, orc):
    """Q2_K keys with Q3_K values (gpuFusedKVLinearQ2KQ3K) and misaligned x
    run as two launches; the fused gate/up rejects a misaligned x."""
    from hippo_leap_amd import attention as A
    from hippo_leap_amd._lib import HLError
    M, K = 500, 512
    rng = np.random.default_rng(7900)
    ka, vb = random_rows(rng, 10, M, K), random_rows(rng, 11, M, K)
    x = orc.normal(K, 7901)
    xbuf = torch.zeros(K + 4, device="cuda")
    xbuf[1:1 + K] = torch.from_numpy(x).cuda()
    xal = torch.from_numpy(x).cuda()
    for xd in (xal, xbuf[1:1 + K]):
        k = torch.full((M,), float("nan"), device="cuda")
        v = torch.full((M,), float("nan"), device="cuda")
        A.gpu_fused_kv_linear_quant(k, v, xd, torch.from_numpy(ka).cuda(), torch.from_numpy(vb).cuda(),
                                    K, M, 10, 11)
        torch.cuda.synchronize()
        assert rel_err(k.cpu().numpy(), orc.dequant_rows(10, ka, M, K).astype(np.float64) @ x) < TOL_F32
        assert rel_err(v.cpu().numpy(), orc.dequant_rows(11, vb, M, K).astype(np.float64) @ x) < TOL_F32
    w = torch.from_numpy(ka).cuda()
    with pytest.raises(HLError, match="16-byte aligned"):
        A.gpu_fused_gate_up_silu_quant(k, xbuf[1:1 + K], w, w, K, M, 10)
    with pytest.raises(HLError, match="unsupported quant type"):
        A.gpu_fused_gate_up_silu_quant(k, xal, w, w, K, M, 9)
