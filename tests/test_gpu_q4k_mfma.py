"""GPU parity of the Q4_K GEMV on the matrix cores (matrices of 2^25 weights
and more: hl_gpu_linear_col_quant and the fused gate/up and K/V pairs,
backends/naive.nim:1580-1592, 1905-1920, 1799-1814) against the oracle's
dequantised rows (quant.nim dequantRowQ4K :244-277) and an fp64 product.

That kernel carries x as two fp16 parts with a power-of-two scale per
256-element block; the cases below cover blocks whose magnitudes differ by
up to 1e60, zeros, fp32 subnormals, rows counts that are odd or not a
multiple of the workgroup's, K with a partial 8-block group, the largest K
it takes (32768) and the first it does not.  Bar: 1e-4 relative (fp32)."""
import numpy as np
import pytest
import torch

from gguf_pack import random_rows
from util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu

SHAPES = [
    (8192, 4096),    # exactly 2^25 weights
    (8193, 4096),    # odd M: the last row pair has one row
    (6554, 5120),    # 20 blocks: a group of 4 blocks after two of 8
    (2731, 12288),   # six groups
    (1024, 32768),   # sixteen groups, one wave each
    (1025, 33024),   # beyond the MFMA kernel's K: the other direct kernel
]


def run(orc, raw, x, M, K):
    from hippo_leap_amd import attention as A
    y = torch.full((M,), float("nan"), device="cuda")
    A.gpu_linear_col_quant(y, torch.from_numpy(x).cuda(), torch.from_numpy(raw).cuda(), K, M, 12)
    torch.cuda.synchronize()
    W = orc.dequant_rows(12, raw, M, K).astype(np.float64)
    return y.cpu().numpy(), W @ x.astype(np.float64)


@pytest.mark.parametrize("shape", SHAPES)
def test_q4k_mfma_shapes(hl, orc, shape):
    M, K = shape
    print(f"q4k mfma shape M={M} K={K}", flush=True)
    rng = np.random.default_rng(8000 + M)
    raw = random_rows(rng, 12, M, K)
    got, ref = run(orc, raw, orc.normal(K, 8100 + M), M, K)
    assert rel_err(got, ref) < TOL_F32


def scaled_x(orc, K, seed, mags):
    """x whose 256-element blocks have magnitudes mags[b % len(mags)]."""
    x = orc.normal(K, seed).astype(np.float64)
    for b in range(K // 256):
        x[256 * b:256 * (b + 1)] *= mags[b % len(mags)]
    return x.astype(np.float32)


@pytest.mark.parametrize("kind", ["spread", "huge_tiny", "zeros", "subnormal", "mixed_in_block"])
def test_q4k_mfma_x_range(hl, orc, kind):
    """Per-block scaling: each block's largest |x| maps to [2^13, 2^14), so
    blocks of any magnitude keep 22 significant bits."""
    M, K = 8192, 4096
    print(f"q4k mfma x range: {kind}", flush=True)
    rng = np.random.default_rng(8200)
    raw = random_rows(rng, 12, M, K)
    if kind == "spread":        # 1e-6 .. 1e6 by block
        x = scaled_x(orc, K, 8201, [10.0 ** e for e in range(-6, 7, 2)])
    elif kind == "huge_tiny":   # 1e30 and 1e-30 blocks
        x = scaled_x(orc, K, 8202, [1e30, 1e-30, 1.0])
    elif kind == "zeros":       # zero blocks and zeros inside blocks
        x = scaled_x(orc, K, 8203, [0.0, 1.0, 0.0, 3.0])
        x[::7] = 0.0
    elif kind == "subnormal":   # fp32 subnormals only
        x = scaled_x(orc, K, 8204, [1e-40])
    else:                       # 1e4 and 1e-4 in one block
        x = orc.normal(K, 8205)
        x[::2] *= 1e4
        x[1::2] *= 1e-4
    got, ref = run(orc, raw, x, M, K)
    if kind in ("spread", "huge_tiny"):
        # every block's own part, not only the largest one, is checked: the
        # rows' sums restricted to each magnitude class
        W = orc.dequant_rows(12, raw, M, K).astype(np.float64)
        mags = np.abs(x.reshape(-1, 256)).max(axis=1)
        for cls in np.unique(np.round(np.log10(mags + 1e-300))):
            keep = np.repeat(np.round(np.log10(mags + 1e-300)) == cls, 256)
            xs = np.where(keep, x, 0).astype(np.float32)
            g2, r2 = run(orc, raw, xs, M, K)
            assert rel_err(g2, r2) < TOL_F32, f"class 1e{cls:.0f}"
    assert rel_err(got, ref) < TOL_F32


def test_q4k_mfma_graph_replay(hl, orc):
    """Captured in a HIP graph and replayed with new x in between: every
    replay matches an eager call on the same inputs."""
    from hippo_leap_amd import attention as A
    M, K = 8192, 4096
    print("q4k mfma graph replay", flush=True)
    rng = np.random.default_rng(8300)
    w = torch.from_numpy(random_rows(rng, 12, M, K)).cuda()
    x = torch.from_numpy(orc.normal(K, 8301)).cuda()
    y = torch.zeros(M, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.gpu_linear_col_quant(y, x, w, K, M, 12)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        A.gpu_linear_col_quant(y, x, w, K, M, 12)
    ref = torch.empty(M, device="cuda")
    for i in range(4):
        x.copy_(torch.from_numpy(orc.normal(K, 8310 + i)).cuda())
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        A.gpu_linear_col_quant(ref, x, w, K, M, 12)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"


@pytest.mark.parametrize("M", [8192, 8195])
def test_q4k_mfma_fused_pairs(hl, orc, M):
    """silu(G x) * (U x) and (K x, V x) through the MFMA kernel's pair mode."""
    from hippo_leap_amd import attention as A
    K = 4096
    print(f"q4k mfma fused pairs M={M}", flush=True)
    rng = np.random.default_rng(8400 + M)
    ga, ub = random_rows(rng, 12, M, K), random_rows(rng, 12, M, K)
    x = orc.normal(K, 8401)
    G = orc.dequant_rows(12, ga, M, K).astype(np.float64) @ x.astype(np.float64)
    U = orc.dequant_rows(12, ub, M, K).astype(np.float64) @ x.astype(np.float64)
    xd, gd, ud = torch.from_numpy(x).cuda(), torch.from_numpy(ga).cuda(), torch.from_numpy(ub).cuda()
    y = torch.full((M,), float("nan"), device="cuda")
    y2 = torch.full((M,), float("nan"), device="cuda")
    A.gpu_fused_kv_linear_quant(y, y2, xd, gd, ud, K, M, 12, 12)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), G) < TOL_F32 and rel_err(y2.cpu().numpy(), U) < TOL_F32
    A.gpu_fused_gate_up_silu_quant(y, xd, gd, ud, K, M, 12)
    torch.cuda.synchronize()
    with np.errstate(over="ignore"):
        ref = G / (1 + np.exp(-G)) * U
    assert rel_err(y.cpu().numpy(), ref) < TOL_F32
