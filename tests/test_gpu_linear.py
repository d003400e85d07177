"""GPU parity: the fp32 linear layer (hl_gpu_linear_col, the drop-in for
gpuLinearCol, backends/naive.nim:3519-3547) against the CPU oracle's
restatement of tensor.nim's matmul (tensor.nim:63-81), on both kernels:
the decode GEMV (seq_len == 1) and the fp32-MFMA GEMM (seq_len > 1), with
and without 16-byte loads (K or T not a multiple of 4, misaligned inputs),
ragged tiles, and at the Llama-3-8B projection shapes against an fp64
matmul of the same inputs; the 128 x 128-tile GEMM also over wide exponent
ranges and with inf / NaN operands.  Bar: 1e-4 relative (fp32)."""
import numpy as np
import pytest
import torch

from util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def run_linear(w, x, M, K, T, offset=0):
    """w [M, K], x [K, T] as float32 numpy; offset shifts x by that many
    floats inside its buffer (misaligned 16-byte loads must be avoided)."""
    from hippo_leap_amd import attention as A
    wd = torch.from_numpy(w).cuda()
    xb = torch.zeros(K * T + offset, device="cuda")
    xb[offset:] = torch.from_numpy(x.reshape(-1)).cuda()
    xd = xb[offset:]
    y = torch.full((M * T,), float("nan"), device="cuda")
    A.gpu_linear_col(y, xd, wd, K, M, T)
    torch.cuda.synchronize()
    return y.cpu().numpy().reshape(M, T)


CASES = [
    # M, K, T, x offset (floats)
    (2048, 2048, 1, 0),   # decode GEMV, one wave per row (TinyLlama q/o projection)
    (256, 2048, 1, 0),    # four waves per row (k/v projection)
    (37, 130, 1, 0),      # K % 4 != 0: one float per lane
    (5, 3, 1, 0),         # tiny
    (300, 1000, 1, 1),    # misaligned x: scalar loads
    (256, 512, 64, 0),    # GEMM, 64x64 tiles, exact
    (200, 96, 7, 0),      # T % 4 != 0: scalar loads, ragged tile
    (130, 100, 33, 0),    # K not a multiple of 32 or 4, ragged M and T
    (64, 64, 2, 0),       # smallest prefill
    (96, 72, 40, 2),      # misaligned x
    (2048, 40, 4096, 0),  # 128x128 tiles (>= 512 tiles), K tail inside one chunk
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_linear_col_matches_oracle(hl, orc, case):
    M, K, T, off = CASES[case]
    print(f"linear case {case}: M={M} K={K} T={T} offset={off}", flush=True)
    w = orc.uniform(M * K, 3100 + case).reshape(M, K)
    x = orc.normal(K * T, 3200 + case).reshape(K, T)
    got = run_linear(w, x, M, K, T, off)
    ref = orc.matmul(w, x)
    assert rel_err(got, ref) < TOL_F32


@pytest.mark.parametrize("M,K,T", [(4096, 4096, 1), (1024, 4096, 1), (14336, 4096, 1),
                                   (4096, 4096, 512), (1024, 4096, 4096)])
def test_linear_col_llama8b_shapes(hl, M, K, T):
    """Llama-3-8B projections (q/o 4096x4096, k/v 1024x4096, FFN 14336x4096)
    against a float64 matmul on the GPU of the same fp32 inputs."""
    print(f"linear full shape M={M} K={K} T={T}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(M * 7 + T)
    w = torch.rand(M, K, device="cuda", generator=g) * 2 - 1
    x = torch.randn(K, T, device="cuda", generator=g)
    y = torch.full((M, T), float("nan"), device="cuda")
    from hippo_leap_amd import attention as A
    A.gpu_linear_col(y, x, w, K, M, T)
    ref = (w.double() @ x.double())
    err = ((y.double() - ref).abs().max() / ref.abs().max()).item()
    assert err < TOL_F32, err


def test_linear_col_linearity_and_repeat(hl, orc):
    """W(a x1 + b x2) = a W x1 + b W x2, and a second call gives the same bits."""
    from hippo_leap_amd import attention as A
    M, K, T = 384, 768, 48
    w = torch.from_numpy(orc.uniform(M * K, 3301)).cuda()
    x1 = torch.from_numpy(orc.normal(K * T, 3302)).cuda()
    x2 = torch.from_numpy(orc.normal(K * T, 3303)).cuda()
    ys = []
    for x in (x1, x2, 0.5 * x1 - 2.0 * x2, x1):
        y = torch.empty(M * T, device="cuda")
        A.gpu_linear_col(y, x, w, K, M, T)
        ys.append(y)
    torch.cuda.synchronize()
    comb = (0.5 * ys[0].double() - 2.0 * ys[1].double())
    assert ((ys[2].double() - comb).abs().max() / comb.abs().max()).item() < TOL_F32
    assert torch.equal(ys[0], ys[3])


def _tile128_operands(seed):
    """2048 x 4096 outputs (512 tiles: the 128 x 128-tile GEMM), K = 256."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    M, K, T = 2048, 256, 4096
    w = torch.rand(M, K, device="cuda", generator=g) * 2 - 1
    x = torch.randn(K, T, device="cuda", generator=g)
    return M, K, T, w, x


def test_linear_col_gemm_wide_range(hl):
    """Rows of W scaled by 1e-18 .. 1e18 and columns of x by 1e-15 .. 1e15:
    every output within 1e-4 of its own row/column scale against a float64
    matmul."""
    from hippo_leap_amd import attention as A
    M, K, T, w, x = _tile128_operands(41)
    rs = torch.logspace(-18, 18, M, device="cuda")
    cs = torch.logspace(-15, 15, T, device="cuda")
    w = w * rs[:, None]
    x = x * cs[None, :]
    y = torch.full((M, T), float("nan"), device="cuda")
    A.gpu_linear_col(y, x, w, K, M, T)
    ref = w.double() @ x.double()
    scale = (w.double().abs() @ x.double().abs())  # |W| |x|: the sum's own scale
    err = ((y.double() - ref).abs() / scale).max().item()
    assert err < TOL_F32, err


def test_linear_col_gemm_inf_nan(hl):
    """inf and NaN through the GEMM: an inf weight gives inf where its x is
    nonzero and NaN where it is 0 (inf x 0), a NaN weight NaN, as the
    reference's fp32 products do; every other output matches a float64
    matmul."""
    from hippo_leap_amd import attention as A
    M, K, T, w, x = _tile128_operands(42)
    x = x.abs() + 0.5           # positive, so row 5's sum is +inf
    x[3, 100] = 0.0             # ... except column 100: inf x 0
    w[5, 3] = float("inf")
    w[7, 10] = float("nan")
    y = torch.full((M, T), 7.0, device="cuda")
    A.gpu_linear_col(y, x, w, K, M, T)
    yc = y.cpu()
    assert torch.isnan(yc[7]).all()
    assert torch.isnan(yc[5, 100])
    assert torch.isinf(yc[5, :100]).all() and torch.isinf(yc[5, 101:]).all() and (yc[5, :100] > 0).all()
    fin = torch.ones(M, dtype=torch.bool)
    fin[5] = fin[7] = False
    ref = (w.double() @ x.double()).cpu()
    err = ((yc.double()[fin] - ref[fin]).abs().max() / ref[fin].abs().max()).item()
    assert err < TOL_F32, err
