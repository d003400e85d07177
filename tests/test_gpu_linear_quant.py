"""GPU parity of the quantized decode GEMV (hl_gpu_linear_col_quant, the
drop-in for gpuLinearColQuant, backends/naive.nim:1580-1592) against the
oracle's restatement of quant.nim's dequantisers (pinned in
tests/test_oracle.py) followed by an fp64 product: F16, Q8_0, Q4_K and Q6_K
rows, dword-aligned rows and the byte-load path (row sizes not a multiple of
4), one and four waves per row.  Bar: 1e-4 relative (fp32)."""
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


def test_linear_col_quant_errors(hl):
    from hippo_leap_amd import attention as A
    from hippo_leap_amd._lib import HLError
    x = torch.zeros(512, device="cuda")
    y = torch.zeros(8, device="cuda")
    w = torch.zeros(8 * 512, dtype=torch.uint8, device="cuda")
    with pytest.raises(HLError, match="unsupported quant type"):
        A.gpu_linear_col_quant(y, x, w, 512, 8, 10)
    with pytest.raises(HLError, match="q4_K row size must be multiple of 256"):
        A.gpu_linear_col_quant(y, x, w, 300, 8, 12)
