"""GPU parity of the hidden-state RMSNorms around attention:
hl_gpu_rmsnorm_cols (gpuRmsnormCols, backends/naive.nim:2801-2843) and
hl_gpu_residual_rmsnorm (gpuResidualRmsnorm, naive.nim:2845-2882), against the
oracle's tensor.nim rmsnorm restatements (tensor.nim:83-118), pinned in
tests/test_oracle.py.  Bar: 1e-4 relative (fp32); the residual sum written
back to x is bit-exact (one fp32 add)."""
import numpy as np
import pytest
import torch

from util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,T", [(2048, 1), (4096, 1), (4096, 7), (2048, 64), (4096, 512),
                                   (100, 130), (5120, 63), (16384, 1), (130, 1), (16388, 1)])
def test_rmsnorm_cols_matches_oracle(hl, orc, dim, T):
    from hippo_leap_amd import attention as A
    print(f"rmsnorm_cols dim={dim} T={T}", flush=True)
    x = orc.normal(dim * T, 4000 + dim + T, 0.0, 3.0).reshape(dim, T)
    w = orc.uniform(dim, 4001, 0.5, 1.5)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    out = torch.full((dim, T), float("nan"), device="cuda")
    A.gpu_rmsnorm_cols(out, xd, wd, dim, T, 1e-5)
    ref = orc.rmsnorm_cols(x, w, 1e-5)
    assert rel_err(out.cpu().numpy(), ref) < TOL_F32
    A.gpu_rmsnorm_cols(xd, xd, wd, dim, T, 1e-5)  # in place
    assert rel_err(xd.cpu().numpy(), ref) < TOL_F32


@pytest.mark.parametrize("dim", [2048, 4096, 5120, 77, 16384, 16388, 130])
def test_residual_rmsnorm_matches_oracle(hl, orc, dim):
    from hippo_leap_amd import attention as A
    x = orc.normal(dim, 4100 + dim)
    r = orc.normal(dim, 4200 + dim, 0.0, 0.5)
    w = orc.uniform(dim, 4300 + dim, 0.5, 1.5)
    xd = torch.from_numpy(x).cuda()
    out = torch.full((dim,), float("nan"), device="cuda")
    A.gpu_residual_rmsnorm(out, xd, torch.from_numpy(r).cuda(), torch.from_numpy(w).cuda(), dim,
                           1e-6)
    xs = x + r
    assert np.array_equal(xd.cpu().numpy(), xs)
    assert rel_err(out.cpu().numpy(), orc.rmsnorm(xs.reshape(1, dim), w, 1e-6).reshape(-1)) < TOL_F32


def test_residual_rmsnorm_misaligned(hl, orc):
    """Vectors not on 16 bytes take the scalar kernel; same results."""
    from hippo_leap_amd import attention as A
    dim = 4096
    x = orc.normal(dim, 4400)
    r = orc.normal(dim, 4401, 0.0, 0.5)
    w = orc.uniform(dim, 4402, 0.5, 1.5)
    buf = torch.zeros(dim + 4, device="cuda")
    buf[1:1 + dim] = torch.from_numpy(x).cuda()
    xd = buf[1:1 + dim]
    out = torch.full((dim,), float("nan"), device="cuda")
    A.gpu_residual_rmsnorm(out, xd, torch.from_numpy(r).cuda(), torch.from_numpy(w).cuda(), dim, 1e-6)
    xs = x + r
    assert np.array_equal(xd.cpu().numpy(), xs)
    assert rel_err(out.cpu().numpy(), orc.rmsnorm(xs.reshape(1, dim), w, 1e-6).reshape(-1)) < TOL_F32

