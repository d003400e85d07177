"""GPU: the fp16-operand prefill over the range of its inputs.

The MFMA prefill (bf16/fp16 activations) rounds Q * scale, K and V (after
qkNorm and RoPE) to fp16 operands.  Inputs inside that range, including
large values (3e4) and tiny ones (3e-5, fp16 subnormals), match the CPU
oracle's fp32 attention over the same stored bits (naive.nim:3385-3464)
within the 2e-3 bar, and hl_attn_prefill_range_check reports HL_OK.  A
value of magnitude >= 65520 has no fp16 form: such calls are reported as
HL_ERANGE by the check (the documented contract), including fp16 inputs
that only RoPE pushes past the limit; the caches still hold the exact
values.  The record is per call: a later in-range call on the same
workspace reports HL_OK again."""
import numpy as np
import pytest
import torch

from util import TOL_LOWP, rel_err
from test_gpu_prefill import from_dev, oracle_prefill, to_dev

pytestmark = pytest.mark.gpu


def with_outliers(x, seed, big, n_big, n_tiny):
    """x [R, T] with n_big entries set to +-big and n_tiny to +-3e-5."""
    rng = np.random.default_rng(seed)
    x = x.copy()
    R, T = x.shape
    for n, mag in ((n_big, big), (n_tiny, 3e-5)):
        r, t = rng.integers(0, R, n), rng.integers(0, T, n)
        x[r, t] = mag * rng.choice([-1.0, 1.0], n)
    return x


def prefill_and_check(q, k, v, hq, hkv, d, T, ws=None, **kw):
    from hippo_leap_amd import attention as A
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    a = A.prefill_args(q, k, v, out, hq, hkv, d, T, **kw)
    if ws is None:
        ws = A.workspace(A.prefill_workspace_bytes(a))
    A.attn_prefill(a, ws)
    rc = A.prefill_range_check(a, ws)
    return from_dev(out), rc, ws


def make(orc, hq, hkv, d, T, dt, seed, which="", big=0.0):
    src = []
    for i, (name, h) in enumerate((("q", hq), ("k", hkv), ("v", hkv))):
        x = orc.normal(h * d * T, seed + i).reshape(h * d, T)
        if name in which:
            x = with_outliers(x, seed + 10 + i, big, 6, 40)
        src.append(orc.upcast(orc.to_storage(x, dt), dt).reshape(h * d, T))
    return src


CASES = [
    # hq, hkv, d, T, rope_dim, style, io dtype, tensors with outliers, magnitude
    (8, 2, 128, 200, 128, 0, 2, "kv", 3e4),     # K/V prologue path, Q built in the flash kernel
    (8, 2, 128, 130, 64, 0, 2, "kv", 3e4),      # partial half-split RoPE: prepared-Q layout
    (8, 2, 64, 150, 64, 1, 1, "qkv", 2e4),      # D = 64 (general prologue), fp16, interleaved
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_prefill_large_and_tiny_values_in_range(hl, orc, case):
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, rd, style, dt, which, big = CASES[case]
    print(f"prefill range case {case}", flush=True)
    q, k, v = make(orc, hq, hkv, d, T, dt, 3000 + 20 * case, which, big)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5, style=style, rope_dim=rd)
    out, rc, _ = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                   apply_rope=True, rope_base=5e5, rope_style=style, rope_dim=rd)
    assert rc == A.HL_OK
    err = rel_err(out, ref)
    print(f"case {case} rel err {err:.3e}")
    assert err < TOL_LOWP


@pytest.mark.parametrize("which", ["q", "k", "v"])
@pytest.mark.parametrize("d,rd", [(128, 128), (128, 64)])
def test_prefill_beyond_fp16_is_reported(hl, orc, which, d, rd):
    """bf16 activations of +-1e5 (and tiny ones) in Q, K or V: HL_ERANGE, on
    the K/V-prologue path (rd = d) and the prepared-Q path (rd < d); the
    fp32 caches keep the exact values.  Q needs |q * scale| >= 65520."""
    from hippo_leap_amd import attention as A
    hq, hkv, T, dt = 8, 2, 96, 2
    big = 1e5 if which != "q" else 1e7
    q, k, v = make(orc, hq, hkv, d, T, dt, 3100 + d + rd, which, big)
    kc = torch.zeros(hkv * d, T, dtype=torch.float32, device="cuda")
    vc = torch.zeros(hkv * d, T, dtype=torch.float32, device="cuda")
    _, rc, ws = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                  apply_rope=True, rope_base=5e5, rope_dim=rd, k_cache=kc,
                                  v_cache=vc, max_len=T)
    assert rc == A.HL_ERANGE
    assert np.array_equal(from_dev(vc), v)
    # the same workspace, in-range inputs: the record is per call
    q2, k2, v2 = make(orc, hq, hkv, d, T, dt, 3200 + d + rd)
    ref, _, _ = oracle_prefill(orc, q2, k2, v2, hq, hkv, d, T, base=5e5, rope_dim=rd)
    out, rc2, _ = prefill_and_check(to_dev(q2, dt), to_dev(k2, dt), to_dev(v2, dt), hq, hkv, d, T,
                                    ws=ws, apply_rope=True, rope_base=5e5, rope_dim=rd)
    assert rc2 == A.HL_OK
    assert rel_err(out, ref) < TOL_LOWP


def test_prefill_fp16_rope_overflow_is_reported(hl, orc):
    """fp16 activations of 6e4 that RoPE rotates past 65520 (|v0 c - v1 s| up
    to sqrt(2) * 6e4): reported, though every input is a finite fp16."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, dt = 4, 2, 128, 64, 1
    q, k, v = (orc.normal(h * d * T, 3300 + i).reshape(h * d, T) for i, h in enumerate((hq, hkv, hkv)))
    k[:, 20] = 6e4 * np.sign(k[:, 20])
    q, k, v = (orc.upcast(orc.to_storage(x, dt), dt).reshape(x.shape) for x in (q, k, v))
    assert np.abs(k).max() < 65504
    _, rc, _ = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                 apply_rope=True, rope_base=1e4)
    assert rc == A.HL_ERANGE


def test_prefill_range_check_fp32_path_is_ok(hl, orc):
    """fp32 activations run the fp32 kernel: no operand range limit."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T = 4, 2, 64, 40
    q, k, v = make(orc, hq, hkv, d, T, 0, 3400, "kv", 1e6)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5)
    out, rc, _ = prefill_and_check(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T,
                                   apply_rope=True, rope_base=5e5)
    assert rc == A.HL_OK
    assert rel_err(out, ref) < 1e-4
