"""GPU: the bf16/fp16 prefill over the whole range of its inputs.

The MFMA prefill (bf16/fp16 activations) rounds Q * scale, K and V (after
qkNorm and RoPE) to fp16 operands.  Inputs inside that range, including
large values (3e4) and tiny ones (3e-5, fp16 subnormals), match the CPU
oracle's fp32 attention over the same stored bits (naive.nim:3385-3464)
within the 2e-3 bar on the fp16 path alone.  A value of magnitude >= 65520
has no fp16 form: the call then recomputes its output on the fp32 fallback
that every MFMA prefill launches (gated on the overflow record), and the
output matches the oracle within the same bar with no extra call by the
caller, including fp16 inputs that only RoPE pushes past the limit.  The
outputs are checked first; hl_attn_prefill_fallback_ran then confirms
which path ran.  The record is per call: a later in-range call on the same
workspace (eager or a graph replay) takes the fp16 path again."""
import numpy as np
import pytest
import torch

from util import TOL_LOWP, rel_err
from test_gpu_prefill import TDT, from_dev, oracle_prefill, to_dev

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
    torch.cuda.synchronize()
    res = from_dev(out)  # read before any query of the record
    return res, A.prefill_fallback_ran(a, ws), ws


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
    hq, hkv, d, T, rd, style, dt, which, big = CASES[case]
    print(f"prefill range case {case}", flush=True)
    q, k, v = make(orc, hq, hkv, d, T, dt, 3000 + 20 * case, which, big)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5, style=style, rope_dim=rd)
    out, ran, _ = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                    apply_rope=True, rope_base=5e5, rope_style=style, rope_dim=rd)
    assert not ran
    err = rel_err(out, ref)
    print(f"case {case} rel err {err:.3e}")
    assert err < TOL_LOWP


@pytest.mark.parametrize("which", ["q", "k", "v"])
@pytest.mark.parametrize("d,rd", [(128, 128), (128, 64), (64, 64)])
def test_prefill_beyond_fp16_matches_oracle(hl, orc, which, d, rd):
    """bf16 activations of +-1e5 (and tiny ones) in Q, K or V, on the
    K/V-prologue path (d = rd = 128), the prepared-Q path (rd < d) and the
    general prologue (d = 64): the output matches the oracle within 2e-3
    with no call besides hl_attn_prefill, and the fp32 caches keep the exact
    values.  Q needs |q * scale| >= 65520, hence 1e7."""
    from hippo_leap_amd import attention as A
    hq, hkv, T, dt = 8, 2, 96, 2
    big = 1e5 if which != "q" else 1e7
    print(f"prefill overflow {which} d {d} rd {rd}", flush=True)
    q, k, v = make(orc, hq, hkv, d, T, dt, 3100 + d + rd, which, big)
    ref, _, kref = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5, rope_dim=rd)
    kc = torch.zeros(hkv * d, T, dtype=torch.float32, device="cuda")
    vc = torch.zeros(hkv * d, T, dtype=torch.float32, device="cuda")
    out, ran, ws = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                     apply_rope=True, rope_base=5e5, rope_dim=rd, k_cache=kc,
                                     v_cache=vc, max_len=T)
    err = rel_err(out, ref)
    print(f"rel err {err:.3e}", flush=True)
    assert err < TOL_LOWP
    assert ran
    assert np.array_equal(from_dev(vc), v)
    assert rel_err(from_dev(kc), kref) < 1e-6
    # the same workspace, in-range inputs: the fp16 path alone again
    q2, k2, v2 = make(orc, hq, hkv, d, T, dt, 3200 + d + rd)
    ref2, _, _ = oracle_prefill(orc, q2, k2, v2, hq, hkv, d, T, base=5e5, rope_dim=rd)
    out2, ran2, _ = prefill_and_check(to_dev(q2, dt), to_dev(k2, dt), to_dev(v2, dt), hq, hkv, d,
                                      T, ws=ws, apply_rope=True, rope_base=5e5, rope_dim=rd)
    assert not ran2
    assert rel_err(out2, ref2) < TOL_LOWP


def test_prefill_fp16_rope_overflow_matches_oracle(hl, orc):
    """fp16 activations of 6e4 that RoPE rotates past 65520 (|v0 c - v1 s| up
    to sqrt(2) * 6e4), with qkNorm off: every input is a finite fp16, the
    operand is not, and the fallback gives the oracle's result."""
    hq, hkv, d, T, dt = 4, 2, 128, 64, 1
    q, k, v = (orc.normal(h * d * T, 3300 + i).reshape(h * d, T) for i, h in enumerate((hq, hkv, hkv)))
    k[:, 20] = 6e4 * np.sign(k[:, 20])
    q, k, v = (orc.upcast(orc.to_storage(x, dt), dt).reshape(x.shape) for x in (q, k, v))
    assert np.abs(k).max() < 65504
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=1e4)
    out, ran, _ = prefill_and_check(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), hq, hkv, d, T,
                                    apply_rope=True, rope_base=1e4)
    assert rel_err(out, ref) < TOL_LOWP
    assert ran


@pytest.mark.parametrize("odt", [1, 2])
def test_prefill_fallback_low_precision_output_and_qknorm(hl, orc, odt):
    """The fallback writes fp16 / bf16 outputs (RNE of its fp32 result) and
    applies qkNorm before RoPE, as the fp16 path does: a bf16 K of 1e6 with
    qkNorm weights of 2e5 (normed values reach ~2e5)."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, dt = 8, 2, 128, 80, 2
    q, k, v = make(orc, hq, hkv, d, T, dt, 3500, "k", 1e6)
    wq = orc.uniform(d, 3510, 0.5, 1.5)
    wk = orc.uniform(d, 3511, 1e5, 2e5)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5, wq=wq, wk=wk)
    out = torch.full((hq * d, T), float("nan"), dtype=TDT[odt], device="cuda")
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    a = A.prefill_args(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), out, hq, hkv, d, T,
                       apply_rope=True, rope_base=5e5, q_norm_w=dev(wq), k_norm_w=dev(wk),
                       eps=1e-6)
    ws = A.workspace(A.prefill_workspace_bytes(a))
    A.attn_prefill(a, ws)
    torch.cuda.synchronize()
    got = from_dev(out)
    err = rel_err(got, ref)
    print(f"fallback out dtype {odt} rel err {err:.3e}", flush=True)
    assert err < TOL_LOWP + (4e-3 if odt == 2 else 5e-4)  # plus one output rounding
    assert A.prefill_fallback_ran(a, ws)


def test_prefill_fallback_graph_replays(hl, orc):
    """A captured prefill replayed on overflowing and then on in-range
    inputs (copied into the same input buffers between replays): every
    replay matches its eager result, and the record follows each replay."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T, dt = 8, 2, 128, 96, 2
    bad = make(orc, hq, hkv, d, T, dt, 3600, "v", 1e5)
    good = make(orc, hq, hkv, d, T, dt, 3700)
    qd, kd, vd = (to_dev(x, dt) for x in good)
    out = torch.empty(hq * d, T, dtype=torch.float32, device="cuda")
    a = A.prefill_args(qd, kd, vd, out, hq, hkv, d, T, apply_rope=True, rope_base=5e5)
    ws = A.workspace(A.prefill_workspace_bytes(a))
    eager = {}
    for name, src in (("bad", bad), ("good", good)):
        for dst, x in zip((qd, kd, vd), src):
            dst.copy_(to_dev(x, dt))
        A.attn_prefill(a, ws)
        torch.cuda.synchronize()
        eager[name] = (from_dev(out).copy(), A.prefill_fallback_ran(a, ws))
    assert eager["bad"][1] and not eager["good"][1]
    ref_bad, _, _ = oracle_prefill(orc, *bad, hq, hkv, d, T, base=5e5)
    assert rel_err(eager["bad"][0], ref_bad) < TOL_LOWP
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.attn_prefill(a, ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        A.attn_prefill(a, ws)
    for name in ("bad", "good", "good", "bad", "good"):
        src = bad if name == "bad" else good
        for dst, x in zip((qd, kd, vd), src):
            dst.copy_(to_dev(x, dt))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out), eager[name][0]), name
        assert A.prefill_fallback_ran(a, ws) == eager[name][1], name


def test_prefill_fp32_path_has_no_fallback(hl, orc):
    """fp32 activations run the fp32 kernel: no operand range limit."""
    from hippo_leap_amd import attention as A
    hq, hkv, d, T = 4, 2, 64, 40
    q, k, v = make(orc, hq, hkv, d, T, 0, 3400, "kv", 1e6)
    ref, _, _ = oracle_prefill(orc, q, k, v, hq, hkv, d, T, base=5e5)
    out, ran, _ = prefill_and_check(to_dev(q, 0), to_dev(k, 0), to_dev(v, 0), hq, hkv, d, T,
                                    apply_rope=True, rope_base=5e5)
    assert not ran
    assert rel_err(out, ref) < 1e-4
