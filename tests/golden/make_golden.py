"""Writes the golden fixtures under tests/golden/ (small .npz files).

Inputs come from the oracle's seeded generator (oracle.uniform / normal, the
same counter-based SplitMix64 stream the tests use), expected outputs from an
fp64 NumPy implementation written here independently of oracle/hl_oracle.c,
and every attention expectation is cross-checked at generation time against
torch.nn.functional.scaled_dot_product_attention in fp64 (a library routine,
used only here).  The reference itself is Nim and not runnable in this
image; its own tests hold no attention goldens (tests/test_quant.nim:5-15,
the halfToFloat KAT, is checked directly in tests/test_oracle.py).

Semantics encoded (reference: monofuel/hippo_leap):
  GQA kvh = h // (Hq/Hkv)                       backends/naive.nim:3307-3308
  score = (q.k) * (1/sqrt(D)), softmax, p.V     naive.nim:3324-3367, tensor.nim:120-139
  causal j <= i                                 naive.nim:3403
  half-split RoPE with theta = powf(1/base, 2i/rd)  naive.nim:3020-3030, 3850-3861
  interleaved RoPE                              tensor.nim:141-166
  per-head RMSNorm before RoPE                  naive.nim:2910-2915, 4066-4074

Run: python tests/golden/make_golden.py   (rewrites the .npz files)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402


def theta64(rope_dim, base):
    # the fp32 table the backend builds, held in fp64 for the reference math
    i = np.arange(rope_dim // 2, dtype=np.float32)
    th = np.power(np.float32(1.0) / np.float32(base), (np.float32(2.0) * i) / np.float32(rope_dim),
                  dtype=np.float32)
    return th.astype(np.float64)


def rope64(x, pos, rope_dim, theta, style):
    """x: [..., D] fp64 rows at positions pos (broadcast over leading dims)."""
    x = x.copy()
    half = rope_dim // 2
    ang = np.asarray(pos, dtype=np.float64)[..., None] * theta
    c, s = np.cos(ang), np.sin(ang)
    if style == 0:
        i0, i1 = np.arange(half), np.arange(half) + half
    else:
        i0, i1 = 2 * np.arange(half), 2 * np.arange(half) + 1
    v0, v1 = x[..., i0].copy(), x[..., i1].copy()
    x[..., i0] = v0 * c - v1 * s
    x[..., i1] = v0 * s + v1 * c
    return x


def rmsnorm64(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def attn64(q, k, v, causal):
    """q [Hq, Tq, D], k/v [Hkv, Tk, D] fp64 -> [Hq, Tq, D]."""
    hq, hkv = q.shape[0], k.shape[0]
    g = hq // hkv
    out = np.empty_like(q)
    for h in range(hq):
        kh, vh = k[h // g], v[h // g]
        s = q[h] @ kh.T / np.sqrt(q.shape[-1])
        if causal:
            s = s + np.triu(np.full(s.shape, -np.inf), 1 + (k.shape[1] - q.shape[1]))
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        out[h] = (p / p.sum(-1, keepdims=True)) @ vh
    return out


def sdpa_check(q, k, v, causal, ref):
    g = q.shape[0] // k.shape[0]
    qt = torch.from_numpy(q)[None]
    kt = torch.from_numpy(np.repeat(k, g, 0))[None]
    vt = torch.from_numpy(np.repeat(v, g, 0))[None]
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)[0].numpy()
    err = np.abs(o - ref).max() / np.abs(ref).max()
    assert err < 1e-12, f"fp64 reference disagrees with torch SDPA: {err}"


def decode_case(name, dtype, hq=4, hkv=2, d=64, L=67, max_len=80, seed=11):
    n = hkv * d * max_len
    q = oracle.uniform(hq * d, seed)
    kc = oracle.to_storage(oracle.uniform(n, seed + 1), dtype)
    vc = oracle.to_storage(oracle.uniform(n, seed + 2), dtype)
    kf = oracle.upcast(kc, dtype).reshape(hkv, d, max_len)[:, :, :L].astype(np.float64)
    vf = oracle.upcast(vc, dtype).reshape(hkv, d, max_len)[:, :, :L].astype(np.float64)
    qq = q.astype(np.float64).reshape(hq, 1, d)
    kk, vv = kf.transpose(0, 2, 1), vf.transpose(0, 2, 1)
    exp = attn64(qq, kk, vv, causal=False)
    sdpa_check(qq, kk, vv, False, exp)
    np.savez(os.path.join(HERE, f"{name}.npz"), q=q, k_cache=kc, v_cache=vc,
             expected=exp.reshape(-1), shape=np.array([hq, hkv, d, L, max_len, dtype]))


def prefill_case(name, hq=4, hkv=2, d=64, T=33, base=10000.0, style=0, seed=21):
    q = oracle.normal(hq * d * T, seed).reshape(hq * d, T)
    k = oracle.normal(hkv * d * T, seed + 1).reshape(hkv * d, T)
    v = oracle.normal(hkv * d * T, seed + 2).reshape(hkv * d, T)
    th = theta64(d, base)
    pos = np.arange(T)
    qh = rope64(q.astype(np.float64).reshape(hq, d, T).transpose(0, 2, 1), pos, d, th, style)
    kh = rope64(k.astype(np.float64).reshape(hkv, d, T).transpose(0, 2, 1), pos, d, th, style)
    vh = v.astype(np.float64).reshape(hkv, d, T).transpose(0, 2, 1)
    exp = attn64(qh, kh, vh, causal=True)
    sdpa_check(qh, kh, vh, True, exp)
    np.savez(os.path.join(HERE, f"{name}.npz"), q=q, k=k, v=v,
             q_roped=qh.transpose(0, 2, 1).reshape(hq * d, T),
             k_roped=kh.transpose(0, 2, 1).reshape(hkv * d, T),
             expected=exp.transpose(0, 2, 1).reshape(hq * d, T),
             shape=np.array([hq, hkv, d, T, style]), base=np.array([base]))


def decode_step_case(name, dtype, hq=8, hkv=2, d=128, prev=37, max_len=48, base=1e6, seed=31,
                     eps=1e-6):
    """qkNorm -> RoPE at pos=prev -> store k,v at column prev -> attention over prev+1."""
    n = hkv * d * max_len
    q = oracle.normal(hq * d, seed)
    k = oracle.normal(hkv * d, seed + 1)
    v = oracle.normal(hkv * d, seed + 2)
    wq = oracle.uniform(d, seed + 3, 0.5, 1.5)
    wk = oracle.uniform(d, seed + 4, 0.5, 1.5)
    kc = oracle.to_storage(oracle.normal(n, seed + 5), dtype)
    vc = oracle.to_storage(oracle.normal(n, seed + 6), dtype)
    th = theta64(d, base)
    qn = rope64(rmsnorm64(q.astype(np.float64).reshape(hq, d), wq, eps), prev, d, th, 0)
    kn = rope64(rmsnorm64(k.astype(np.float64).reshape(hkv, d), wk, eps), prev, d, th, 0)
    # the new column is stored in the cache dtype (RNE) before attention reads it
    k_new = oracle.upcast(oracle.to_storage(kn.astype(np.float32), dtype), dtype).astype(np.float64)
    v_new = oracle.upcast(oracle.to_storage(v.reshape(hkv, d), dtype), dtype).astype(np.float64)
    kf = oracle.upcast(kc, dtype).reshape(hkv, d, max_len).astype(np.float64)[:, :, :prev + 1].copy()
    vf = oracle.upcast(vc, dtype).reshape(hkv, d, max_len).astype(np.float64)[:, :, :prev + 1].copy()
    kf[:, :, prev] = k_new
    vf[:, :, prev] = v_new
    kk, vv = kf.transpose(0, 2, 1), vf.transpose(0, 2, 1)
    exp = attn64(qn[:, None, :], kk, vv, causal=False)
    sdpa_check(qn[:, None, :], kk, vv, False, exp)
    np.savez(os.path.join(HERE, f"{name}.npz"), q=q, k=k, v=v, wq=wq, wk=wk, k_cache=kc,
             v_cache=vc, q_rot=qn.reshape(-1), k_rot=kn.reshape(-1), expected=exp.reshape(-1),
             shape=np.array([hq, hkv, d, prev, max_len, dtype]), base=np.array([base]),
             eps=np.array([eps]))


def main():
    decode_case("decode_f32", oracle.F32)
    decode_case("decode_f16", oracle.F16, seed=12)
    decode_case("decode_bf16", oracle.BF16, seed=13)
    prefill_case("prefill_f32_halfsplit", style=0)
    prefill_case("prefill_f32_interleaved", style=1, seed=24)
    decode_step_case("decode_step_bf16_qknorm", oracle.BF16)
    decode_step_case("decode_step_f16_qknorm", oracle.F16, seed=41)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
