"""Benchmark of the MI355X attention stage (one GPU).

Headline workload ("decode attn GB/s at 2K ctx"):
  Llama-3.2-1B-shape batched decode step, fp16 KV cache: B=8 sequences with
  2048 cached positions each, one new token per sequence (L = 2049),
  Hq=32 / Hkv=8, D=64, RoPE theta 5e5, K/V ~ N(0, 0.5) (sigma 0.5).
  One step = hl_decode_step: RoPE of the new q/k, the K/V write at column
  2048 and split-K attention with its merge, in one launch; the W warmup and
  K timed steps each run as one captured HIP graph.  16 cache sets are
  rotated (16 x 33.6 MB > the 256 MB Infinity Cache) so every step streams
  its K/V from HBM.  The caches use the reference's column-major layout.
  value = algorithmic K+V bytes of one step / step time (GB/s).

Extra objects on the same JSON line:
  prefill: configs[3], Llama-3-8B-shape causal prefill, bf16, T=4096,
    Hq32/Hkv8, D128, RoPE 5e5, KV cache written; TFLOP/s on causal FLOPs
    4*Hq*D*T(T+1)/2 (prologue + flash kernel).
  decode_c5: configs[4], Qwen3-30B-A3B-shape decode, bf16 KV, B=16, L=32769,
    Hq32/Hkv4, D128, qkNorm + RoPE 1e6.
  decode_c5_tiled, decode_c3_tiled: the same steps with the caches in the
    opt-in tiled layout (HL_KV_TILED32: per kv head, 32-column tiles of
    [D][32]), same values.
  decode_c5_fp8, decode_c3_fp8: the same steps with fp8 e4m3 caches (tiled),
    GB/s of the fp8 bytes (half of the bf16/fp16 bytes per position).
  decode_c5_paged: the c5 step with the caches in a page pool (HL_KV_PAGED32)
    reached through a shuffled block table.
  decode_c1, prefill_c2: configs[0] and configs[1], the reference's fp32
    call contract (hl_gpu_attention_decode; fp32 prefill with RoPE 1e4 and
    the cache write), timed for reference: they are parity cases, not the
    metric.
  prefill_fp32_llama8b: the same fp32 prefill contract at the Llama-3-8B
    attention shape (head dim 128, T=4096).
  roofline: the fused step kernel (qkNorm/RoPE + KV write + split-K
    attention + merge) timed with HIP events on the stream it runs on.
  linear: hl_gpu_linear_col (the gpuLinearCol drop-in, fp32) at the
    projection shapes around attention: decode GEMV GB/s (weights from HBM)
    and prefill GEMM TFLOP/s against the fp32 peak; hl_gpu_linear_col_quant
    (gpuLinearColQuant) decode GEMV GB/s over F16, Q8_0, Q4_K, Q6_K weights.
  model_decode: greedy decode of Llama-3-8B- and Llama-3.2-1B-shaped dense
    decoders (Q4_K weights, random values) through hl_forward_decode_token,
    ms per token.
  decode_ends: greedy argmax over the logits (hl_argmax_async / hl_gpu_argmax)
    and the token embedding (hl_gpu_embedding), the ends of a decode step.
  cpu_baseline: the C oracle (single-threaded scalar fp32 restatement of the
    reference's tensor.nim math) timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16/fp16 MFMA
FP32_PEAK_TFLOPS = 157.3       # MI355X fp32 (vector / matrix)
METRIC = "decode attn GB/s (%HBM peak) at 2K ctx; prefill attn TFLOP/s (%MFMA peak)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def event_time_ms(torch, fn, iters):
    """Average ms per call of fn() from HIP events on torch's current stream
    (the stream every library call is given).  Eager launches: includes the
    host's launch rate when kernels are shorter than a Python call."""
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(iters):
        fn(i)
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


# HBM bytes per launch of the fused c3 step kernel, measured with rocprofv3
# FETCH_SIZE / WRITE_SIZE and scaled by a copy kernel of known size (the
# summary with the commands is profiles/decode_step_c3_traffic.md); to be
# re-measured whenever the decode kernel changes.
C3_STEP_TRAFFIC_BYTES = 35_169_893
# The same for the c5 step kernel (column-major bf16 caches) and for one c4
# prefill (kv_prologue_kernel + prefill_mfma_kernel + the gated fallback pass):
# profiles/decode_step_c5_traffic.md, profiles/prefill_c4_mfma_util_and_traffic.md.
C5_STEP_TRAFFIC_BYTES = 1_116_977_918
C4_PREFILL_TRAFFIC_BYTES = 211_350_387


def capture(torch, fn, n, first=0):
    """Captures n calls fn(first), fn(first+1), ... into one HIP graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(first)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(first + i)
    torch.cuda.synchronize()
    return g


def graph_time_ms(torch, fn, n_inner=64, replays=8):
    """Average ms per fn() call: n_inner calls captured in a HIP graph, the
    graph replayed `replays` times between HIP events on the current stream."""
    g = capture(torch, fn, n_inner)
    g.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(replays):
        g.replay()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / (replays * n_inner)


# ---------------------------------------------------------------------------
# Decode (c3 headline, c5 extra)
# ---------------------------------------------------------------------------
class DecodeWorkload:
    def __init__(self, torch, A, B, hq, hkv, d, prev, kv_dtype, sigma, base, n_sets, qknorm, seed,
                 kv_layout=0):
        self.t, self.A = torch, A
        self.B, self.hq, self.hkv, self.d, self.prev = B, hq, hkv, d, prev
        self.L = prev + 1
        self.max_len = (self.L + 63) // 64 * 64  # cache columns: allocation rounded to 64
        g = torch.Generator(device="cuda").manual_seed(seed)
        n = B * hkv * d * self.max_len
        cast = (lambda x: x.to(kv_dtype).view(torch.uint8)) if kv_dtype == torch.float8_e4m3fn \
            else (lambda x: x.to(kv_dtype))  # fp8: e4m3 bytes
        self.kc = [cast(torch.randn(n, generator=g, device="cuda") * sigma) for _ in range(n_sets)]
        self.vc = [cast(torch.randn(n, generator=g, device="cuda") * sigma) for _ in range(n_sets)]
        self.table = None
        if kv_layout == 2:  # same values in a page pool, through a shuffled block table
            nt = self.max_len // 32
            perm = torch.randperm(B * nt, generator=torch.Generator().manual_seed(seed))
            self.table = perm.reshape(B, nt).to(torch.int32).cuda()
            self.kc = [A.kv_to_paged(c, hkv, d, self.max_len, self.table, B * nt) for c in self.kc]
            self.vc = [A.kv_to_paged(c, hkv, d, self.max_len, self.table, B * nt) for c in self.vc]
        elif kv_layout:  # same values, stored as 32-column tiles
            self.kc = [A.kv_to_tiled(c, hkv, d, self.max_len) for c in self.kc]
            self.vc = [A.kv_to_tiled(c, hkv, d, self.max_len) for c in self.vc]
        self.kv_layout = kv_layout
        self.q = torch.randn(B * hq * d, generator=g, device="cuda") * sigma
        self.k = torch.randn(B * hkv * d, generator=g, device="cuda") * sigma
        self.v = torch.randn(B * hkv * d, generator=g, device="cuda") * sigma
        self.wq = self.wk = None
        if qknorm:
            self.wq = torch.rand(d, generator=g, device="cuda") + 0.5
            self.wk = torch.rand(d, generator=g, device="cuda") + 0.5
        self.base = base
        self.out = torch.empty(B * hq * d, device="cuda")
        self.args = [A.decode_args(self.q, kc, vc, self.out, hq, hkv, d, self.max_len, self.L,
                                   kv_layout=kv_layout, block_table=self.table)
                     for kc, vc in zip(self.kc, self.vc)]
        self.ws = A.decode_workspace(self.args[0])
        self.rs = [A.rope_store_args(self.q, self.k, self.v, kc, vc, hq, hkv, d, self.max_len, prev,
                                     base, q_norm_w=self.wq, k_norm_w=self.wk, eps=1e-6,
                                     kv_layout=kv_layout, block_table=self.table)
                   for kc, vc in zip(self.kc, self.vc)]
        self.step_ws = A.decode_step_workspace(self.rs[0], self.args[0])
        self.kv_bytes = 2 * B * hkv * d * self.L * self.kc[0].element_size()  # columns < L
        self.flops = 4 * B * hq * d * self.L

    def rope_store(self, i):
        s = i % len(self.kc)
        self.A.rope_store_decode(self.q, self.k, self.v, self.kc[s], self.vc[s], self.hq, self.hkv,
                                 self.d, self.max_len, self.prev, self.base, q_norm_w=self.wq,
                                 k_norm_w=self.wk, eps=1e-6, kv_layout=self.kv_layout,
                                 block_table=self.table)

    def attend(self, i):
        self.A.attn_decode(self.args[i % len(self.args)], self.ws)

    def two_calls(self, i):
        self.rope_store(i)
        self.attend(i)

    def step(self, i):
        """One fused launch: qkNorm + RoPE + cache store + attention."""
        s = i % len(self.args)
        self.A.decode_step(self.rs[s], self.args[s], self.step_ws)


def bench_decode(torch, A, wl, steps, warmup):
    """Returns a dict of ms: the timed step (host clock), the step kernel
    (HIP events over a graph of steps), attention alone, rope+store alone,
    the two-call step, and the eager step.

    The W warmup and K timed steps are each captured into a HIP graph (as a
    serving loop would run them); the timed graph is bracketed by
    synchronize() on both sides and timed with the host clock."""
    gw = capture(torch, wl.step, warmup)
    gt = capture(torch, wl.step, steps, first=warmup)
    gw.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gt.replay()
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"step": step_ms, "kernel": graph_time_ms(torch, wl.step),
            "attn": graph_time_ms(torch, wl.attend), "rope_store": graph_time_ms(torch, wl.rope_store),
            "two_calls": graph_time_ms(torch, wl.two_calls),
            "eager": event_time_ms(torch, wl.step, 20)}


# ---------------------------------------------------------------------------
# Prefill (c4)
# ---------------------------------------------------------------------------
class PrefillWorkload:
    """c4's prefill; the KV cache in kv_layout (None: the layout the library
    recommends for a bf16 cache of T columns, hl_kv_cache_preferred_layout,
    which a backend's initKvCache allocates)."""
    def __init__(self, torch, A, T=4096, hq=32, hkv=8, d=128, base=5e5, seed=7, kv_layout=None):
        g = torch.Generator(device="cuda").manual_seed(seed)
        bf = torch.bfloat16
        self.q = torch.randn(hq * d, T, generator=g, device="cuda").to(bf)
        self.k = torch.randn(hkv * d, T, generator=g, device="cuda").to(bf)
        self.v = torch.randn(hkv * d, T, generator=g, device="cuda").to(bf)
        self.kc = torch.empty(hkv * d, T, dtype=bf, device="cuda")
        self.vc = torch.empty(hkv * d, T, dtype=bf, device="cuda")
        self.out = torch.empty(hq * d, T, dtype=torch.float32, device="cuda")  # fp32 like act1
        if kv_layout is None:
            kv_layout = int(A._lib.load().hl_kv_cache_preferred_layout(A.HL_BF16, T))
        self.kv_layout = kv_layout
        self.a = A.prefill_args(self.q, self.k, self.v, self.out, hq, hkv, d, T, apply_rope=True,
                                rope_base=base, k_cache=self.kc, v_cache=self.vc, max_len=T,
                                kv_layout=kv_layout)
        self.ws = A.workspace(A.prefill_workspace_bytes(self.a))
        self.A = A
        self.flops = 4 * hq * d * T * (T + 1) // 2

    def step(self, i):
        self.A.attn_prefill(self.a, self.ws)


# ---------------------------------------------------------------------------
# CPU baseline: the C oracle on this host, one thread
# ---------------------------------------------------------------------------
def cpu_baseline(budget_s=12.0):
    import oracle
    oracle.lib()
    B, hq, hkv, d, L = 8, 32, 8, 64, 2049
    per = hkv * d * L
    kb = oracle.to_storage(oracle.normal(B * per, 1, 0, 0.5), oracle.F16)
    vb = oracle.to_storage(oracle.normal(B * per, 2, 0, 0.5), oracle.F16)
    q = oracle.normal(B * hq * d, 3, 0, 0.5)
    kf = oracle.upcast(kb, oracle.F16)
    vf = oracle.upcast(vb, oracle.F16)
    steps, t_total = 0, 0.0
    while t_total < budget_s:
        t0 = time.perf_counter()
        for b in range(B):
            oracle.attention_decode(q[b * hq * d:(b + 1) * hq * d], kf[b * per:(b + 1) * per],
                                    vf[b * per:(b + 1) * per], hq, hkv, d, L, L)
        t_total += time.perf_counter() - t0
        steps += 1
    kv_bytes = 2 * B * per * 2
    return {
        "value": round(kv_bytes * steps / t_total / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{steps} full c3 decode steps (8 seqs x 32 heads x 2049 cols, fp16 bits "
                  f"upcast to fp32) through the scalar C oracle, {t_total:.1f} s on 1 thread",
        "ms_per_step": round(t_total * 1e3 / steps, 3),
        "host_nproc": os.cpu_count(),
    }


def cpu_baseline_prefill():
    """The c4 prefill's attention on the scalar C oracle, one thread, on a
    bounded sample: query head 0 (kv head 0) over all 4096 causal rows, the
    same bf16-stored N(0,1) inputs upcast to fp32.  The full prefill is 32
    such heads; the rate is the sample's causal FLOPs / its time (RoPE and
    the cache write, a few percent of the work, are not timed)."""
    import oracle
    oracle.lib()
    T, hq, hkv, d = 4096, 32, 8, 128
    up = lambda n, seed: oracle.upcast(oracle.to_storage(oracle.normal(n, seed), oracle.BF16), oracle.BF16)
    # head 0 reads rows 0 .. d-1 of q and kv head 0's rows of k, v: only
    # those rows are generated (the other rows are never read)
    q = np.zeros((hq * d, T), np.float32)
    q[:d] = up(d * T, 41).reshape(d, T)
    k = np.zeros((hkv * d, T), np.float32)
    v = np.zeros((hkv * d, T), np.float32)
    k[:d] = up(d * T, 42).reshape(d, T)
    v[:d] = up(d * T, 43).reshape(d, T)
    t0 = time.perf_counter()
    oracle.attention_prefill(q, k, v, hq, hkv, d, T, heads=(0, 1))
    dt = time.perf_counter() - t0
    flops = 4 * d * T * (T + 1) // 2  # one head
    return {
        "value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
        "sample": f"c4 query head 0 of 32, all {T} causal rows (D=128, bf16-stored inputs as fp32) "
                  f"through the scalar C oracle, {dt:.1f} s on 1 thread; the full c4 prefill is "
                  f"32 such heads ({32 * dt:.0f} s at this rate)",
        "full_prefill_s_estimate": round(32 * dt, 1),
    }


def decode_extra(wl, t, workload):
    """Extra decode object: host-clock step rate, step-kernel roofline."""
    ach = wl.kv_bytes / (t["kernel"] * 1e-3) / 1e9
    return {
        "workload": workload,
        "kv_layout": {0: "colmajor (reference)", 1: "tiled32", 2: "paged32"}[wl.kv_layout],
        "kv_dtype": {1: "fp8 e4m3", 2: "bf16/fp16"}.get(wl.kc[0].element_size(), "fp32"),
        "value": round(wl.kv_bytes / (t["step"] * 1e-3) / 1e9, 2), "unit": "GB/s",
        "ms_per_step": round(t["step"], 5),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": wl.kv_bytes, "avg_us": round(t["kernel"] * 1e3, 3)},
        "attention_only_us": round(t["attn"] * 1e3, 3),
        "attention_only_frac": round(wl.kv_bytes / (t["attn"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "two_call_step_us": round(t["two_calls"] * 1e3, 3),
    }


# ---------------------------------------------------------------------------
# fp32 linear layer (gpuLinearCol drop-in): the projections around attention
# ---------------------------------------------------------------------------
def bench_linear(torch, A):
    """hl_gpu_linear_col at the projection shapes of the configs' models.
    Decode (seq_len 1): GB/s over the weight bytes (+ x, y), weights rotated
    over > 512 MB of copies so every call reads them from HBM.  Prefill:
    TFLOP/s on 2*M*K*T against the fp32 peak."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(13)
    for name, M, K in (("decode_tinyllama_q", 2048, 2048), ("decode_llama8b_q", 4096, 4096),
                       ("decode_llama8b_kv", 1024, 4096), ("decode_llama8b_ffn_up", 14336, 4096)):
        wbytes = M * K * 4
        n = max(2, -(-(600 << 20) // wbytes))
        ws = [torch.rand(M, K, generator=g, device="cuda") for _ in range(n)]
        x = torch.randn(K, generator=g, device="cuda")
        y = torch.empty(M, device="cuda")
        fn = lambda i: A.gpu_linear_col(y, x, ws[i % n], K, M, 1)
        ms = graph_time_ms(torch, fn, n_inner=max(n, 16), replays=4)
        nbytes = wbytes + (K + M) * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"shape": f"W {M}x{K} fp32, T=1", "us": round(ms * 1e3, 3), "unit": "GB/s",
                     "value": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                     "weight_copies": n}
        log(f"linear {name}: {ms*1e3:.2f} us, {gbs:.0f} GB/s")
        del ws
    for name, M, K, T in (("prefill_tinyllama_q_c2", 2048, 2048, 512),
                          ("prefill_llama8b_q_c4", 4096, 4096, 4096)):
        w = torch.rand(M, K, generator=g, device="cuda")
        x = torch.randn(K, T, generator=g, device="cuda")
        y = torch.empty(M, T, device="cuda")
        fn = lambda i: A.gpu_linear_col(y, x, w, K, M, T)
        ms = graph_time_ms(torch, fn, n_inner=8, replays=4)
        tf = 2.0 * M * K * T / (ms * 1e-3) / 1e12
        out[name] = {"shape": f"W {M}x{K} x X {K}x{T} fp32", "us": round(ms * 1e3, 2),
                     "unit": "TFLOP/s", "value": round(tf, 2),
                     "frac_fp32_peak": round(tf / FP32_PEAK_TFLOPS, 4)}
        log(f"linear {name}: {ms*1e3:.1f} us, {tf:.1f} TFLOP/s")
        del w, x, y
    # Quantized decode GEMV (gpuLinearColQuant drop-in): GB/s over the packed
    # weight bytes (+ x, y).  Weights are random bytes of the packed size:
    # the kernel has no data-dependent branches, so the rate does not depend
    # on the values.
    for qname, qt, qk, qb in (("f16", 1, 1, 2), ("q8_0", 8, 32, 34), ("q4_k", 12, 256, 144),
                              ("q6_k", 14, 256, 210), ("q5_k", 13, 256, 176),
                              ("q5_0", 6, 32, 22), ("q5_1", 7, 32, 24), ("q2_k", 10, 256, 84),
                              ("q3_k", 11, 256, 110), ("iq4_nl", 20, 32, 18)):
        for sname, M, K in (("llama8b_q", 4096, 4096), ("llama8b_ffn_up", 14336, 4096)):
            wbytes = M * K // qk * qb
            n = max(2, -(-(600 << 20) // wbytes))
            ws = [torch.randint(0, 256, (wbytes,), generator=g, device="cuda", dtype=torch.uint8)
                  for _ in range(n)]
            x = torch.randn(K, generator=g, device="cuda")
            y = torch.empty(M, device="cuda")
            fn = lambda i: A.gpu_linear_col_quant(y, x, ws[i % n], K, M, qt)
            ms = graph_time_ms(torch, fn, n_inner=max(n, 16), replays=4)
            gbs = (wbytes + (K + M) * 4) / (ms * 1e-3) / 1e9
            name = f"decode_{sname}_{qname}"
            out[name] = {"shape": f"W {M}x{K} {qname}, T=1", "us": round(ms * 1e3, 3),
                         "unit": "GB/s", "value": round(gbs, 1),
                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "weight_copies": n}
            log(f"linear {name}: {ms*1e3:.2f} us, {gbs:.0f} GB/s")
            del ws
    torch.cuda.empty_cache()
    return out


MODEL_SHAPES = {
    "llama-3-8b": dict(n_layer=32, n_emb=4096, n_head=32, n_head_kv=8, head_dim=128, rope_dim=128,
                       n_ff=14336, n_vocab=128256, max_len=512, rms_eps=1e-5, rope_base=5e5),
    # the model of the reference's own decode benchmark (Llama-3.2-1B Q4_K_M)
    "llama-3.2-1b": dict(n_layer=16, n_emb=2048, n_head=32, n_head_kv=8, head_dim=64, rope_dim=64,
                         n_ff=8192, n_vocab=128256, max_len=512, rms_eps=1e-5, rope_base=5e5),
}


def bench_models(torch):
    return {name: bench_model(torch, name, cfg) for name, cfg in MODEL_SHAPES.items()}


def bench_model(torch, name, cfg):
    """Greedy decode of a dense decoder of the given shape through
    hl_forward_decode_token: Q4_K layer weights, Q6_K output head, fp32
    embedding, fp32 caches of 512 positions.  Weights are random bytes with
    their fp16 block scales set to 5e-4 (finite, moderate activations).
    Tokens chain on the device; the time is the host clock over 16 tokens
    after 3 warm-up tokens (positions 3..18)."""
    import numpy as np
    from hippo_leap_amd.model import DenseDecoder
    E, ff, kv = cfg["n_emb"], cfg["n_ff"], cfg["n_head_kv"] * cfg["head_dim"]
    g = torch.Generator(device="cuda").manual_seed(23)
    half = torch.from_numpy(np.array([5e-4], np.float16).view(np.uint8).copy()).cuda()

    def gguf(rows, cols, bb, scale_at):
        nb = rows * cols // 256
        w = torch.randint(0, 256, (nb, bb), generator=g, device="cuda", dtype=torch.uint8)
        for o in scale_at:
            w[:, o:o + 2] = half
        return w.reshape(-1)

    q4 = lambda r, c: gguf(r, c, 144, (0, 2))  # d, dmin
    layers, wbytes = [], 0
    for _ in range(cfg["n_layer"]):
        L = {"attn_norm": torch.ones(E, device="cuda"), "ffn_norm": torch.ones(E, device="cuda"),
             "wq": q4(E, E), "wk": q4(kv, E), "wv": q4(kv, E), "wo": q4(E, E),
             "w_gate": q4(ff, E), "w_up": q4(ff, E), "w_down": q4(E, ff),
             "k_cache": torch.zeros(kv, cfg["max_len"], device="cuda"),
             "v_cache": torch.zeros(kv, cfg["max_len"], device="cuda")}
        for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            L[n + "_type"] = 12
            wbytes += L[n].numel()
        layers.append(L)
    out = gguf(cfg["n_vocab"], E, 210, (208,))
    wbytes += out.numel()
    emb = torch.randn(cfg["n_vocab"], E, generator=g, device="cuda")
    m = DenseDecoder(torch, cfg, emb, torch.ones(E, device="cuda"), out, 14, layers)
    toks = torch.zeros(20, dtype=torch.int32, device="cuda")
    toks[0] = 128000
    for p in range(3):
        m.step(p, toks[p:p + 1], toks[p + 1:p + 2])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for p in range(3, 19):
        m.step(p, toks[p:p + 1], toks[p + 1:p + 2])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / 16
    valid = bool(((toks[1:] >= 0) & (toks[1:] < cfg["n_vocab"])).all().item())
    # The same 16 steps captured in one HIP graph and replayed (a serving
    # loop's form: no per-kernel host launch cost), host clock per replay.
    graph_ms = None
    try:
        st = torch.cuda.Stream()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            with torch.cuda.graph(gr, stream=st):
                for p in range(3, 19):
                    m.step(p, toks[p:p + 1], toks[p + 1:p + 2])
        gr.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(4):
            gr.replay()
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - t0) * 1e3 / 64
    except Exception as e:  # noqa: BLE001 - reported, not fatal
        log(f"model decode {name}: graph capture failed: {e}")
    res = {"model": f"{name} shape, Q4_K layers, Q6_K head (random weights)", "ms_per_token": round(ms, 3),
           "tokens_per_s": round(1e3 / ms, 1), "weight_bytes": wbytes,
           "weight_GB_per_s": round(wbytes / (ms * 1e-3) / 1e9, 1), "positions": "3..18",
           "tokens_in_vocab": valid}
    if graph_ms is not None:
        res["graph_ms_per_token"] = round(graph_ms, 3)
        res["graph_weight_GB_per_s"] = round(wbytes / (graph_ms * 1e-3) / 1e9, 1)
    # The backend contract over a cache descriptor (hl_forward_decode): the
    # same weights, a bf16 KV cache in the library's preferred (tiled)
    # layout, so each layer's qk-norm + RoPE + cache write + attention is one
    # fused launch; positions 3..18 as above, and 2048..2063 (an 8K cache,
    # attention over ~2K columns).
    try:
        from hippo_leap_amd import _lib as L_
        from hippo_leap_amd.model import DenseModel, KvCache
        cfg2 = dict(cfg, max_len=8192)
        dm = DenseModel(torch, cfg2, emb, torch.ones(E, device="cuda"), out, 14, layers, kv_dtype=L_.HL_BF16)
        for start, key in ((3, "fused_ms_per_token"), (2048, "fused_ms_per_token_at_2k")):
            dm.cache.desc.cur_len = start - 3
            for p in range(start - 3, start):
                dm.decode(toks[0:1], toks[1:2])
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for p in range(16):
                dm.decode(toks[0:1], toks[1:2])
            torch.cuda.synchronize()
            res[key] = round((time.perf_counter() - t0) * 1e3 / 16, 3)
        res["fused_kv_cache"] = f"bf16, layout {int(dm.cache.desc.kv_layout)} (1 = tiled32), max_len 8192"
        del dm
    except Exception as e:  # noqa: BLE001 - reported, not fatal
        log(f"model decode {name}: descriptor path failed: {e}")
    log(f"model decode {name}: {ms:.3f} ms/token, {1e3 / ms:.1f} tokens/s, "
        f"{res['weight_GB_per_s']} GB/s of weights")
    del m, layers, emb, out
    torch.cuda.empty_cache()
    return res


def bench_ends(torch, A):
    """The decode step's ends: greedy argmax over a vocabulary of logits
    (hl_argmax_async, result left on the device as in a captured decode loop;
    hl_gpu_argmax adds a device-to-host copy and a stream wait) and the token
    embedding lookup (one token; a 4096-token prefill)."""
    out = {}
    g = torch.Generator(device="cuda").manual_seed(17)
    res = torch.empty(1, dtype=torch.int32, device="cuda")
    for name, n in (("argmax_llama3_vocab", 128256), ("argmax_qwen3_vocab", 151936)):
        xs = [torch.randn(n, generator=g, device="cuda") for _ in range(64)]
        A.argmax_async(xs[0], n, res)
        ms = graph_time_ms(torch, lambda i: A.argmax_async(xs[i % 64], n, res), 64, 4)
        t0 = time.perf_counter()
        for i in range(50):
            A.gpu_argmax(xs[i % 64], n)
        host_ms = (time.perf_counter() - t0) / 50 * 1e3
        out[name] = {"n": n, "us": round(ms * 1e3, 3), "unit": "GB/s",
                     "value": round(n * 4 / (ms * 1e-3) / 1e9, 1),
                     "with_host_result_us": round(host_ms * 1e3, 1)}
        log(f"{name}: {ms*1e3:.2f} us in a graph, {host_ms*1e3:.1f} us with the host result")
        del xs
    for name, n_emb, n_tok in (("embedding_decode_llama8b", 4096, 1),
                               ("embedding_prefill_llama8b_t4096", 4096, 4096)):
        n_vocab = 128256
        w = torch.randn(n_vocab, n_emb, generator=g, device="cuda")
        toks = [torch.randint(0, n_vocab, (n_tok,), generator=g, device="cuda",
                              dtype=torch.int32) for _ in range(16)]
        o = torch.empty(n_emb, n_tok, device="cuda")
        ms = graph_time_ms(torch, lambda i: A.gpu_embedding(o, w, toks[i % 16], n_emb, n_tok,
                                                            n_vocab), 16, 4)
        nbytes = 2 * n_emb * n_tok * 4
        out[name] = {"n_emb": n_emb, "n_tokens": n_tok, "us": round(ms * 1e3, 3), "unit": "GB/s",
                     "value": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        log(f"{name}: {ms*1e3:.2f} us")
        del w
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["all", "decode", "prefill", "c5", "fp32", "linear", "model"],
                    default="all")
    ap.add_argument("--layouts", choices=["both", "colmajor", "tiled"], default="both",
                    help="KV-cache layouts of the decode runs (the headline c3 line is column-major; "
                         "one layout per run keeps a profiler's per-kernel averages to one layout)")
    ap.add_argument("--calib", action="store_true",
                    help="also run a 256 MiB -> 256 MiB elementwise copy (3x): the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is designed but not built)"}))
        sys.exit(2)

    import torch
    from hippo_leap_amd import attention as A
    torch.cuda.init()
    info = A.device_info()
    log(f"device: {info['arch']} CUs={info['cu_count']} clk={info['clock_khz']} kHz")

    if args.calib:  # an elementwise kernel that reads and writes 256 MiB each
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

    result = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
              "data": "synthetic (seeded torch.randn on the GPU, random values of the "
                      "configs' shapes/distributions)"}

    if args.only in ("all", "decode") and args.layouts != "tiled":
        log("decode c3 ...")
        wl = DecodeWorkload(torch, A, B=8, hq=32, hkv=8, d=64, prev=2048,
                            kv_dtype=torch.float16, sigma=0.5, base=5e5, n_sets=16,
                            qknorm=False, seed=3)
        t = bench_decode(torch, A, wl, args.steps, args.warmup)
        step_ms = t["step"]
        value = wl.kv_bytes / (step_ms * 1e-3) / 1e9
        achieved = wl.kv_bytes / (t["kernel"] * 1e-3) / 1e9
        result.update({
            "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(step_ms, 5),
            "dtype": "f16",
            "config": {"workload": "c3: Llama-3.2-1B-shape batched decode, fp16 KV", "batch": 8,
                       "cached_positions": 2048, "attn_len": 2049, "n_head": 32, "n_head_kv": 8,
                       "head_dim": 64, "rope_theta": 5e5, "kv_sigma": 0.5,
                       "rotating_cache_sets": 16,
                       "step": "hl_decode_step (qkNorm/RoPE + KV store + split-K attention, "
                               "one launch)"},
            "roofline": {"bound": "hbm", "kernel": "decode_mfma_kernel (fused step)",
                         "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": C3_STEP_TRAFFIC_BYTES,
                         "traffic_source": "profiles/decode_step_c3_traffic.md: rocprofv3 "
                                           "FETCH_SIZE x 1.99981 + WRITE_SIZE x 1.0 per launch",
                         "algorithmic_bytes": wl.kv_bytes,
                         "avg_us": round(t["kernel"] * 1e3, 3)},
            "attention_only_us": round(t["attn"] * 1e3, 3),
            "rope_store_only_us": round(t["rope_store"] * 1e3, 3),
            "two_call_step_us": round(t["two_calls"] * 1e3, 3),
            "eager_ms_per_step": round(t["eager"], 5),
        })
        # Cache-resident ("warm") figure, labelled as such: one cache set
        # (33.6 MB) replayed, so its K/V stay in the 256 MB MALL.
        warm_ms = graph_time_ms(torch, lambda i: wl.step(0))
        # The floor of any one kernel that reads 33.6 MB: a plain streaming
        # read of the same byte count (16 rotating buffers, past the MALL),
        # at a few grid sizes; the best is the floor the step is compared to.
        bufs = [torch.empty(wl.kv_bytes, dtype=torch.uint8, device="cuda") for _ in range(16)]
        for b_ in bufs:
            b_.fill_(1)
        sink = torch.zeros(4, dtype=torch.int32, device="cuda")
        # Grid sizes x loads in flight per thread x (grid-stride, contiguous
        # chunk per workgroup); the best of all is the floor.
        floor = {}
        for nblk in (256, 512, 1024, 2048, 4096):
            for ipt in (4, 8, 16):
                for contig in (0, 1):
                    floor[f"{nblk}x{ipt}{'c' if contig else 'g'}"] = graph_time_ms(
                        torch, lambda i, nb=nblk, f=ipt, c=contig: A.probe_stream_read(
                            bufs[i % 16], sink, nb, inflight=f, contiguous=bool(c)))
        best = min(floor.values())
        best_cfg = min(floor, key=floor.get)
        result["stream_floor_c3"] = {
            "bytes": wl.kv_bytes, "us": round(best * 1e3, 3),
            "GBs": round(wl.kv_bytes / (best * 1e-3) / 1e9, 1),
            "frac_hbm": round(wl.kv_bytes / (best * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "best_config": best_cfg,
            "us_by_config": {k: round(v * 1e3, 3) for k, v in floor.items()},
            "config_key": "<workgroups>x<loads in flight per thread><g: grid-stride | c: chunk per workgroup>",
            "step_kernel_over_floor": round(t["kernel"] / best, 3),
            "note": "hl_probe_stream_read: one launch that only streams the c3 byte count"}
        log(f"stream floor c3: {best*1e3:.2f} us ({wl.kv_bytes / (best * 1e-3) / 1e9:.0f} GB/s); "
            f"best {best_cfg}; {', '.join(f'{k}: {v*1e3:.2f}' for k, v in floor.items())}")
        del bufs
        result["warm_cache_resident"] = {
            "value": round(wl.kv_bytes / (warm_ms * 1e-3) / 1e9, 2), "unit": "GB/s",
            "ms_per_step": round(warm_ms, 5),
            "note": "same step kernel on one cache set, K/V resident in the MALL; not HBM-bound"}
        log(f"decode c3: step {step_ms*1e3:.2f} us, step kernel {t['kernel']*1e3:.2f} us "
            f"({achieved:.0f} GB/s), attention alone {t['attn']*1e3:.2f} us, rope+store "
            f"{t['rope_store']*1e3:.2f} us, two calls {t['two_calls']*1e3:.2f} us")
        del wl
        torch.cuda.empty_cache()
    if args.only in ("all", "decode") and args.layouts != "colmajor":
        log("decode_c3_tiled ...")
        wl = DecodeWorkload(torch, A, B=8, hq=32, hkv=8, d=64, prev=2048,
                            kv_dtype=torch.float16, sigma=0.5, base=5e5, n_sets=16,
                            qknorm=False, seed=3, kv_layout=1)
        t = bench_decode(torch, A, wl, args.steps, args.warmup)
        result["decode_c3_tiled"] = decode_extra(wl, t, "c3 step, caches in the tiled layout")
        log(f"decode_c3_tiled: step {t['step']*1e3:.2f} us, step kernel {t['kernel']*1e3:.2f} us")
        del wl
        torch.cuda.empty_cache()
        log("decode_c3_fp8 ...")
        wl = DecodeWorkload(torch, A, B=8, hq=32, hkv=8, d=64, prev=2048,
                            kv_dtype=torch.float8_e4m3fn, sigma=0.5, base=5e5, n_sets=16,
                            qknorm=False, seed=3, kv_layout=1)
        t = bench_decode(torch, A, wl, args.steps, args.warmup)
        result["decode_c3_fp8"] = decode_extra(wl, t, "c3 step, fp8 e4m3 caches in the tiled "
                                               "layout (half the bytes)")
        log(f"decode_c3_fp8: step {t['step']*1e3:.2f} us, step kernel {t['kernel']*1e3:.2f} us")
        del wl
        torch.cuda.empty_cache()

    if args.only in ("all", "fp32"):
        # The reference-contract fp32 path (configs[0] decode, configs[1] prefill):
        # the entry points a Nim caller of gpuAttentionDecode / gpuAttentionPrefill hits.
        log("decode c1 / prefill c2 (fp32) ...")
        g = torch.Generator(device="cuda").manual_seed(11)
        n1 = 4 * 64 * 512
        sets = [(torch.rand(n1, generator=g, device="cuda") * 2 - 1,
                 torch.rand(n1, generator=g, device="cuda") * 2 - 1) for _ in range(256)]
        q1 = torch.rand(32 * 64, generator=g, device="cuda") * 2 - 1
        o1 = torch.empty_like(q1)
        lib = A._lib.load()
        st = lambda: torch.cuda.current_stream().cuda_stream
        c1 = lambda i: A.check(lib.hl_gpu_attention_decode(
            o1.data_ptr(), q1.data_ptr(), sets[i % 256][0].data_ptr(), sets[i % 256][1].data_ptr(),
            32, 4, 64, 512, 512, st()))
        ms1 = graph_time_ms(torch, c1, 256, 4)
        b1 = 2 * n1 * 4
        result["decode_c1"] = {
            "workload": "c1: TinyLlama-shape decode, fp32 KV, B=1, Hq32/Hkv4, D64, L=512 "
                        "(hl_gpu_attention_decode, the reference's call contract; 256 rotating "
                        "cache sets = 268 MB)",
            "us": round(ms1 * 1e3, 3), "unit": "GB/s", "value": round(b1 / (ms1 * 1e-3) / 1e9, 1),
            "frac_hbm": round(b1 / (ms1 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "1 MB per call: launch- and latency-bound"}
        T2 = 512
        q2 = torch.randn(32 * 64, T2, generator=g, device="cuda")
        k2 = torch.randn(4 * 64, T2, generator=g, device="cuda")
        v2 = torch.randn(4 * 64, T2, generator=g, device="cuda")
        kc2 = torch.empty(4 * 64, T2, device="cuda")
        vc2 = torch.empty(4 * 64, T2, device="cuda")
        o2 = torch.empty(32 * 64, T2, device="cuda")
        a2 = A.prefill_args(q2, k2, v2, o2, 32, 4, 64, T2, rope_base=1e4, apply_rope=True,
                            k_cache=kc2, v_cache=vc2, max_len=T2)
        ws2 = A.workspace(A.prefill_workspace_bytes(a2))
        ms2 = graph_time_ms(torch, lambda i: A.attn_prefill(a2, ws2), 32, 4)
        f2 = 4 * 32 * 64 * T2 * (T2 + 1) // 2
        result["prefill_c2"] = {
            "workload": "c2: TinyLlama-shape causal prefill, fp32, T=512, Hq32/Hkv4, D64, RoPE 1e4, "
                        "KV cache written (prologue + split-operand flash kernel)",
            "us": round(ms2 * 1e3, 3), "unit": "TFLOP/s",
            "value": round(f2 / (ms2 * 1e-3) / 1e12, 3),
            "frac_fp32_peak": round(f2 / (ms2 * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4)}
        log(f"decode c1: {ms1*1e3:.2f} us; prefill c2: {ms2*1e3:.1f} us "
            f"({f2 / (ms2 * 1e-3) / 1e12:.2f} TFLOP/s)")
        del sets
        # The same fp32 contract at the Llama-3-8B attention shape (head dim
        # 128, T=4096): what gpuAttentionPrefill of the reference's fp32
        # backend runs for that model.
        T8, hq8, hkv8, d8 = 4096, 32, 8, 128
        q8 = torch.randn(hq8 * d8, T8, generator=g, device="cuda")
        k8 = torch.randn(hkv8 * d8, T8, generator=g, device="cuda")
        v8 = torch.randn(hkv8 * d8, T8, generator=g, device="cuda")
        kc8 = torch.empty(hkv8 * d8, T8, device="cuda")
        vc8 = torch.empty(hkv8 * d8, T8, device="cuda")
        o8 = torch.empty(hq8 * d8, T8, device="cuda")
        a8 = A.prefill_args(q8, k8, v8, o8, hq8, hkv8, d8, T8, rope_base=5e5, apply_rope=True,
                            k_cache=kc8, v_cache=vc8, max_len=T8)
        ws8 = A.workspace(A.prefill_workspace_bytes(a8))
        ms8 = graph_time_ms(torch, lambda i: A.attn_prefill(a8, ws8), 8, 4)
        f8 = 4 * hq8 * d8 * T8 * (T8 + 1) // 2
        result["prefill_fp32_llama8b"] = {
            "workload": "Llama-3-8B-shape causal prefill, fp32, T=4096, Hq32/Hkv8, D128, RoPE 5e5, "
                        "fp32 KV cache written (prologue + split-operand flash kernel)",
            "us": round(ms8 * 1e3, 1), "unit": "TFLOP/s",
            "value": round(f8 / (ms8 * 1e-3) / 1e12, 2),
            "frac_fp32_peak": round(f8 / (ms8 * 1e-3) / 1e12 / FP32_PEAK_TFLOPS, 4),
            "note": "the products run as three fp16 MFMAs on hi/lo splits, hence above the fp32 peak"}
        log(f"prefill fp32 Llama-3-8B shape: {ms8*1e3:.1f} us ({f8 / (ms8 * 1e-3) / 1e12:.1f} TFLOP/s)")
        del q8, k8, v8, kc8, vc8, o8, ws8
        torch.cuda.empty_cache()

    if args.only in ("all", "prefill"):
        log("prefill c4 ...")
        pw = PrefillWorkload(torch, A)
        for i in range(max(2, args.warmup // 2)):
            pw.step(i)
        torch.cuda.synchronize()
        # The same prefill writing a cache in the reference's column-major
        # layout, timed alternately with the preferred one in the order
        # preferred, column-major, column-major, preferred (the shader clock
        # ramps after a pause and drifts under sustained load, so a fixed
        # order favours one of them): each figure is the mean of its two runs.
        pc = PrefillWorkload(torch, A, kv_layout=A.HL_KV_COLMAJOR)
        pc.step(0)
        reps = max(2, args.steps // 40)
        runs = {"pref": [], "col": []}
        for key in ("pref", "col", "col", "pref"):
            runs[key].append(graph_time_ms(torch, pw.step if key == "pref" else pc.step, n_inner=8, replays=reps))
        ms, ms_col = sum(runs["pref"]) / 2, sum(runs["col"]) / 2
        tf = pw.flops / (ms * 1e-3) / 1e12
        del pc
        result["prefill"] = {
            "workload": "c4: Llama-3-8B-shape causal prefill bf16, T=4096, Hq32/Hkv8, D128, "
                        "RoPE 5e5, KV cache written",
            "dtype": "bf16 in, fp16 MFMA operands, fp32 accumulation and output",
            "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
            "kv_layout": {0: "colmajor", 1: "tiled32", 2: "paged32"}[pw.kv_layout] +
                         " (hl_kv_cache_preferred_layout for a bf16 cache)",
            "colmajor_cache": {"ms_per_step": round(ms_col, 4),
                               "value": round(pw.flops / (ms_col * 1e-3) / 1e12, 2),
                               "note": "the same prefill writing the reference's column-major "
                                       "[Hkv*D, max_len] cache"},
            "roofline": {"bound": "mfma", "kernel": "kv_prologue_kernel + prefill_mfma_kernel",
                         "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "traffic": C4_PREFILL_TRAFFIC_BYTES,
                         "traffic_source": "profiles/prefill_c4_mfma_util_and_traffic.md: "
                                           "FETCH_SIZE x 1.99981 + WRITE_SIZE of both kernels",
                         "mfma_util_at_actual_clock": 0.465,
                         "mfma_util_source": "same profile: SQ_VALU_MFMA_BUSY_CYCLES / "
                                             "(GRBM_GUI_ACTIVE per XCD x 1024 SIMDs)",
                         "algorithmic_flops": pw.flops},
        }
        if not args.no_cpu:
            log("cpu baseline (prefill sample) ...")
            cb = cpu_baseline_prefill()
            cb["gpu_over_cpu"] = round(tf / cb["value"], 1)
            result["prefill"]["cpu_baseline"] = cb
        log(f"prefill c4: {ms:.3f} ms, {tf:.1f} TFLOP/s (column-major cache: {ms_col:.3f} ms)")
        del pw
        torch.cuda.empty_cache()

    if args.only in ("all", "c5"):
        for layout, key, kvdt in ((0, "decode_c5", torch.bfloat16),
                                  (1, "decode_c5_tiled", torch.bfloat16),
                                  (1, "decode_c5_fp8", torch.float8_e4m3fn),
                                  (2, "decode_c5_paged", torch.bfloat16)):
            if args.layouts == ("tiled" if layout == 0 else "colmajor"):
                continue
            log(f"{key} ...")
            wl = DecodeWorkload(torch, A, B=16, hq=32, hkv=4, d=128, prev=32768,
                                kv_dtype=kvdt, sigma=1.0, base=1e6, n_sets=1 if kvdt == torch.bfloat16 else 2,
                                qknorm=True, seed=5, kv_layout=layout)
            t = bench_decode(torch, A, wl, args.steps, max(3, args.warmup))
            kvname = "fp8 e4m3" if kvdt == torch.float8_e4m3fn else "bf16"
            result[key] = decode_extra(wl, t, f"c5: Qwen3-30B-A3B-shape decode, {kvname} KV, B=16, "
                                       "L=32769, Hq32/Hkv4, D128, qkNorm + RoPE 1e6")
            if key == "decode_c5":
                result[key]["roofline"]["traffic"] = C5_STEP_TRAFFIC_BYTES
                result[key]["roofline"]["traffic_source"] = "profiles/decode_step_c5_traffic.md"
            log(f"{key}: step {t['step']*1e3:.1f} us, step kernel {t['kernel']*1e3:.1f} us "
                f"({result[key]['roofline']['achieved']:.0f} GB/s), attention alone "
                f"{t['attn']*1e3:.1f} us")
            del wl
            torch.cuda.empty_cache()

    if args.only in ("all", "linear"):
        result["linear"] = bench_linear(torch, A)
    if args.only in ("all", "model"):
        result["model_decode"] = bench_models(torch)
        result["decode_ends"] = bench_ends(torch, A)

    if not args.no_cpu:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline()
        if "value" in result:
            result["cpu_baseline"]["gpu_over_cpu"] = round(result["value"] /
                                                           result["cpu_baseline"]["value"], 1)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
