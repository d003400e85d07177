"""GPU parity of the decode-step ends: greedy argmax (hl_gpu_argmax,
hl_argmax_async; gpuArgmax, backends/naive.nim:1922-2127) and the token
embedding (hl_gpu_embedding; gpuEmbedding, naive.nim:2975-3001), against the
CPU oracle's literal restatements.  Bar: identical indices (ties, NaN and
-inf included) and bit-identical embeddings."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 7, 2048, 2049, 65537, 128256, 152064, 262144, 600001]


def gpu_argmax_both(x_np, offset=0):
    from hippo_leap_amd import attention as A
    buf = torch.zeros(x_np.size + offset, device="cuda")
    buf[offset:] = torch.from_numpy(x_np).cuda()
    x = buf[offset:]
    host = A.gpu_argmax(x, x_np.size)
    dev = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    A.argmax_async(x, x_np.size, dev)
    torch.cuda.synchronize()
    return host, int(dev.item())


@pytest.mark.parametrize("n", SIZES)
def test_argmax_matches_oracle(hl, orc, n):
    print(f"argmax n={n}", flush=True)
    x = orc.normal(n, 3600 + n % 997)
    ref = orc.argmax(x)
    assert gpu_argmax_both(x) == (ref, ref)


@pytest.mark.parametrize("n,levels", [(200000, 3), (70000, 2), (131072, 1), (65537, 1), (999, 2)])
def test_argmax_ties_match_oracle(hl, orc, n, levels):
    print(f"argmax ties n={n} levels={levels}", flush=True)
    x = np.random.default_rng(n + levels).integers(0, levels, n).astype(np.float32)
    ref = orc.argmax(x)
    assert gpu_argmax_both(x) == (ref, ref)
    assert gpu_argmax_both(x, offset=1) == (ref, ref)   # unaligned: scalar loads


def test_argmax_special_values(hl, orc):
    cases = [
        np.array([np.nan, -np.inf, -3.4e38, 1.0], np.float32),
        np.array([np.nan, -np.inf, -3.4e38], np.float32),
        np.array([-0.0, 0.0, -0.0], np.float32),
        np.full(5000, -np.inf, np.float32),
        np.full(70000, np.nan, np.float32),
    ]
    big = np.full(300000, -5.0, np.float32)
    big[::7] = np.nan
    big[[1234, 299999, 65536 + 1234]] = 3.0
    cases.append(big)
    for x in cases:
        ref = orc.argmax(x)
        assert gpu_argmax_both(x) == (ref, ref), x[:8]
    from hippo_leap_amd import attention as A
    empty = torch.zeros(4, device="cuda")
    assert A.gpu_argmax(empty, 0) == -1


def test_argmax_repeat_and_graph_replay(hl, orc):
    """The arrival counter resets itself: repeated calls of different sizes
    and HIP-graph replays (eager work in between) give the oracle's answer."""
    from hippo_leap_amd import attention as A
    xs = [orc.normal(n, 3700 + n) for n in (128256, 5000, 600001, 128256)]
    for x in xs:
        ref = orc.argmax(x)
        assert gpu_argmax_both(x) == (ref, ref)
    x = torch.from_numpy(xs[0]).cuda()
    ref = orc.argmax(xs[0])
    res = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    A.argmax_async(x, x.numel(), res)  # first call outside capture allocates the scratch
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        A.argmax_async(x, x.numel(), res)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        A.argmax_async(x, x.numel(), res)
    for _ in range(4):
        res.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(res.item()) == ref
        assert A.gpu_argmax(x, x.numel()) == ref


@pytest.mark.parametrize("n_emb,n_tok", [(2048, 1), (4096, 1), (100, 7), (4096, 300), (130, 65)])
def test_embedding_matches_oracle(hl, orc, n_emb, n_tok):
    from hippo_leap_amd import attention as A
    print(f"embedding n_emb={n_emb} n_tok={n_tok}", flush=True)
    n_vocab = 1000
    w = orc.normal(n_vocab * n_emb, 3800 + n_emb).reshape(n_vocab, n_emb)
    tok = np.random.default_rng(n_tok).integers(0, n_vocab, n_tok).astype(np.int32)
    tok[0] = n_vocab - 1
    out = torch.full((n_emb, n_tok), float("nan"), device="cuda")
    A.gpu_embedding(out, torch.from_numpy(w).cuda(), torch.from_numpy(tok).cuda(), n_emb, n_tok,
                    n_vocab)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), orc.embedding(w, tok, n_emb))


def test_embedding_out_of_range_token_is_nan(hl, orc):
    from hippo_leap_amd import attention as A
    n_vocab, n_emb = 10, 64
    w = torch.from_numpy(orc.normal(n_vocab * n_emb, 3900)).cuda()
    tok = torch.tensor([2, 10, -1, 9], dtype=torch.int32, device="cuda")
    out = torch.zeros(n_emb, 4, device="cuda")
    A.gpu_embedding(out, w, tok, n_emb, 4, n_vocab)
    o = out.cpu().numpy()
    assert np.isnan(o[:, 1]).all() and np.isnan(o[:, 2]).all()
    wn = w.cpu().numpy().reshape(n_vocab, n_emb)
    assert np.array_equal(o[:, 0], wn[2]) and np.array_equal(o[:, 3], wn[9])
