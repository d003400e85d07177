"""GPU: hl_gpu_attention_decode_noalloc (the decode drop-in whose split-K
workspace is the library's static device scratch) against
hl_gpu_attention_decode, the existing entry point with the same kernels, and
against the oracle: two calls in a row, the second with a smaller input, then
a shape larger than the scratch (a clear error, nothing launched)."""
import ctypes

import numpy as np
import pytest
import torch

from util import TOL_F32, rel_err

pytestmark = pytest.mark.gpu


def _case(orc, hq, hkv, d, L, max_len, seed):
    n = hkv * d * max_len
    return orc.uniform(hq * d, seed), orc.uniform(n, seed + 1), orc.uniform(n, seed + 2)


def _call(hl, fn, q, kb, vb, hq, hkv, d, L, max_len):
    qd, kd, vd = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (q, kb, vb))
    dst = torch.full((hq * d,), float("nan"), device="cuda")
    rc = getattr(hl, fn)(dst.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), hq, hkv, d, L,
                         max_len, None)
    torch.cuda.synchronize()
    return rc, dst.cpu().numpy()


def test_noalloc_decode_matches_dropin(hl, orc):
    from hippo_leap_amd import _lib
    # a large shape first, then a smaller one (fewer heads, shorter context):
    # the second call reuses the scratch the first left behind; the third has
    # more (sequence, kv head) units, so its arrival counters reach past the
    # region earlier calls kept zero (the entry point clears it first)
    for hq, hkv, d, L, max_len, seed in ((32, 8, 128, 3000, 3008, 1500), (32, 4, 64, 512, 512, 1510),
                                         (128, 128, 64, 200, 256, 1520)):
        q, kb, vb = _case(orc, hq, hkv, d, L, max_len, seed)
        rc, got = _call(hl, "hl_gpu_attention_decode_noalloc", q, kb, vb, hq, hkv, d, L, max_len)
        assert rc == _lib.HL_OK, hl.hl_last_error()
        rc, ref_lib = _call(hl, "hl_gpu_attention_decode", q, kb, vb, hq, hkv, d, L, max_len)
        assert rc == _lib.HL_OK, hl.hl_last_error()
        assert rel_err(got, ref_lib) < TOL_F32, (hq, L)
        g = hq // hkv  # kv head 0's query heads against the oracle
        sub = orc.attention_decode(q[:g * d], kb[:d * max_len], vb[:d * max_len], g, 1, d, L, max_len)
        assert rel_err(got[:g * d], sub) < TOL_F32, (hq, L)
    # repeated: the scratch keeps the last call's contents and stays correct
    rc, again = _call(hl, "hl_gpu_attention_decode_noalloc", q, kb, vb, hq, hkv, d, L, max_len)
    assert rc == _lib.HL_OK and rel_err(again, ref_lib) < TOL_F32


def test_noalloc_decode_rejects_oversized_shape(hl):
    from hippo_leap_amd import _lib
    # 1024 query heads of 128 dims over 64 kv heads and a long context: the
    # split-K partials exceed the 1 MiB scratch.  The plan (the same one
    # hl_attn_decode_workspace_bytes reports for these args) is checked first,
    # so the call below is known to return before launching anything.
    fake = 1 << 20  # validation and planning never dereference the pointers
    hq, hkv, d, L = 1024, 64, 128, 65536
    a = _lib.DecodeArgs()
    a.batch, a.n_head, a.n_head_kv, a.head_dim = 1, hq, hkv, d
    a.kv_dtype, a.max_len, a.seq_len = _lib.HL_F32, L, L
    a.q = a.k_cache = a.v_cache = a.out = fake
    need = hl.hl_attn_decode_workspace_bytes(ctypes.byref(a))
    assert need > (1 << 20), need
    rc = hl.hl_gpu_attention_decode_noalloc(fake, fake, fake, fake, hq, hkv, d, L, L, None)
    assert rc == _lib.HL_ECAPACITY
    assert "scratch" in hl.hl_last_error().decode()
