"""Shared helpers for the parity tests (tolerance metric, loaders)."""
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Tolerances from the north star: 1e-4 relative for fp32 KV, 2e-3 for fp16/bf16.
TOL_F32 = 1e-4
TOL_LOWP = 2e-3


def rel_err(got, ref) -> float:
    """max|got - ref| / max|ref| over the tensor (NaN anywhere -> inf)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
