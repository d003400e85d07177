"""Register budgets of the attention kernels (CPU only).

The flash, decode and prologue kernels are sized to the gfx950 register
file; a change that makes the compiler spill (to scratch) costs 10-40% with
correct results, so only the timings would show it.  This test compiles the
sources for gfx950 with the compiler's resource remarks and requires zero
scratch bytes for every instantiation of the kernels below, including the
fallback pass's gated kernels, whose item loops once spilled.
"""
import concurrent.futures
import os
import re
import subprocess

import pytest

from hippo_leap_amd import build as hb

CHECKED = {
    "prefill.hip": ("prefill_mfma_kernel", "prefill_f32mfma_kernel"),
    "rope_store.hip": ("kv_prologue_kernel", "prologue_kernel", "headvec_kernel", "store_cols_kernel"),
    "decode.hip": ("decode_mfma_kernel", "decode_f32_kernel"),
}


def _resources(src):
    r = subprocess.run([hb.hipcc(), *hb.compile_flags(), "-Rpass-analysis=kernel-resource-usage",
                        "--offload-device-only", "-c", os.path.join(hb.CSRC, src), "-o", os.devnull],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-3000:]
    kernels, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark: ([A-Za-z /\[\]]+): (\S+)", line)
        if m and cur is not None:
            cur[m.group(1).strip()] = m.group(2)
    return src, kernels


@pytest.fixture(scope="module")
def resources():
    try:
        hb.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    with concurrent.futures.ThreadPoolExecutor(len(CHECKED)) as ex:
        return dict(ex.map(_resources, CHECKED))


@pytest.mark.parametrize("src", sorted(CHECKED))
def test_no_scratch(resources, src):
    kernels = resources[src]
    seen = 0
    for name, res in kernels.items():
        if not any(k in name for k in CHECKED[src]):
            continue
        seen += 1
        assert res.get("ScratchSize [bytes/lane]") == "0", (name, res)
    assert seen, f"no checked kernel found in {src}"
