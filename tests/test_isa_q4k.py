"""Code-generation check of the Q4_K matrix-core GEMV (CPU only).

q4k_mfma_kernel keeps the weight loads of three steps in flight with
buffer-load builtins.  Two code shapes silently drain that prefetch, with
correct results and ~5% more decode time on Llama-3-8B-shaped models:
  * a buffer resource the compiler cannot prove wave-uniform, which it
    wraps in a readfirstlane waterfall loop (``s_cbranch_execnz`` around a
    ``buffer_load``);
  * a full ``s_waitcnt vmcnt(0)`` inside the step loop, which the compiler
    inserts when a resource is selected in VGPRs that alias in-flight loads.
This test compiles linear_quant.hip for gfx950 to AMD assembly and checks
every instantiation of the kernel for both: the only vmcnt(0) is the one
after the loop, and no load sits in a waterfall loop.
"""
import os
import re
import subprocess

import pytest

from hippo_leap_amd import build as hb

SRC = os.path.join(hb.CSRC, "linear_quant.hip")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    try:
        cc = hb.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "linear_quant.s"
    r = subprocess.run([cc, *hb.compile_flags(), "--offload-device-only", "-S", SRC, "-o", str(out)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    return out.read_text()


def _kernels(text):
    bodies = {}
    for m in re.finditer(r"^(_ZN2hl12_GLOBAL__N_115q4k_mfma_kernel\w+):", text, re.M):
        end = text.index("s_endpgm", m.end())
        lines = [l.split(";")[0].strip() for l in text[m.end():end].split("\n")]
        bodies[m.group(1)] = [l for l in lines if l and not l.startswith(".") or l.startswith(".LBB")]
    return bodies


def test_q4k_mfma_loads_stay_in_flight(asm):
    bodies = _kernels(asm)
    assert len(bodies) >= 4, "expected the <0>, <1>, <2> and <1, norm> instantiations"
    for name, body in bodies.items():
        full = [i for i, l in enumerate(body) if "vmcnt(0)" in l]
        loads = [i for i, l in enumerate(body) if l.startswith("buffer_load")]
        assert loads, name
        # the final drain follows the last weight load
        assert len(full) == 1 and full[0] > loads[-1], (name, full, loads[-4:])
        # no load inside a waterfall loop: a label, the load, then a branch back on exec
        for i in loads:
            nxt = body[i + 1:i + 4]
            assert not any(l.startswith("s_cbranch_execnz") for l in nxt), (name, body[i - 3:i + 4])
