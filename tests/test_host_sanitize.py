"""The library's host code (argument validation, split and workspace
planning, the model and cache descriptor checks of api.hip and model.hip)
built with AddressSanitizer and UndefinedBehaviorSanitizer on the host side
only (-Xarch_host -fsanitize=...; device code is compiled as usual) and
driven by tests/sanitize/host_checks.cpp: the reference's ValueError
prechecks, workspace planning over a sweep of decode / step / prefill /
forward shapes, and the refusal of a workspace one byte short.  No GPU is
needed: every call returns before its first launch.  Runs on the CPU only
(it compiles every source, about a minute on 8 cores)."""
import concurrent.futures
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "hippo_leap_amd", "csrc")
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=undefined"]


def _hipcc():
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc is needed to build the sanitized host code")
def test_host_code_under_asan_ubsan(tmp_path):
    hipcc = _hipcc()
    common = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-I", os.path.join(ROOT, "include"),
              "-I", CSRC, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *SAN]
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))

    def compile_one(src):
        obj = str(tmp_path / (src[:-4] + ".o"))
        r = subprocess.run([hipcc, *common, "-fPIC", "-c", os.path.join(CSRC, src), "-o", obj],
                           capture_output=True, text=True)
        assert r.returncode == 0, f"{src}:\n{r.stderr[-3000:]}"
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, srcs))
    exe = str(tmp_path / "host_checks")
    r = subprocess.run([hipcc, *common, "-x", "c++", os.path.join(ROOT, "tests", "sanitize", "host_checks.cpp"),
                        "-x", "none", *objs, "-o", exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-5000:]
    assert "host checks passed" in out
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-5000:]
