"""The C-ABI's host-side checks under AddressSanitizer and
UndefinedBehaviorSanitizer, on a machine without a GPU.

The library is rebuilt host-only with both sanitizers (``build.py``'s
``sanitize`` form: no device code, so no kernel can run from it) into a
temporary directory, and ``tests/test_capi_cpu.py`` runs against it in a child
process that preloads the ASan runtime (Python itself is not instrumented).
That file's argument sweep calls every entry point with each argument in turn
set to a hostile value, so an integer overflow, a wrapped pointer or an
out-of-bounds access in any validation path aborts the child and fails here.
"""
import glob
import importlib.util
import os
import shutil
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _asan_runtime():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hits = sorted(glob.glob(os.path.join(rocm, "llvm/lib/clang/*/lib/linux/"
                                               "libclang_rt.asan-x86_64.so")))
    return hits[-1] if hits else None


def _build_module():
    spec = importlib.util.spec_from_file_location(
        "_sd_build_san", os.path.join(ROOT, "specdec-nanovllm_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.skipif(torch.cuda.device_count() > 0,
                    reason="the sweep passes fake device addresses: CPU-only machines")
def test_capi_checks_under_asan_and_ubsan(tmp_path):
    rt = _asan_runtime()
    if rt is None or shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc or the clang ASan runtime is not installed")
    lib = _build_module().build(sanitize=True, out=str(tmp_path / "libspecdec_amd_san.so"))
    env = dict(os.environ,
               LD_PRELOAD=rt,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               SPECDEC_AMD_LIBRARY=lib)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_capi_cpu.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    report = r.stdout[-4000:] + r.stderr[-6000:]
    assert r.returncode == 0, report
    assert "passed" in r.stdout and "skipped" not in r.stdout.splitlines()[-1], report
