"""Build recipe for ``libspecdec_amd.so`` (the C-ABI library of this package).

Every ``csrc/*.hip`` / ``csrc/*.cpp`` is compiled for gfx950 with hipcc and
linked into one shared library next to this file. The library links against
``libamdhip64.so.7`` by soname only (no rpath into /opt/rocm), so inside a
process that imported torch first it binds to the HIP runtime torch already
loaded.

Run directly (``python specdec-nanovllm_amd/build.py``) or through
``__graft_entry__.build()``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB_NAME = "libspecdec_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-I", INCLUDE, "-I", CSRC,
    # Packed FP32 instructions stay off on this hardware pool (hipcc only).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer build (the C-ABI's
# argument checks on a machine without a GPU): the host pass only, with an empty
# device image (no kernel can run from this build), the sanitizer runtime
# preloaded by the process that opens the library.
SANITIZE_FLAGS = [
    "-O1", "-g", "-fno-omit-frame-pointer", "--cuda-host-only",
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
]


def build(verbose: bool = False, sanitize: bool = False, out: str | None = None) -> str:
    """Compile all sources and link ``libspecdec_amd.so`` (or ``out``); returns its
    path. ``sanitize``: the host-only sanitizer build (no kernels; for the
    argument-validation tests)."""
    cc = hipcc()
    srcs = sources()
    lib_path = out or LIB_PATH
    extra = SANITIZE_FLAGS if sanitize else []
    tmp = tempfile.mkdtemp(prefix="sd_build_", dir=os.path.dirname(lib_path))
    try:
        if sanitize:
            empty = os.path.join(tmp, "empty.fatbin")
            open(empty, "wb").close()
            extra = extra + ["-Xclang", "-fcuda-include-gpubinary", "-Xclang", empty]

        def compile_one(src: str) -> str:
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            lang = ["-x", "hip"] if src.endswith(".cpp") else []
            cmd = [cc, *COMMON_FLAGS, *extra, *lang, "-c", src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
            return obj

        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            objs = list(ex.map(compile_one, srcs))
        out_tmp = lib_path + ".tmp"
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", out_tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
        os.replace(out_tmp, lib_path)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return lib_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
