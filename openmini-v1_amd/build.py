"""Builds libopenmini_qmm.so for gfx950 with hipcc (in-tree, next to this file).

    python openmini-v1_amd/build.py            # compile every source, then link
    python openmini-v1_amd/build.py --asan     # host code with AddressSanitizer:
                                               # _build/asan/libopenmini_qmm_asan.so

Each .hip source compiles to its own object in parallel; the shared library
exports only the C-ABI declared in include/openmini_qmm.h.  The ASan variant
instruments host code only (every -fsanitize= goes after -Xarch_host; device code is
the same as the release build) and needs the clang ASan runtime preloaded
(asan_runtime() names it); tests/test_gguf_asan.py runs the GGUF parser fuzz on it.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libopenmini_qmm.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions stay disabled for all device code (they have produced
# silent wrong results on this hardware pool); the host pass ignores the feature.
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the kernels post-process every MFMA result on the VALU,
    # and the AGPR form costs a v_accvgpr_read per element and serialises the MFMAs.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # The first kernel arguments arrive in SGPRs (gfx950 kernarg preloading): a
    # launch-bound kernel starts without waiting on a scalar load of its arguments.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-I", os.path.join(ROOT, "include"),
]


ASAN_DIR = os.path.join(BUILD_DIR, "asan")
ASAN_LIB_PATH = os.path.join(ASAN_DIR, "libopenmini_qmm_asan.so")
# host pass only: each sanitizer option preceded by -Xarch_host
ASAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime() -> str:
    """The clang ASan runtime a process must preload to load the ASan variant."""
    found = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError("clang ASan runtime not found under /opt/rocm/lib/llvm")
    return found[-1]


def _compile(src: str, out_dir: str = BUILD_DIR, extra=()) -> str:
    obj = os.path.join(out_dir, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, asan: bool = False) -> str:
    out_dir, lib_path = (ASAN_DIR, ASAN_LIB_PATH) if asan else (BUILD_DIR, LIB_PATH)
    extra = ASAN_HOST if asan else ()
    os.makedirs(out_dir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda src: _compile(src, out_dir, extra), sources))
    tmp = lib_path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *extra, "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path}")
    return lib_path


if __name__ == "__main__":
    build(verbose=True, asan="--asan" in sys.argv[1:])
    sys.exit(0)
