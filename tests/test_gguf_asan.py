"""The GGUF parser under host AddressSanitizer (CPU only).

openmini-v1_amd/build.py --asan builds the library with every host translation unit
instrumented (device code unchanged).  A child process preloads the clang ASan runtime,
loads that build and feeds it the fixed-seed GGUF mutants of tests/gguf_fixtures.py
(both dialects), the oversized-dims and the huge-array files: every file must parse or
fail with a status, and ASan must report nothing.  Reference recipe for a sanitizer
target: openmini-server/tests/quant_simd_regression_test.rs:15-16."""
import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "openmini-v1_amd")

_CHILD = r"""
import ctypes, os, struct, sys
sys.path[:0] = [sys.argv[1], sys.argv[2], os.path.join(sys.argv[1], "tests")]
from openmini_qmm import _native
_native.LIB_PATH = sys.argv[3]
import gguf_fixtures as fx
L = _native.lib()
maps = open("/proc/self/maps").read()
assert "libclang_rt.asan" in maps and "libopenmini_qmm_asan" in maps, "ASan runtime or build not mapped"

path = os.path.join(sys.argv[4], "m.gguf")
ok = bad = 0
def one(data, dialect):
    global ok, bad
    open(path, "wb").write(data)
    h = ctypes.c_void_p()
    rc = L.openmini_qmm_gguf_open(path.encode(), dialect, ctypes.byref(h))
    if rc != 0:
        bad += 1
        return
    ok += 1
    hdr = _native.GgufHeader()
    assert L.openmini_qmm_gguf_header(h, ctypes.byref(hdr)) == 0
    name = ctypes.create_string_buffer(256)
    for i in range(hdr.distinct_tensors):
        assert L.openmini_qmm_gguf_tensor_name(h, i, name, 256) == 0
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        if L.openmini_qmm_gguf_tensor_data(h, name.value, ctypes.byref(p), ctypes.byref(n)) == 0 and n.value:
            ctypes.string_at(p, n.value)  # every byte of the view is readable
    key = ctypes.create_string_buffer(256)
    for i in range(hdr.distinct_keys):
        assert L.openmini_qmm_gguf_meta_key(h, i, key, 256) == 0
        s, sl = ctypes.create_string_buffer(64), ctypes.c_size_t()
        L.openmini_qmm_gguf_get_string(h, key.value, s, 64, ctypes.byref(sl))
    L.openmini_qmm_gguf_close(h)
for dialect, data in fx.mutations(int(sys.argv[5]), int(sys.argv[6])):
    one(data, 1 if dialect == "reference" else 2)
for dims in ([2**33, 2**33], [3, 2**62 + 1], [2**40, 2**9]):
    one(fx.build([], [("t", dims, 0, bytes(64))], "reference"), 1)
print("parsed", ok, "failed", bad)
"""


def _asan_lib() -> str:
    sys.path.insert(0, PKG)
    import build as B  # openmini-v1_amd/build.py
    srcs = glob.glob(os.path.join(PKG, "csrc", "*")) + glob.glob(os.path.join(ROOT, "include", "*.h"))
    if not os.path.exists(B.ASAN_LIB_PATH) or os.path.getmtime(B.ASAN_LIB_PATH) < max(map(os.path.getmtime, srcs)):
        B.build(asan=True)
    return B.ASAN_LIB_PATH, B.asan_runtime()


def test_gguf_fuzz_under_host_asan(tmp_path):
    lib, rt = _asan_lib()
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=86")
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT, PKG, lib, str(tmp_path), "20261203", "2500"],
                       env=env, capture_output=True, text=True, timeout=600)
    assert "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-4000:])
    ok, bad = int(r.stdout.split()[1]), int(r.stdout.split()[3])
    assert ok > 0 and bad > 0 and ok + bad == 2503
