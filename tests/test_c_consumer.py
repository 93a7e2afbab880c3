"""The C-ABI from plain C: tests/c_consumer.c is compiled with gcc against
include/openmini_qmm.h and linked to the built libopenmini_qmm.so, as a Rust / cgo /
JNI binding would be, and run as a separate process.  The host mode needs no device;
the device mode (upload, decode GEMV, check against a C restatement of the reference's
Q4_0 dequantize + linear) runs on an MI355X."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "openmini-v1_amd")


@pytest.fixture(scope="module")
def consumer(tmp_path_factory):
    if not os.path.exists(os.path.join(LIBDIR, "libopenmini_qmm.so")):
        pytest.fail("libopenmini_qmm.so is not built: run __graft_entry__.build() first")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler on this machine")
    exe = str(tmp_path_factory.mktemp("c_consumer") / "c_consumer")
    cmd = [cc, "-std=c11", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c_consumer.c"), "-o", exe,
           "-L", LIBDIR, "-lopenmini_qmm", f"-Wl,-rpath,{LIBDIR}", "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def run(exe, mode):
    p = subprocess.run([exe, mode], capture_output=True, text=True, timeout=120)
    print(p.stdout, p.stderr)
    assert p.returncode == 0, (p.returncode, p.stdout, p.stderr)
    return p.stdout


def test_c_consumer_host(consumer):
    assert "host ok" in run(consumer, "host")


@pytest.mark.gpu
def test_c_consumer_device(consumer):
    print("c_consumer device: Q4_0 N=80 K=256 B=3,8", flush=True)
    assert "device ok" in run(consumer, "device")
