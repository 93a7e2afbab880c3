"""The Rust side of the boundary (openmini-v1_amd/rust/) against include/openmini_qmm.h.

There is no Rust toolchain in this image, so the FFI module is checked as text: every
C function of the header is declared in ffi.rs with the same name, the same number of
parameters and the corresponding Rust type for each (pointer constness included), and
nothing else is declared; the #[repr(C)] structs have the header's fields in order.
The CMake native build description (openmini-v1_amd/native/CMakeLists.txt) configures."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "openmini_qmm.h")
FFI = os.path.join(ROOT, "openmini-v1_amd", "rust", "ffi.rs")

C2R = {"int": "c_int", "size_t": "usize", "int64_t": "i64", "uint64_t": "u64", "uint32_t": "u32",
       "int32_t": "i32", "uint16_t": "u16", "float": "f32", "char": "c_char", "void": "c_void",
       "openmini_qweight_t": "QWeight", "openmini_qmm_gguf_t": "Gguf",
       "openmini_qmm_weight_info_t": "WeightInfo", "openmini_qmm_gguf_header_t": "GgufHeader",
       "openmini_qmm_gguf_tensor_info_t": "GgufTensorInfo",
       "openmini_qmm_log_callback_t": "Option<LogCallback>"}


def _c_type(t: str) -> str:
    """A C parameter type -> the Rust FFI type it must be declared as."""
    t = " ".join(t.split())
    parts = t.split("*")
    base = [w for w in parts[0].replace("const", " ").split() if w]
    r = C2R[base[-1]]
    for level in range(len(parts) - 1):
        r = ("*const " if "const" in parts[level] else "*mut ") + r
    return r


def header_functions():
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"^\s*((?:const\s+)?[\w\s\*]+?)\s*\b(openmini_qmm_\w+)\s*\(([^;]*?)\)\s*;",
                                      src, flags=re.M | re.S):
        params = []
        a = args.strip()
        if a and a != "void":
            for p in a.split(","):
                ty, _nm = re.match(r"(.*?)(\w+)$", " ".join(p.split())).groups()
                params.append(_c_type(ty))
        out[name] = (params, None if ret.strip() == "void" else _c_type(ret))
    return out


def rust_functions():
    src = open(FFI).read()
    block = src[src.index('extern "C" {'):]
    block = block[:block.index("\n}\n")]
    out = {}
    for name, args, ret in re.findall(r"pub fn (openmini_qmm_\w+)\((.*?)\)(?:\s*->\s*([^;]+))?;", block, flags=re.S):
        params = [p.split(":", 1)[1].strip() for p in args.split(",") if p.strip()]
        out[name] = (params, ret.strip() if ret else None)
    return out


def test_every_header_function_is_declared_alike():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 50
    assert set(h) == set(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name in h:
        assert h[name] == r[name], (name, h[name], r[name])


@pytest.mark.parametrize("c_name,r_name", [("openmini_qmm_weight_info_t", "WeightInfo"),
                                           ("openmini_qmm_gguf_header_t", "GgufHeader"),
                                           ("openmini_qmm_gguf_tensor_info_t", "GgufTensorInfo")])
def test_repr_c_structs_match(c_name, r_name):
    hsrc = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct \{([^{}]*)\}\s*" + c_name + ";", hsrc).group(1)
    c_fields = [(m.group(2), C2R[m.group(1)] if not m.group(3) else f"[{C2R[m.group(1)]}; {m.group(3)}]")
                for m in re.finditer(r"(\w+)\s+(\w+)(?:\[(\d+)\])?;", body)]
    rsrc = open(FFI).read()
    rbody = re.search(r"pub struct " + r_name + r" \{(.*?)\}", rsrc, flags=re.S).group(1)
    r_fields = re.findall(r"pub (\w+): ([^,]+),", rbody)
    assert [t for _, t in c_fields] == [t.strip() for _, t in r_fields], (c_fields, r_fields)
    # names differ only where `type` is a Rust keyword
    assert [n.replace("type", "tensor_type") if n == "type" else n for n, _ in c_fields] == [n for n, _ in r_fields]


@pytest.mark.skipif(shutil.which("cmake") is None or not os.path.isdir("/opt/rocm"), reason="cmake / ROCm absent")
def test_cmake_native_build_configures(tmp_path):
    r = subprocess.run(["cmake", "-S", os.path.join(ROOT, "openmini-v1_amd", "native"), "-B", str(tmp_path),
                        "-DCMAKE_PREFIX_PATH=/opt/rocm", "-DCMAKE_HIP_COMPILER=/opt/rocm/lib/llvm/bin/clang++"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "HIP architectures gfx950" in r.stdout
