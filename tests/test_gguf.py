"""GGUF reader (host side of the loader path): parsing in both dialects, metadata
getters, tensor lookup and data views, and the reference's error behaviour.  Host-only
calls: no GPU is touched.  Expectations follow the reference's own GGUF tests
(src/model/inference/gguf.rs:2755-3050) on the same fixture bytes, plus the GGUF
specification for the standard dialect."""
import struct

import numpy as np
import pytest

import gguf_fixtures as fx
from openmini_qmm import gguf as G


def write(tmp_path, data: bytes, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_reference_minimal_fixture(tmp_path):
    """gguf.rs:2755-2788 test_gguf_file_parsing, :2900-2920 header, :2922-2955 info,
    :2790-2814 data access, :3024-3051 metadata accessors."""
    g = G.GgufFile(write(tmp_path, fx.build_minimal_gguf()), G.REFERENCE)
    assert (g.version, g.tensor_count, g.metadata_kv_count) == (3, 1, 3)
    assert g.get_string("general.architecture") == "llama"
    assert g.get_u32("llama.embedding_length") == 4096 and g.get_u32("llama.block_count") == 32
    assert g.get_string("nonexistent.key") is None and g.get_u32("nonexistent.u32") is None
    t = g.tensors["model.token_embd.weight"]
    assert t.dims == [4096] and t.tensor_type == 0
    assert t.num_elements() == 4096 and t.data_size() == 16384
    data = g.get_tensor_data("model.token_embd.weight")
    assert data.size == 4096 * 4
    assert np.all(data.view(np.float32) == 0.5)
    assert t.offset % 32 == 0


def test_auto_reads_the_reference_dialect(tmp_path):
    g = G.GgufFile(write(tmp_path, fx.build_minimal_gguf()))
    assert g.dialect == G.REFERENCE
    assert np.all(g.get_tensor_data("model.token_embd.weight").view(np.float32) == 0.5)


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_standard_dialect_relative_aligned_offsets(tmp_path, alignment):
    a = np.arange(96, dtype=np.float32)
    b = np.arange(5, dtype=np.uint8)
    meta = [("general.architecture", fx.STRING, "llama")]
    if alignment != 32:
        meta.append(("general.alignment", fx.U32, alignment))
    data = fx.build(meta, [("a", [96], 0, a.tobytes()), ("b", [5], 24, b.tobytes()),
                           ("c", [32, 2], 2, bytes(36))], "standard", alignment=alignment)
    for dialect in (G.STANDARD, G.AUTO):
        g = G.GgufFile(write(tmp_path, data), dialect)
        assert g.dialect == G.STANDARD and g.alignment == alignment
        assert np.array_equal(g.get_tensor_data("a").view(np.float32), a)
        assert np.array_equal(g.get_tensor_data("b"), b)
        assert all(t.offset % alignment == 0 for t in g.tensors.values())
        assert g.tensors["c"].data_size() == 36 and g.tensors["c"].dims == [32, 2]


def test_every_value_type_and_getter_conversions(tmp_path):
    """gguf.rs:73-101 value types; getters get_u32 (UInt32 | Int32), get_u64 (UInt64 |
    Int64 | UInt32 | Int32), get_f32 (Float32 only), get_string (gguf.rs:143-209)."""
    meta = [("u8", fx.U8, 200), ("i8", fx.I8, -5), ("u16", fx.U16, 60000), ("i16", fx.I16, -300),
            ("u32", fx.U32, 4000000000), ("i32", fx.I32, -7), ("f32", fx.F32, 1.5), ("b", fx.BOOL, True),
            ("s", fx.STRING, "héllo"), ("arr", fx.ARRAY, (fx.U32, [1, 2, 3])),
            ("sarr", fx.ARRAY, (fx.STRING, ["a", "bc"])), ("u64", fx.U64, 1 << 40), ("i64", fx.I64, -(1 << 40)),
            ("f64", fx.F64, 2.25)]
    for dialect in ("reference", "standard"):
        g = G.GgufFile(write(tmp_path, fx.build(meta, [], dialect)))
        assert g.keys == [m[0] for m in meta]
        assert g.get_u32("u32") == 4000000000 and g.get_u32("i32") == (-7) & 0xFFFFFFFF
        assert g.get_u32("u8") is None and g.get_u32("u64") is None
        assert g.get_u64("u64") == 1 << 40 and g.get_u64("i64") == (-(1 << 40)) & (2 ** 64 - 1)
        assert g.get_u64("u32") == 4000000000 and g.get_u64("u16") is None
        assert g.get_f32("f32") == 1.5 and g.get_f32("f64") is None
        assert g.get_string("s") == "héllo" and g.get_string("u8") is None
        assert g.value_type("arr") == ("Array", 3) and g.value_type("sarr") == ("Array", 2)
        assert g.value_type("b") == ("Bool", 0) and g.value_type("missing") is None


def test_later_definitions_replace_earlier_ones(tmp_path):
    """HashMap::insert semantics of parse_metadata / parse_tensor_info (gguf.rs:1744,
    :2027): the last definition of a key or tensor name wins."""
    data = fx.build([("k", fx.U32, 1), ("k", fx.U32, 2)],
                    [("t", [4], 0, np.ones(4, np.float32).tobytes()), ("t", [2], 0, np.full(2, 3, np.float32).tobytes())],
                    "reference")
    g = G.GgufFile(write(tmp_path, data), G.REFERENCE)
    assert g.get_u32("k") == 2 and g.metadata_kv_count == 2 and g.keys == ["k"]
    assert g.tensors["t"].dims == [2] and np.all(g.get_tensor_data("t").view(np.float32) == 3)


@pytest.mark.parametrize("data,msg", [
    (bytes(10), "too small"),                                                           # gguf.rs:2859-2872
    (struct.pack("<IIQQ", 0x12345678, 3, 0, 0), "Invalid GGUF magic"),                   # gguf.rs:2836-2857
    (b"GGUF partial data...", "too small"),                                             # gguf.rs:2973-2996
])
def test_reference_error_cases(tmp_path, data, msg):
    with pytest.raises(G.GgufError) as ei:
        G.GgufFile(write(tmp_path, data))
    assert msg in str(ei.value)


def test_missing_file_is_an_os_error():
    with pytest.raises(G.GgufError) as ei:  # gguf.rs:2957-2971
        G.GgufFile("/nonexistent/file.gguf")
    assert "no such file" in str(ei.value).lower() and "os error" in str(ei.value)


@pytest.mark.parametrize("dialect", [G.REFERENCE, G.STANDARD])
def test_malformed_fields(tmp_path, dialect):
    hdr = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
    # string longer than the 1 MB cap (gguf.rs:1777-1784)
    with pytest.raises(G.GgufError, match="String too long"):
        G.GgufFile(write(tmp_path, hdr + struct.pack("<Q", (1 << 20) + 1) + bytes(32)), dialect)
    # unknown value type 13
    tid = struct.pack("<B", 13) if dialect == G.REFERENCE else struct.pack("<I", 13)
    with pytest.raises(G.GgufError, match="Unknown value type"):
        G.GgufFile(write(tmp_path, hdr + fx._str("k") + tid + bytes(16)), dialect)
    # nested arrays (gguf.rs:1948-1950)
    inner = (struct.pack("<B", fx.ARRAY) if dialect == G.REFERENCE else struct.pack("<I", fx.ARRAY))
    body = fx._str("k") + inner + inner + struct.pack("<Q", 1) + bytes(16)
    with pytest.raises(G.GgufError, match="Nested arrays"):
        G.GgufFile(write(tmp_path, hdr + body), dialect)
    # too many dimensions (gguf.rs:1996-2002) and unknown tensor type (:2011-2012)
    thdr = struct.pack("<IIQQ", 0x46554747, 3, 1, 0)
    with pytest.raises(G.GgufError, match="Too many dimensions"):
        G.GgufFile(write(tmp_path, thdr + fx._str("t") + struct.pack("<I", 9) + bytes(128)), dialect)
    ttid = struct.pack("<B", 6) if dialect == G.REFERENCE else struct.pack("<I", 6)
    with pytest.raises(G.GgufError, match="Unknown tensor type: 6"):
        G.GgufFile(write(tmp_path, thdr + fx._str("t") + struct.pack("<IQ", 1, 4) + ttid + bytes(16)), dialect)


def test_tensor_data_out_of_bounds(tmp_path):
    """get_tensor_data -> None / get_tensor_data_by_ref -> "Tensor data out of bounds"
    (gguf.rs:2038-2044, 2066-2068) when the data does not fit in the file."""
    data = bytearray(fx.build_minimal_gguf())
    data = bytes(data[:-4])  # last f32 cut off
    g = G.GgufFile(write(tmp_path, data), G.REFERENCE)
    assert g.get_tensor_data("model.token_embd.weight") is None
    assert g.get_tensor_data("absent") is None


def test_truncation_never_crashes(tmp_path):
    """Every prefix of a multi-tensor file is either parsed or reported as an error
    (the reference indexes the map without checks and can panic here)."""
    q = np.random.default_rng(0).integers(0, 256, 2 * 18 * 4, dtype=np.uint8)
    full = fx.build([("general.architecture", fx.STRING, "llama"), ("a", fx.ARRAY, (fx.U32, [1, 2]))],
                    [("w", [64, 4], 2, q.tobytes()), ("x", [8], 0, bytes(32))], "reference")
    ok = 0
    for cut in range(0, len(full) + 1, 3):
        try:
            g = G.GgufFile(write(tmp_path, full[:cut]), G.REFERENCE)
            ok += 1
            for name in g.tensors:
                g.get_tensor_data(name)
        except G.GgufError:
            pass
    assert ok >= 1


def test_loader_names_and_shapes(tmp_path):
    """QuantizedWeightLoader tensor names (quant_loader.rs:95-138) and the [K, N] GGUF
    dims of a projection (ne0 = K contiguous)."""
    K, N = 64, 48
    q = np.random.default_rng(1).integers(0, 256, N * (K // 32) * 18, dtype=np.uint8)
    names = [f"model.layers.0.attention.{p}" for p in ("q_proj", "k_proj", "v_proj", "o_proj")] + \
            [f"model.layers.0.ffn.{p}" for p in ("gate_proj", "up_proj", "down_proj")]
    data = fx.build([], [(n, [K, N], 2, q.tobytes()) for n in names], "reference")
    g = G.GgufFile(write(tmp_path, data))
    assert sorted(g.tensors) == sorted(names)
    t = g.tensors["model.layers.0.ffn.up_proj"]
    assert t.dims == [K, N] and t.data_size() == q.size
    assert np.array_equal(g.get_tensor_data(t.name), q)


def _utf8_expectation(raw: bytes) -> str:
    """The reference's message for a string of these bytes (gguf.rs:1780,
    String::from_utf8), pinned by Python's strict UTF-8 decoder: the same RFC 3629
    rules and the same error position and length (maximal invalid subpart)."""
    try:
        raw.decode("utf-8")
        return ""
    except UnicodeDecodeError as e:
        if e.reason == "unexpected end of data":
            return f"Invalid UTF-8 string: incomplete utf-8 byte sequence from index {e.start}"
        return f"Invalid UTF-8 string: invalid utf-8 sequence of {e.end - e.start} bytes from index {e.start}"


UTF8_CASES = [
    b"ab\xffcd",               # invalid start byte
    b"ab\xc0\x80cd",           # overlong NUL
    b"ab\xe0\x80\x80cd",       # overlong 3-byte form
    b"ab\xed\xa0\x80cd",       # UTF-16 surrogate
    b"ab\xf4\x90\x80\x80cd",   # above U+10FFFF
    b"ab\xe4\xb8xcd",          # third byte not a continuation
    b"ab\xf0\x9f\x98xcd",      # fourth byte not a continuation
    b"ab\xe4\xb8",             # ends inside a sequence
    "权重.中文".encode(),       # valid multi-byte text
    "w\U0001F642".encode(),    # valid 4-byte sequence
]


@pytest.mark.parametrize("dialect", [G.REFERENCE, G.STANDARD])
@pytest.mark.parametrize("where", ["key", "value", "tensor"])
@pytest.mark.parametrize("raw", UTF8_CASES)
def test_strings_must_be_utf8(tmp_path, dialect, where, raw):
    """Every GGUF string (keys, string values, tensor names) goes through
    String::from_utf8 in the reference: invalid UTF-8 is an error naming the position,
    valid text is kept byte for byte."""
    hole = "Q" * len(raw)
    key, value, tname = (hole if where == "key" else "k"), (hole if where == "value" else "v"), \
        (hole if where == "tensor" else "t")
    data = fx.build([(key, fx.STRING, value)], [(tname, [32], 0, bytes(128))],
                    "reference" if dialect == G.REFERENCE else "standard")
    assert data.count(hole.encode()) == 1
    data = data.replace(hole.encode(), raw)
    want = _utf8_expectation(raw)
    if want:
        with pytest.raises(G.GgufError) as ei:
            G.GgufFile(write(tmp_path, data), dialect)
        assert want in str(ei.value)
        return
    g = G.GgufFile(write(tmp_path, data), dialect)
    text = raw.decode()
    if where == "key":
        assert g.keys == [text] and g.get_string(text) == "v"
    elif where == "value":
        assert g.get_string("k") == text
    else:
        assert list(g.tensors) == [text] and g.get_tensor_data(text) is not None


def test_random_mutations_parse_or_fail_cleanly(tmp_path):
    """Fixed-seed mutation fuzzing of a multi-tensor file in both dialects: byte
    overwrites, 64-bit counts / lengths / offsets set to extreme values, truncation.
    Every file either parses (and its tensor views stay in the file) or raises
    GgufError; nothing else escapes and nothing crashes.  The same mutants run under
    host AddressSanitizer in tests/test_gguf_asan.py."""
    dialects = {"reference": G.REFERENCE, "standard": G.STANDARD}
    path = write(tmp_path, b"")
    parsed = failed = 0
    for dialect, b in fx.mutations(20261202, 600):
        with open(path, "wb") as f:
            f.write(b)
        try:
            g = G.GgufFile(path, dialects[dialect])
        except G.GgufError:
            failed += 1
            continue
        parsed += 1
        for name in g.tensors:
            view = g.get_tensor_data(name)
            if view is not None:  # inside the file, and every byte readable
                assert len(view) <= len(b)
                int(view.sum(dtype=np.uint64))
    assert parsed > 0 and failed > 0


@pytest.mark.parametrize("dims", [[2**33, 2**33], [3, 2**62 + 1], [2**40, 2**9]])
def test_oversized_tensor_dims_are_out_of_bounds(tmp_path, dims):
    """A tensor whose element count overflows 64 bits, wraps to a small byte count
    (F32: 4 * (3 * (2^62 + 1)) mod 2^64 = 12), or exceeds 2^48 elements reports
    "Tensor data out of bounds" instead of a wrapped size: no view, no dequantization."""
    data = fx.build([], [("t", dims, 0, bytes(64))], "reference")
    g = G.GgufFile(write(tmp_path, data), G.REFERENCE)
    assert g.get_tensor_data("t") is None


_HUGE_ARRAY_CHILD = r"""
import ctypes, resource, sys
sys.path[:0] = sys.argv[2:]
from openmini_qmm import _native
L = _native.lib()
vm = 0
for line in open("/proc/self/status"):
    if line.startswith("VmSize:"):
        vm = int(line.split()[1]) * 1024
lim = vm + (2 << 30)
resource.setrlimit(resource.RLIMIT_AS, (lim, lim))
h = ctypes.c_void_p()
rc = L.openmini_qmm_gguf_open(sys.argv[1].encode(), 2, ctypes.byref(h))
print(rc, L.openmini_qmm_last_error().decode())
"""


def test_huge_array_count_fails_with_memory_error(tmp_path):
    """A u8 metadata array whose count fits in the file but whose parsed values outrun
    host memory (40 M elements, ~3.5 GB of parsed values against 2 GiB of address space
    left) fails with MEMORY; std::bad_alloc does not escape openmini_qmm_gguf_open.  Run
    in a child process with a capped address space."""
    import subprocess
    import sys
    n = 40_000_000
    path = tmp_path / "huge_array.gguf"
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQ", 0x46554747, 3, 0, 1))
        f.write(struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", fx.ARRAY, fx.U8, n))
        f.write(bytes(n))
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    paths = [os.path.dirname(here), os.path.join(os.path.dirname(here), "openmini-v1_amd")]
    r = subprocess.run([sys.executable, "-c", _HUGE_ARRAY_CHILD, str(path), *paths],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    rc, msg = r.stdout.strip().split(" ", 1)
    assert int(rc) == -1, r.stdout  # OPENMINI_QMM_ERR_MEMORY
    assert "allocation" in msg
