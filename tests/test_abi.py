"""The C-ABI library loads and exports every symbol include/openmini_qmm.h declares.
Only host-side validation is exercised here (no device is touched)."""
import ctypes
import os
import re

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "openmini_qmm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(openmini_qmm_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("openmini_qmm_upload", "openmini_qmm_gemv", "openmini_qmm_gemm_bf16",
                 "openmini_qmm_dequantize", "openmini_qmm_dequant_weight", "openmini_qmm_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from openmini_qmm import _native
    L = _native.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes table covers the header exactly
    assert sorted(_native.SIGNATURES) == declared_functions()


def test_host_only_validation():
    from openmini_qmm import _native
    L = _native.lib()
    assert L.openmini_qmm_version() == b"0.1.0"
    out = ctypes.c_size_t()
    assert L.openmini_qmm_required_bytes(2, 4096 * 11008, ctypes.byref(out)) == 0
    assert out.value == 25_362_432
    assert L.openmini_qmm_required_bytes(7, 33, ctypes.byref(out)) == 0 and out.value == 68
    # every layout the dequantization entry points take (gguf.rs:348-379, 431-438)
    for t, n, want in ((3, 33, 40), (10, 32, 68), (11, 256, 162), (12, 257, 288), (13, 256, 176),
                       (14, 512, 420), (15, 1, 258), (0, 3, 12), (1, 3, 6)):
        assert L.openmini_qmm_required_bytes(t, n, ctypes.byref(out)) == 0 and out.value == want, t
    assert L.openmini_qmm_required_bytes(16, 32, ctypes.byref(out)) == _native.ERR_UNSUPPORTED
    assert L.openmini_qmm_estimate_memory_usage(2, 64) == 36 + 256

    h = ctypes.c_void_p()
    buf = np.zeros(64, dtype=np.uint8)
    p = ctypes.c_void_p(buf.ctypes.data)
    # K not a multiple of 32
    assert L.openmini_qmm_upload(2, p, buf.size, 1, 48, ctypes.byref(h)) == _native.ERR_INVALID_PARAM
    assert b"multiple of 32" in L.openmini_qmm_last_error()
    # too few bytes: InsufficientData{expected=36, actual=20}
    assert L.openmini_qmm_upload(2, p, 20, 1, 64, ctypes.byref(h)) == _native.ERR_INSUFFICIENT_DATA
    assert b"expected 36" in L.openmini_qmm_last_error() and b"actual 20" in L.openmini_qmm_last_error()
    # weight types: Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K; Q2_K is dequantized only
    assert L.openmini_qmm_upload(10, p, 64, 1, 256, ctypes.byref(h)) == _native.ERR_UNSUPPORTED
    assert b"Q5_K=13" in L.openmini_qmm_last_error() and b"Q8_K=15" in L.openmini_qmm_last_error()
    # Q8_K: 256-element super-blocks of 258 bytes
    assert L.openmini_qmm_upload(15, p, 64, 1, 288, ctypes.byref(h)) == _native.ERR_INVALID_PARAM
    assert b"multiple of 256" in L.openmini_qmm_last_error()
    assert L.openmini_qmm_upload(15, p, 64, 2, 512, ctypes.byref(h)) == _native.ERR_INSUFFICIENT_DATA
    assert b"expected 1032" in L.openmini_qmm_last_error()
    # tiled codes must stay below 4 GiB (32-bit buffer offsets in the kernels)
    assert L.openmini_qmm_upload(7, p, 64, 1 << 19, 8192, ctypes.byref(h)) == _native.ERR_INVALID_PARAM
    assert b"exceed 4 GiB" in L.openmini_qmm_last_error()
    # safe_dequantize semantics: n == 0 is Ok, short input reports expected bytes
    exp = ctypes.c_size_t(123)
    assert L.openmini_qmm_dequantize(2, None, 0, 0, None, ctypes.byref(exp)) == 0 and exp.value == 0
    assert L.openmini_qmm_dequantize(2, p, 10, 32, p, ctypes.byref(exp)) == _native.ERR_INSUFFICIENT_DATA
    assert exp.value == 18
    assert L.openmini_qmm_dequantize(10, p, 64, 32, p, ctypes.byref(exp)) == _native.ERR_UNSUPPORTED
    # Q4_1 is validated like Q4_0 / Q8_0: 20-byte blocks
    assert L.openmini_qmm_dequantize(3, p, 10, 32, p, ctypes.byref(exp)) == _native.ERR_INSUFFICIENT_DATA
    assert exp.value == 20
    # quant::dequantize semantics: unknown layouts are refused before any device work
    assert L.openmini_qmm_dequantize_any(16, p, 64, 256, p) == _native.ERR_UNSUPPORTED
    assert L.openmini_qmm_dequantize_any(12, None, 0, 0, None) == 0
    # layer projections: argument checks that precede any device work
    arr = (ctypes.c_void_p * 5)()
    assert L.openmini_qmm_gemv_multi(None, 1, p, arr, 1, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemv_multi(arr, 0, p, arr, 1, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemv_multi(arr, 5, p, arr, 1, None) == _native.ERR_INVALID_PARAM
    assert b"count=5" in L.openmini_qmm_last_error()
    assert L.openmini_qmm_gemv_multi(arr, 1, p, arr, 1, None) == _native.ERR_INVALID_PARAM
    assert b"null weight" in L.openmini_qmm_last_error()
    assert L.openmini_qmm_ffn_gate_up(None, None, p, p, 1, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_ffn_gate_up_bf16(None, None, p, p, 1, None) == _native.ERR_INVALID_PARAM
    # the GEMM ceiling yardstick validates before touching a device
    assert L.openmini_qmm_gemm_ceiling(7, 512, 11008, 4096, None, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemm_ceiling(12, 512, 11008, 4096, p, None) == _native.ERR_UNSUPPORTED
    assert L.openmini_qmm_gemm_ceiling(7, 512, 11008, 4100, p, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_gemm_ceiling(7, 0, 11008, 4096, p, None) == _native.ERR_INVALID_PARAM


def test_q8k_weights_take_q8_0_chunks():
    """A Q8_K super-block is read as fp16 d and 256 int8 codes, value q * d
    (quant.rs:768-800): eight Q8_0 blocks sharing d, so a Q8_K weight is stored as Q8_0
    chunks and occupies what the Q8_0 weight of its shape does."""
    from openmini_qmm import weight_device_bytes
    for n, k in ((1, 256), (37, 2304), (11008, 4096), (4096, 11008), (8192, 28672)):
        assert weight_device_bytes(15, n, k) == weight_device_bytes(7, n, k), (n, k)


def test_python_mirror_raises_reference_errors():
    import pytest
    from openmini_qmm import InsufficientData, UnsupportedType, safe_dequantize_q4_0, safe_dequantize
    with pytest.raises(InsufficientData) as ei:
        safe_dequantize_q4_0(bytes(10), 32)
    assert (ei.value.expected, ei.value.actual) == (18, 10)
    with pytest.raises(UnsupportedType):
        safe_dequantize(b"", 10, 32)
    with pytest.raises(InsufficientData) as ei:
        safe_dequantize(bytes(30), 3, 64)
    assert (ei.value.expected, ei.value.actual) == (40, 30)
    assert safe_dequantize_q4_0(b"", 0).size == 0


def test_log_callback_receives_every_failure():
    """openmini_set_log_callback semantics (native/include/openmini.h:151-155): the
    sink sees each failure's message with its user data; a null sink stops it."""
    from openmini_qmm import _native
    L = _native.lib()
    seen = []

    @_native.LOG_CALLBACK
    def sink(level, text, user):
        seen.append((level, text.decode(), user))

    assert L.openmini_qmm_set_log_callback(sink, ctypes.c_void_p(1234)) == 0
    try:
        out = ctypes.c_size_t()
        assert L.openmini_qmm_required_bytes(16, 32, ctypes.byref(out)) == _native.ERR_UNSUPPORTED
        h = ctypes.c_void_p()
        assert L.openmini_qmm_upload(2, None, 0, 1, 48, ctypes.byref(h)) == _native.ERR_INVALID_PARAM
    finally:
        assert L.openmini_qmm_set_log_callback(_native.LOG_CALLBACK(), None) == 0
    assert len(seen) == 2, seen
    assert all(lv == _native.LOG_ERROR and u == 1234 for lv, _, u in seen)
    assert "16" in seen[0][1]  # the unsupported type id
    assert "multiple of 32" in seen[1][1]
    assert L.openmini_qmm_required_bytes(16, 32, ctypes.byref(out)) == _native.ERR_UNSUPPORTED
    assert len(seen) == 2  # logging is off again


def test_element_counts_are_bounded():
    """Element counts above 2^48 are rejected before any size is computed from them (no
    wrapped byte count can pass the InsufficientData check), on every entry point that
    takes one; the byte count at the limit is the closed form ceil(n / bs) * bpb."""
    from openmini_qmm import _native
    L = _native.lib()
    out = ctypes.c_size_t()
    lim = 1 << 48
    for t, bs, bpb in ((0, 1, 4), (1, 1, 2), (2, 32, 18), (3, 32, 20), (7, 32, 34), (10, 256, 68),
                       (11, 256, 162), (12, 256, 144), (13, 256, 176), (14, 256, 210), (15, 256, 258)):
        assert L.openmini_qmm_required_bytes(t, lim, ctypes.byref(out)) == 0
        assert out.value == -(-lim // bs) * bpb
        for n in (lim + 1, 2**62 + 1, 2**64 - 1):
            assert L.openmini_qmm_required_bytes(t, n, ctypes.byref(out)) == _native.ERR_INVALID_PARAM
            assert b"exceeds the maximum 2^48" in L.openmini_qmm_last_error()
            assert L.openmini_qmm_estimate_memory_usage(t, n) == 2**64 - 1
    buf = (ctypes.c_uint8 * 16)()
    dst = (ctypes.c_float * 4)()
    exp = ctypes.c_size_t()
    # F32 with 2^62 + 1 elements: 4 n wraps to 4 bytes, which the 16-byte buffer would cover
    assert L.openmini_qmm_dequantize_any(0, buf, 16, 2**62 + 1, dst) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_dequantize_any_device(0, buf, 16, 2**62 + 1, dst, None) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_dequantize(2, buf, 16, 2**62 + 1, dst, ctypes.byref(exp)) == _native.ERR_INVALID_PARAM
    assert L.openmini_qmm_dequantize_device(2, buf, 16, 2**62 + 1, dst, None, ctypes.byref(exp)) == \
        _native.ERR_INVALID_PARAM


def test_soa_bytes_host_rules(orc):
    """openmini_qmm_soa_bytes: the output length of convert_to_soa_layout for every arm,
    against the oracle's restatement; ids GgufTensorType lacks are UNSUPPORTED."""
    from openmini_qmm import _native
    L = _native.lib()
    out = ctypes.c_size_t()
    for t in list(range(0, 30)):
        for length, n in ((0, 5), (37, 0), (37, 5), (1000, 33), (18 * 4, 128), (3, 1 << 40)):
            rc = L.openmini_qmm_soa_bytes(t, length, n, ctypes.byref(out))
            if t in (6, 9):
                assert rc == _native.ERR_UNSUPPORTED
                continue
            assert rc == 0 and out.value == orc.lib().orc_soa_bytes(t, length, n), (t, length, n)
    assert L.openmini_qmm_soa_bytes(2, 10, (1 << 48) + 1, ctypes.byref(out)) == _native.ERR_INVALID_PARAM
