"""ctypes front end of the CPU oracle (qmm_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker or the CPU baseline, never
as the thing measured or shipped.  The product library (libopenmini_qmm.so)
neither links nor calls anything here.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqmm_oracle.so")

F32, F16, Q4_0, Q4_1, Q8_0 = 0, 1, 2, 3, 7
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 10, 11, 12, 13, 14, 15
QK = 32
BYTES_PER_BLOCK = {Q4_0: 18, Q4_1: 20, Q8_0: 34, Q2_K: 68, Q3_K: 162, Q4_K: 144, Q5_K: 176,
                   Q6_K: 210, Q8_K: 258}
BLOCK_SIZE = {Q4_0: 32, Q4_1: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256,
              Q6_K: 256, Q8_K: 256}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p, sz, i, f, u16 = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                           ctypes.c_float, ctypes.c_uint16)
        sig = {
            "orc_f16_to_f32": (f, [u16]),
            "orc_f32_to_f16": (u16, [f]),
            "orc_f32_to_bf16": (u16, [f]),
            "orc_bf16_to_f32": (f, [u16]),
            "orc_block_size": (sz, [i]),
            "orc_bytes_per_block": (sz, [i]),
            "orc_data_size": (sz, [i, sz]),
            "orc_dequantize_q4_0": (None, [p, sz, sz, p]),
            "orc_dequantize_q8_0": (None, [p, sz, sz, p]),
            "orc_dequantize": (i, [i, p, sz, sz, p]),
            "orc_safe_dequantize": (i, [i, p, sz, sz, p, ctypes.POINTER(sz)]),
            "orc_convert_to_soa": (sz, [i, p, sz, sz, p]),
            "orc_soa_bytes": (sz, [i, sz, sz]),
            "orc_quantize_q4_0": (None, [p, sz, p]),
            "orc_quantize_q8_0": (None, [p, sz, p]),
            "orc_linear_f64": (None, [i, p, sz, sz, p, sz, p]),
            "orc_linear_bf16x_f64": (None, [i, p, sz, sz, p, sz, p]),
            "orc_cpu_asrun_linear": (None, [p, sz, sz, p, sz, p, p, i]),
            "orc_cpu_fused_linear": (None, [i, p, sz, sz, p, sz, p, sz, sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u8(data) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8)) \
        if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, dtype=np.uint8)


# ---- scalar conversions --------------------------------------------------------

def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    return lib().orc_f32_to_f16(x)


def f32_to_bf16(x: float) -> int:
    return lib().orc_f32_to_bf16(x)


def f32_to_bf16_array(x: np.ndarray) -> np.ndarray:
    fn = lib().orc_f32_to_bf16
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([fn(float(v)) for v in flat], dtype=np.uint16).reshape(x.shape)


# ---- geometry / dequant ----------------------------------------------------------

def data_size(qtype: int, n: int) -> int:
    return lib().orc_data_size(qtype, n)


def dequantize(qtype: int, data, n: int) -> np.ndarray:
    """quant::dequantize (zero tail on short input)."""
    d = _u8(data)
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequantize(qtype, _ptr(d) if d.size else None, d.size, n, _ptr(out))
    return out


def safe_dequantize(qtype: int, data, n: int):
    """quant_simd::safe_dequantize -> (status, out, expected).
    status 0 = Ok, 1 = InsufficientData, 2 = UnsupportedType."""
    d = _u8(data)
    out = np.empty(max(n, 1), dtype=np.float32)
    exp = ctypes.c_size_t(0)
    st = lib().orc_safe_dequantize(qtype, _ptr(d) if d.size else None, d.size, n, _ptr(out),
                                   ctypes.byref(exp))
    return st, (out[:n] if st == 0 else None), exp.value


def restated(qtype: int) -> bool:
    """Whether quant::dequantize's arm for `qtype` is restated in the oracle."""
    out = np.empty(1, dtype=np.float32)
    return bool(lib().orc_dequantize(qtype, None, 0, 0, _ptr(out)))


def convert_to_soa(qtype: int, data, n: int) -> np.ndarray:
    """quant_simd::convert_to_soa_layout (quant_simd.rs:3245-3397), every arm."""
    d = _u8(data)
    total = lib().orc_soa_bytes(qtype, d.size, n)
    out = np.zeros(max(total, 1), dtype=np.uint8)
    m = lib().orc_convert_to_soa(qtype, _ptr(d) if d.size else None, d.size, n, _ptr(out))
    assert m == total
    return out[:m]


# ---- synthetic quantizers --------------------------------------------------------

def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    assert x.size % QK == 0
    out = np.empty(x.size // QK * BYTES_PER_BLOCK[qtype], dtype=np.uint8)
    fn = lib().orc_quantize_q4_0 if qtype == Q4_0 else lib().orc_quantize_q8_0
    fn(_ptr(x), x.size, _ptr(out))
    return out


# ---- contraction ------------------------------------------------------------------

def linear_f64(qtype: int, w: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    """y[B, N] = x[B, K] . W[N, K]^T, fp64 accumulation (model.rs:1050-1064)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    B = x.shape[0]
    y = np.empty((B, N), dtype=np.float64)
    lib().orc_linear_f64(qtype, _ptr(_u8(w)), N, K, _ptr(x), B, _ptr(y))
    return y


def linear_bf16x_f64(qtype: int, w: np.ndarray, N: int, K: int, xb16: np.ndarray) -> np.ndarray:
    xb16 = np.ascontiguousarray(xb16, dtype=np.uint16).reshape(-1, K)
    M = xb16.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    lib().orc_linear_bf16x_f64(qtype, _ptr(_u8(w)), N, K, _ptr(xb16), M, _ptr(y))
    return y


def silu_f64(v: np.ndarray) -> np.ndarray:
    """silu(v) = v / (1 + exp(-v)) (model.rs:1187-1189), in fp64.  exp overflow for
    v < -709 gives v / inf = -0.0, the limit."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def ffn_hidden_f64(qtype: int, wg: np.ndarray, wu: np.ndarray, N: int, K: int,
                   x: np.ndarray) -> np.ndarray:
    """FFNWeights::forward's hidden state (model.rs:728-730):
    silu(x . Wg^T) * (x . Wu^T), fp64."""
    return silu_f64(linear_f64(qtype, wg, N, K, x)) * linear_f64(qtype, wu, N, K, x)


def ffn_hidden_bf16x_f64(qtype: int, wg: np.ndarray, wu: np.ndarray, N: int, K: int,
                         xb16: np.ndarray) -> np.ndarray:
    """The same on bf16 activations (raw bits)."""
    return (silu_f64(linear_bf16x_f64(qtype, wg, N, K, xb16))
            * linear_bf16x_f64(qtype, wu, N, K, xb16))


def cpu_asrun_linear(w_f32: np.ndarray, x: np.ndarray, scratch: np.ndarray | None,
                     transpose_copy: bool) -> np.ndarray:
    N, K = w_f32.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    y = np.empty((x.shape[0], N), dtype=np.float32)
    lib().orc_cpu_asrun_linear(_ptr(w_f32), N, K, _ptr(x), x.shape[0], _ptr(y),
                               _ptr(scratch) if scratch is not None else None,
                               1 if transpose_copy else 0)
    return y


def cpu_fused_linear(qtype: int, w: np.ndarray, N: int, K: int, x: np.ndarray,
                     y: np.ndarray, n0: int, n1: int) -> None:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    lib().orc_cpu_fused_linear(qtype, _ptr(w), N, K, _ptr(x), x.shape[0], _ptr(y), n0, n1)


# ---- reference test-data generators (closed forms) ---------------------------------

def create_test_q4_0_data(n: int) -> np.ndarray:
    """tests/quant_simd_regression_test.rs:30-48: d_i = f16(0.1 + 0.01 i),
    byte j = v << 4 | v with v = (16 i + j) % 16."""
    blocks = (n + QK - 1) // QK
    out = bytearray()
    for i in range(blocks):
        h = f32_to_f16(np.float32(0.1) + np.float32(i) * np.float32(0.01))
        out += bytes([h & 0xFF, h >> 8])
        for j in range(16):
            v = (i * 16 + j) % 16
            out.append(((v << 4) | (v & 0x0F)) & 0xFF)
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


def create_test_q4_1_data(n: int) -> np.ndarray:
    """tests/quant_simd_regression_test.rs:72-94: d_i = f16(0.15 + 0.015 i),
    m_i = f16(-1.0 + 0.1 i), byte j = v << 4 | v with v = (16 i + j) % 16."""
    blocks = (n + QK - 1) // QK
    out = bytearray()
    for i in range(blocks):
        h = f32_to_f16(np.float32(0.15) + np.float32(i) * np.float32(0.015))
        m = f32_to_f16(np.float32(-1.0) + np.float32(i) * np.float32(0.1))
        out += bytes([h & 0xFF, h >> 8, m & 0xFF, m >> 8])
        for j in range(16):
            v = (i * 16 + j) % 16
            out.append(((v << 4) | (v & 0x0F)) & 0xFF)
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()


def create_test_q8_0_data(n: int) -> np.ndarray:
    """tests/quant_simd_regression_test.rs:51-69: d_i = f16(0.2 + 0.02 i),
    byte j = ((32 i + j) % 256) as i8."""
    blocks = (n + QK - 1) // QK
    out = bytearray()
    for i in range(blocks):
        h = f32_to_f16(np.float32(0.2) + np.float32(i) * np.float32(0.02))
        out += bytes([h & 0xFF, h >> 8])
        for j in range(32):
            out.append((i * 32 + j) % 256)
    return np.frombuffer(bytes(out), dtype=np.uint8).copy()
