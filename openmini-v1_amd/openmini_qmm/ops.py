"""Host-side mirror of OpenMini-V1's quantized-linear operator interface, over the
HIP C-ABI.  Names, argument meaning and error behaviour follow the reference
(paths relative to openmini-server/):

  QuantError / InsufficientData / UnsupportedType   quant_simd.rs:91-103
  safe_dequantize{,_q4_0,_q8_0,_q4_1}               quant_simd.rs:150-302
  dequantize / dequantize_simd                      quant.rs:56-79, quant_simd.rs:304-313
  GpuQuantOps -> HipQuantOps                        quant_simd.rs:2944-2986 (trait),
                                                    :3137-3188 (the CUDA stub it replaces)
  GemmEngine -> HipQuantGemmEngine                  model/inference/gemm_engine.rs:37-56
  linear / linear_gemm                              model/inference/model.rs:1050-1064

Every computation runs in libopenmini_qmm.so on the GPU; nothing here falls back
to the CPU.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

from . import _native
from ._native import QmmError, check, lib

QK = 32


class GgufTensorType(enum.IntEnum):
    """GGUF type ids, model/inference/gguf.rs:219-240: the layouts this library
    dequantizes (weights for the GEMV: Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K and Q8_K; for
    the GEMM the same without Q4_1 and Q5_K)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 7
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    Q8K = 15

    def bytes_per_block(self) -> int:  # gguf.rs:356-379
        return {0: 4, 1: 2, 2: 18, 3: 20, 7: 34, 10: 68, 11: 162, 12: 144, 13: 176, 14: 210,
                15: 258}[int(self)]

    def block_size(self) -> int:  # gguf.rs:327-338
        return 1 if int(self) < 2 else 32 if int(self) < 10 else 256


# ---- quant_simd::QuantError --------------------------------------------------------

class QuantError(Exception):
    pass


class InsufficientData(QuantError):
    def __init__(self, expected: int, actual: int):
        super().__init__(f"InsufficientData {{ expected: {expected}, actual: {actual} }}")
        self.expected = expected
        self.actual = actual


class UnsupportedType(QuantError):
    def __init__(self, tensor_type):
        super().__init__(f"UnsupportedType({tensor_type!r})")
        self.tensor_type = tensor_type


class InvalidInput(QuantError):
    pass


def _as_u8(data) -> np.ndarray:
    if isinstance(data, np.ndarray):
        return np.ascontiguousarray(data.view(np.uint8).ravel())
    return np.frombuffer(bytes(data), dtype=np.uint8)


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a.size else None


# ---- device memory ----------------------------------------------------------------

class DeviceBuffer:
    """Owned device allocation (openmini_qmm_malloc / openmini_qmm_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(lib().openmini_qmm_malloc(ctypes.byref(self.ptr), self.nbytes))

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().openmini_qmm_memcpy_h2d(self.ptr, _ptr(a), a.nbytes, stream))

    def download(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib().openmini_qmm_memcpy_d2h(_ptr(out), self.ptr, out.nbytes, stream))
        return out

    def fill(self, byte: int, stream=None) -> None:
        check(lib().openmini_qmm_memset(self.ptr, byte, self.nbytes, stream))

    def free(self) -> None:
        if self.ptr:
            lib().openmini_qmm_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(lib().openmini_qmm_stream_create(ctypes.byref(self.handle)))

    def synchronize(self) -> None:
        check(lib().openmini_qmm_stream_synchronize(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().openmini_qmm_stream_destroy(self.handle)
        except Exception:
            pass


def stream_copy(dst: DeviceBuffer, src: DeviceBuffer, nbytes: int, stream=None) -> None:
    """The streaming-copy yardstick kernel (openmini_qmm_stream_copy): `nbytes` read and
    written once, the reference reading for HBM traffic counters."""
    assert nbytes <= src.nbytes and nbytes <= dst.nbytes
    check(lib().openmini_qmm_stream_copy(dst.ptr, src.ptr, nbytes, stream))


def stream_read(src: DeviceBuffer, nbytes: int, sink: DeviceBuffer, stream=None) -> None:
    """The read-only streaming yardstick (openmini_qmm_stream_read): `nbytes` read once,
    nothing written; the single-launch floor of a read-bound kernel of that size."""
    assert nbytes <= src.nbytes and sink.nbytes >= 4
    check(lib().openmini_qmm_stream_read(src.ptr, nbytes, sink.ptr, stream))

def gemm_ceiling(qtype: int, m: int, n: int, k: int, sink: DeviceBuffer, stream=None) -> None:
    """The prefill GEMM's compute-only ceiling (openmini_qmm_gemm_ceiling): its grid and
    per-block register work for an m x n x k Q4_0 / Q8_0 problem, without memory
    traffic.  `sink` (4 bytes) is written only if a sentinel is hit."""
    check(lib().openmini_qmm_gemm_ceiling(int(qtype), int(m), int(n), int(k), sink.ptr, stream))


def init(device: int = 0) -> None:
    check(lib().openmini_qmm_init(device))


# ---- weights ------------------------------------------------------------------------

class QuantizedWeight:
    """A GGUF Q4_0 / Q4_1 / Q8_0 / Q4_K / Q5_K / Q6_K / Q8_K tensor W[n_rows, k_cols]
    uploaded and repacked in HBM, served by the decode GEMV and (all but Q4_1 / Q5_K,
    whose blocks carry a minimum) the prefill GEMM; dequantize() takes Q4_0 and Q8_0
    handles, and Q8_K ones (stored as the Q8_0 blocks of the same values).

    Replaces QuantizedWeightLoader::load_tensor_data (quant_loader.rs:76-92), which
    dequantizes to f32 at load; here the raw blocks stay quantized on the GPU."""

    def __init__(self, tensor_type: int, gguf_blocks, n_rows: int, k_cols: int):
        data = _as_u8(gguf_blocks)
        self.handle = ctypes.c_void_p()
        check(lib().openmini_qmm_upload(int(tensor_type), _ptr(data), data.size, int(n_rows),
                                        int(k_cols), ctypes.byref(self.handle)))
        self.tensor_type = GgufTensorType(int(tensor_type))
        self.n_rows = int(n_rows)
        self.k_cols = int(k_cols)

    @classmethod
    def from_device(cls, tensor_type: int, d_blocks: DeviceBuffer, nbytes: int, n_rows: int,
                    k_cols: int, stream=None) -> "QuantizedWeight":
        self = cls.__new__(cls)
        self.handle = ctypes.c_void_p()
        check(lib().openmini_qmm_upload_device(int(tensor_type), d_blocks.ptr, int(nbytes),
                                               int(n_rows), int(k_cols), stream,
                                               ctypes.byref(self.handle)))
        self.tensor_type = GgufTensorType(int(tensor_type))
        self.n_rows, self.k_cols = int(n_rows), int(k_cols)
        return self

    @classmethod
    def from_device_into(cls, tensor_type: int, d_blocks: DeviceBuffer, nbytes: int, n_rows: int,
                         k_cols: int, d_mem: DeviceBuffer, offset: int = 0, stream=None) -> "QuantizedWeight":
        """Uploads into caller memory: `offset` bytes into `d_mem` (256-byte aligned),
        weight_device_bytes(...) long (openmini_qmm_upload_device_into).  The weight
        must be closed before d_mem is freed."""
        if offset < 0 or offset % 256:
            raise InvalidInput(f"offset {offset} is not a non-negative multiple of 256")
        self = cls.__new__(cls)
        self.handle = ctypes.c_void_p()
        check(lib().openmini_qmm_upload_device_into(int(tensor_type), d_blocks.ptr, int(nbytes), int(n_rows),
                                                    int(k_cols), ctypes.c_void_p(d_mem.ptr.value + offset),
                                                    max(0, d_mem.nbytes - offset), stream,
                                                    ctypes.byref(self.handle)))
        self.tensor_type = GgufTensorType(int(tensor_type))
        self.n_rows, self.k_cols = int(n_rows), int(k_cols)
        return self

    def gemm_min_rows(self) -> int:
        """The fewest activation rows from which linear() runs the fp32 prefill GEMM on
        this weight (openmini_qmm_gemm_min_rows): between GEMM_MIN_ROWS_LOW and
        GEMM_MIN_ROWS by the weight's shape, 0 for the block-minimum types (never)."""
        t = lib().openmini_qmm_gemm_min_rows(self.handle)
        check(t if t < 0 else 0)
        return int(t)

    def prefill_gemm(self, m: int) -> bool:
        """Whether linear() on m rows of this weight runs the fp32 prefill GEMM (the
        library's rule, asked of the library)."""
        t = self.gemm_min_rows()
        return t > 0 and m >= t

    def info(self) -> _native.WeightInfo:
        info = _native.WeightInfo()
        check(lib().openmini_qmm_weight_info(self.handle, ctypes.byref(info)))
        return info

    def dequantize(self) -> np.ndarray:
        """f32 W[n_rows, k_cols], bit-identical to quant::dequantize of the blocks."""
        out = DeviceBuffer(self.n_rows * self.k_cols * 4)
        check(lib().openmini_qmm_dequant_weight(self.handle, out.ptr, None))
        return out.download(np.float32, (self.n_rows, self.k_cols))

    def gemv(self, d_x: DeviceBuffer, d_y: DeviceBuffer, batch: int, stream=None) -> None:
        check(lib().openmini_qmm_gemv(self.handle, d_x.ptr, d_y.ptr, int(batch), stream))

    def gemm_bf16(self, d_x: DeviceBuffer, d_y: DeviceBuffer, m: int, stream=None) -> None:
        check(lib().openmini_qmm_gemm_bf16(self.handle, d_x.ptr, d_y.ptr, int(m), stream))

    def gemm_f32(self, d_x: DeviceBuffer, d_y: DeviceBuffer, m: int, d_work: "DeviceBuffer" = None,
                 stream=None) -> None:
        """Prefill GEMM on fp32 activations (openmini_qmm_gemm_f32); allocates the
        workspace when none is given."""
        work = d_work if d_work is not None else gemm_f32_workspace(int(m), self.k_cols)
        check(lib().openmini_qmm_gemm_f32(self.handle, d_x.ptr, d_y.ptr, int(m), work.ptr, work.nbytes, stream))

    def close(self) -> None:
        if self.handle:
            lib().openmini_qmm_free_weight(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def weight_device_bytes(tensor_type: int, n_rows: int, k_cols: int) -> int:
    """Device bytes an uploaded weight of this type and shape occupies
    (openmini_qmm_weight_device_bytes): the size QuantizedWeight.from_device_into needs."""
    out = ctypes.c_size_t()
    check(lib().openmini_qmm_weight_device_bytes(int(tensor_type), int(n_rows), int(k_cols), ctypes.byref(out)))
    return int(out.value)


def gemm_f32_workspace(m: int, k_cols: int) -> DeviceBuffer:
    """A device workspace for openmini_qmm_gemm_f32 / _ffn_gate_up_f32 (256-byte aligned:
    the device allocator's granularity)."""
    nbytes = int(lib().openmini_qmm_gemm_f32_workspace_bytes(int(m), int(k_cols)))
    if nbytes == 0:
        raise InvalidInput(f"no workspace for m={m}, K={k_cols}")
    return DeviceBuffer(nbytes)


# Rows from which the host calls run the fp32 prefill GEMM instead of the decode GEMVs
# (the library's own threshold for openmini_qmm_linear_host): per weight,
# QuantizedWeight.gemm_min_rows(), between GEMM_MIN_ROWS_LOW and GEMM_MIN_ROWS.
GEMM_MIN_ROWS = 128
GEMM_MIN_ROWS_LOW = 64


# ---- quant_simd safe API (validated dequantization) on the GPU ----------------------

def dequantize(data, tensor_type, n: int) -> np.ndarray:
    """quant::dequantize (quant.rs:56-79), which dequantize_simd (quant_simd.rs:304-313)
    matches value for value: the blocks that fit in `data` are dequantized, the rest
    of the n outputs are 0.0; bit-identical to the reference.  F32 / F16 input shorter
    than n elements: the whole elements, then 0.0 (dequantize_simd's fixed-length
    result, quant_simd.rs:332-340; quant::dequantize_f32 / _f16, quant.rs:95-133,
    return the same leading values without the zero tail).  Types the library does
    not implement raise UnsupportedType (the reference returns zeros)."""
    tt = int(tensor_type)
    buf = _as_u8(data)
    out = np.empty(max(int(n), 0), dtype=np.float32)
    rc = lib().openmini_qmm_dequantize_any(tt, _ptr(buf), buf.size, int(n), _ptr(out) if n else None)
    if rc == _native.ERR_UNSUPPORTED:
        raise UnsupportedType(tensor_type)
    check(rc)
    return out


dequantize_simd = dequantize


def safe_dequantize(data, tensor_type, n: int) -> np.ndarray:
    """quant_simd::safe_dequantize (quant_simd.rs:284-302): n == 0 -> empty;
    Q4_0 / Q8_0 / Q4_1: short input -> InsufficientData{expected, actual};
    F16 / F32: dequantize_simd without a length check (:293-299); other types ->
    UnsupportedType."""
    tt = int(tensor_type)
    if tt in (GgufTensorType.F16, GgufTensorType.F32):
        return dequantize(data, tt, n)
    if tt not in (GgufTensorType.Q4_0, GgufTensorType.Q8_0, GgufTensorType.Q4_1):
        raise UnsupportedType(tensor_type)
    buf = _as_u8(data)
    out = np.empty(max(int(n), 0), dtype=np.float32)
    expected = ctypes.c_size_t(0)
    rc = lib().openmini_qmm_dequantize(tt, _ptr(buf), buf.size, int(n),
                                       _ptr(out) if n else None, ctypes.byref(expected))
    if rc == _native.ERR_INSUFFICIENT_DATA:
        raise InsufficientData(expected.value, buf.size)
    if rc == _native.ERR_UNSUPPORTED:
        raise UnsupportedType(tensor_type)
    check(rc)
    return out


def safe_dequantize_q4_0(data, n: int) -> np.ndarray:
    return safe_dequantize(data, GgufTensorType.Q4_0, n)


def safe_dequantize_q8_0(data, n: int) -> np.ndarray:
    return safe_dequantize(data, GgufTensorType.Q8_0, n)


def safe_dequantize_q4_1(data, n: int) -> np.ndarray:
    return safe_dequantize(data, GgufTensorType.Q4_1, n)


def convert_to_soa_layout(data, tensor_type, n: int, block_size: int = 32) -> np.ndarray:
    """quant_simd::convert_to_soa_layout (quant_simd.rs:3245-3397) on the GPU: the AoS ->
    SoA byte permutation of Q4_0 / Q4_1 / Q8_0 blocks, the truncated copy of F32 / F16,
    the input itself for other types; empty for empty input or n == 0.  block_size is
    unused, as in the reference."""
    del block_size
    tt = int(tensor_type)
    buf = _as_u8(data)
    total = ctypes.c_size_t(0)
    rc = lib().openmini_qmm_soa_bytes(tt, buf.size, int(n), ctypes.byref(total))
    if rc == _native.ERR_UNSUPPORTED:
        raise UnsupportedType(tensor_type)
    check(rc)
    out = np.empty(total.value, dtype=np.uint8)
    if total.value:
        check(lib().openmini_qmm_convert_to_soa(tt, _ptr(buf), buf.size, int(n), _ptr(out)))
    return out


# ---- GpuQuantOps ----------------------------------------------------------------------

class HipQuantOps:
    """HIP implementation of trait GpuQuantOps (quant_simd.rs:2944-2986), in place of
    the CudaQuantOps stub (:3137-3188).  Rust's Result<Vec<f32>, String> maps to a
    returned array or a raised GpuQuantOpsError carrying the string.  The per-type
    calls validate their input like safe_dequantize (a short buffer is an error);
    batch_dequantize_gpu takes any implemented type with dequantize_simd's semantics,
    as the reference's working implementation does (MetalQuantOps, :3104-3118)."""

    class GpuQuantOpsError(RuntimeError):
        pass

    def _deq(self, tensor_type: int, data, n: int) -> np.ndarray:
        try:
            return safe_dequantize(data, tensor_type, n)
        except (QuantError, QmmError) as e:
            raise HipQuantOps.GpuQuantOpsError(str(e)) from e

    def dequantize_q4_0_gpu(self, data, n: int) -> np.ndarray:
        return self._deq(GgufTensorType.Q4_0, data, n)

    def dequantize_q8_0_gpu(self, data, n: int) -> np.ndarray:
        return self._deq(GgufTensorType.Q8_0, data, n)

    def dequantize_q4_1_gpu(self, data, n: int) -> np.ndarray:
        return self._deq(GgufTensorType.Q4_1, data, n)

    def batch_dequantize_gpu(self, tensors) -> list:
        try:
            return [dequantize(d, t, n) for (t, d, n) in tensors]
        except (QuantError, QmmError) as e:
            raise HipQuantOps.GpuQuantOpsError(str(e)) from e

    def is_available(self) -> bool:
        return bool(lib().openmini_qmm_is_available())

    def device_info(self) -> str:
        buf = ctypes.create_string_buffer(512)
        lib().openmini_qmm_device_info(buf, len(buf))
        return buf.value.decode()

    def estimate_memory_usage(self, total_elements: int) -> int:
        return int(lib().openmini_qmm_estimate_memory_usage(int(GgufTensorType.Q4_0),
                                                            int(total_elements)))


# ---- GemmEngine sibling ------------------------------------------------------------------

class HipQuantGemmEngine:
    """Quantized sibling of trait GemmEngine (gemm_engine.rs:37-56): the same surface
    (name, backend_type, matmul, batched_matmul, fused_gemm_relu, fused_gemm_silu,
    is_available), host arrays at the edge, the weight a device handle created at load.
    matmul(x, W) computes x . W^T for W[N, K], i.e. what linear() feeds
    GemmEngine::matmul after its W.t() copy (model.rs:1050-1064)."""

    def name(self) -> str:
        return "hip_quant"

    def backend_type(self) -> str:
        return "HipQuant"

    def is_available(self) -> bool:
        return bool(lib().openmini_qmm_is_available())

    def matmul(self, x: np.ndarray, weight: QuantizedWeight) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != weight.k_cols:
            raise InvalidInput(f"x shape {x.shape} does not match W[{weight.n_rows}, {weight.k_cols}]")
        y = np.empty((x.shape[0], weight.n_rows), dtype=np.float32)
        check(lib().openmini_qmm_linear_host(weight.handle, _ptr(x), _ptr(y), x.shape[0]))
        return y

    def batched_matmul(self, x: np.ndarray, weights) -> np.ndarray:
        """GemmEngine::batched_matmul (gemm_engine.rs:73-96): slice i of x[B, M, K] times
        W_i^T; "Batch dimension mismatch" when B differs from the number of weights."""
        x = np.asarray(x, dtype=np.float32)
        if x.ndim != 3 or x.shape[0] != len(weights):
            raise InvalidInput(f"Batch dimension mismatch: {x.shape[0] if x.ndim == 3 else x.shape} "
                               f"vs {len(weights)}")
        n = {w.n_rows for w in weights}
        if len(n) > 1:
            raise InvalidInput("batched weights differ in N")
        return np.stack([self.matmul(x[i], w) for i, w in enumerate(weights)]) if len(weights) else \
            np.zeros((0, x.shape[1], 0), np.float32)

    def fused_gemm_relu(self, x: np.ndarray, weight: QuantizedWeight, bias=None) -> np.ndarray:
        """GemmEngine::fused_gemm_relu (gemm_engine.rs:98-110): relu(x . W^T + bias)."""
        y = self.matmul(x, weight)
        if bias is not None:
            y = y + np.asarray(bias, dtype=np.float32)
        return np.maximum(y, np.float32(0.0))

    def fused_gemm_silu(self, x: np.ndarray, gate: QuantizedWeight, up: QuantizedWeight,
                        bias=None) -> np.ndarray:
        """FFNWeights::forward's hidden state silu(x . Wg^T) * (x . Wu^T) (+ bias)
        (model.rs:728-731): gate and up in one launch (openmini_qmm_ffn_gate_up), or from
        the gate weight's gemm_min_rows() rows on the fp32 prefill GEMMs
        (openmini_qmm_ffn_gate_up_f32).  The
        ndarray fallback's fused_gemm_silu (gemm_engine.rs:112-130) computes
        gate * silu(up) on untransposed weights instead; that branch is not followed."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != gate.k_cols or (gate.n_rows, gate.k_cols) != (up.n_rows, up.k_cols):
            raise InvalidInput(f"x {x.shape}, gate [{gate.n_rows}, {gate.k_cols}], up [{up.n_rows}, "
                               f"{up.k_cols}] do not match")
        dx = DeviceBuffer.from_numpy(x)
        m = x.shape[0]
        dh = DeviceBuffer(m * gate.n_rows * 4)
        if gate.prefill_gemm(m):  # prefill: the fp32 GEMM pair on one split of x
            work = gemm_f32_workspace(m, gate.k_cols)
            check(lib().openmini_qmm_ffn_gate_up_f32(gate.handle, up.handle, dx.ptr, dh.ptr, m, work.ptr,
                                                      work.nbytes, None))
        else:
            check(lib().openmini_qmm_ffn_gate_up(gate.handle, up.handle, dx.ptr, dh.ptr, m, None))
        h = dh.download(np.float32, (m, gate.n_rows))
        return h + np.asarray(bias, dtype=np.float32) if bias is not None else h


_ENGINE = None


def get_gemm_engine() -> HipQuantGemmEngine:
    """Process-wide engine, like get_gemm_engine_manager() (gemm_engine.rs:471-475)."""
    global _ENGINE
    if _ENGINE is None:
        _ENGINE = HipQuantGemmEngine()
    return _ENGINE


def linear_gemm(x: np.ndarray, weight: QuantizedWeight) -> np.ndarray:
    """model.rs:1060-1064: x . W^T through the engine; errors propagate."""
    return get_gemm_engine().matmul(x, weight)


def linear(x: np.ndarray, weight: QuantizedWeight) -> np.ndarray:
    """model.rs:1050-1057.  The reference falls back to a CPU dot on engine error;
    this path has no CPU fallback, so the error propagates."""
    return get_gemm_engine().matmul(x, weight)
