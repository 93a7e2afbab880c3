"""Host mirror of the reference's GGUF reader and weight loader over the C-ABI.

  GgufFile                    src/model/inference/gguf.rs:1357-2110 (open, tensors,
                              metadata getters, get_tensor_data, get_tensor_data_by_ref)
  QuantizedWeightLoader       src/model/inference/quant_loader.rs:54-138 (open,
                              load_tensor, load_attention_weights, load_ffn_weights)

The difference from the reference is the one this library exists for: load_tensor
returns a QuantizedWeight resident on the GPU (raw blocks, repacked there) instead of
an f32 array dequantized at load.  get_tensor_data_by_ref keeps the reference's f32
result, computed on the GPU.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native
from ._native import check, lib
from .ops import QuantizedWeight

AUTO, REFERENCE, STANDARD = 0, 1, 2
VALUE_TYPES = ("UInt8", "Int8", "UInt16", "Int16", "UInt32", "Int32", "Float32", "Bool", "String",
               "Array", "UInt64", "Int64", "Float64")  # gguf.rs:73-101


class GgufError(RuntimeError):
    """anyhow errors of GgufFile (message kept) / QuantizedWeightLoader."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _call(status: int) -> None:
    if status != _native.OK:
        raise GgufError(status, _native.last_error())


class GgufTensor:
    """GgufTensor (gguf.rs:411-439): name, dims (GGUF order), tensor_type, offset."""

    def __init__(self, name: str, info: _native.GgufTensorInfo):
        self.name = name
        self.dims = [int(info.dims[i]) for i in range(info.n_dims)]
        self.tensor_type = int(info.type)
        self.offset = int(info.offset)
        self._n = int(info.n_elements)
        self._size = int(info.data_size)

    def num_elements(self) -> int:
        return self._n

    def data_size(self) -> int:
        return self._size


class GgufFile:
    def __init__(self, path: str, dialect: int = AUTO):
        self.handle = ctypes.c_void_p()
        _call(lib().openmini_qmm_gguf_open(str(path).encode(), int(dialect), ctypes.byref(self.handle)))
        h = _native.GgufHeader()
        check(lib().openmini_qmm_gguf_header(self.handle, ctypes.byref(h)))
        self.version, self.dialect = int(h.version), int(h.dialect)
        self.tensor_count, self.metadata_kv_count = int(h.tensor_count), int(h.metadata_kv_count)
        self.alignment = int(h.alignment)
        self.tensors = {}
        buf = ctypes.create_string_buffer(4096)
        for i in range(int(h.distinct_tensors)):
            _call(lib().openmini_qmm_gguf_tensor_name(self.handle, i, buf, len(buf)))
            name = buf.value.decode()
            info = _native.GgufTensorInfo()
            _call(lib().openmini_qmm_gguf_tensor_info(self.handle, name.encode(), ctypes.byref(info)))
            self.tensors[name] = GgufTensor(name, info)
        self.keys = []
        for i in range(int(h.distinct_keys)):
            _call(lib().openmini_qmm_gguf_meta_key(self.handle, i, buf, len(buf)))
            self.keys.append(buf.value.decode())

    open = classmethod(lambda cls, path, dialect=AUTO: cls(path, dialect))

    # ---- GgufMetadata getters (gguf.rs:143-209): None when absent or of another type
    def get_u32(self, key: str):
        v = ctypes.c_uint32()
        return int(v.value) if lib().openmini_qmm_gguf_get_u32(self.handle, key.encode(), ctypes.byref(v)) == 0 else None

    def get_u64(self, key: str):
        v = ctypes.c_uint64()
        return int(v.value) if lib().openmini_qmm_gguf_get_u64(self.handle, key.encode(), ctypes.byref(v)) == 0 else None

    def get_f32(self, key: str):
        v = ctypes.c_float()
        return float(v.value) if lib().openmini_qmm_gguf_get_f32(self.handle, key.encode(), ctypes.byref(v)) == 0 else None

    def get_string(self, key: str):
        n = ctypes.c_size_t()
        if lib().openmini_qmm_gguf_get_string(self.handle, key.encode(), None, 0, ctypes.byref(n)) != 0:
            return None
        buf = ctypes.create_string_buffer(n.value + 1)
        check(lib().openmini_qmm_gguf_get_string(self.handle, key.encode(), buf, len(buf), ctypes.byref(n)))
        return buf.raw[: n.value].decode()

    def value_type(self, key: str):
        t, n = ctypes.c_int(), ctypes.c_uint64()
        if lib().openmini_qmm_gguf_meta_type(self.handle, key.encode(), ctypes.byref(t), ctypes.byref(n)) != 0:
            return None
        return VALUE_TYPES[t.value], int(n.value)

    # ---- data ------------------------------------------------------------------------
    def get_tensor_data(self, name: str):
        """gguf.rs:2034-2045: the tensor's bytes (a read-only view of the mapping), or
        None when the tensor is absent or its data does not fit in the file."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        if lib().openmini_qmm_gguf_tensor_data(self.handle, name.encode(), ctypes.byref(p), ctypes.byref(n)) != 0:
            return None
        if n.value == 0:
            return np.zeros(0, dtype=np.uint8)
        arr = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), shape=(n.value,))
        arr.flags.writeable = False
        return arr

    def get_tensor_data_by_ref(self, tensor: GgufTensor) -> np.ndarray:
        """gguf.rs:2062-2110: the tensor as f32, dequantized on the GPU."""
        from .ops import DeviceBuffer
        out = DeviceBuffer(max(tensor.num_elements(), 1) * 4)
        _call(lib().openmini_qmm_gguf_dequantize_tensor(self.handle, tensor.name.encode(), out.ptr, None))
        return out.download(np.float32, (tensor.num_elements(),))

    def upload_weight(self, name: str, stream=None) -> QuantizedWeight:
        h = ctypes.c_void_p()
        _call(lib().openmini_qmm_gguf_upload_weight(self.handle, name.encode(), stream, ctypes.byref(h)))
        t = self.tensors[name]
        w = QuantizedWeight.__new__(QuantizedWeight)
        w.handle = h
        from .ops import GgufTensorType
        w.tensor_type = GgufTensorType(t.tensor_type)
        w.n_rows, w.k_cols = t.dims[1], t.dims[0]
        return w

    def close(self) -> None:
        if self.handle:
            lib().openmini_qmm_gguf_close(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QuantizedWeightLoader:
    """quant_loader.rs:54-138 over a GgufFile, weights kept quantized on the GPU."""

    def __init__(self, gguf: GgufFile):
        self.gguf = gguf

    @classmethod
    def open(cls, path: str, use_simd: bool = True, dialect: int = AUTO) -> "QuantizedWeightLoader":
        return cls(GgufFile(path, dialect))

    def load_tensor(self, name: str) -> QuantizedWeight:
        if name not in self.gguf.tensors:
            raise GgufError(_native.ERR_NOT_FOUND, f"Tensor not found: {name}")
        return self.gguf.upload_weight(name)

    def load_attention_weights(self, layer_idx: int) -> dict:
        prefix = f"model.layers.{layer_idx}.attention"
        return {p: self.load_tensor(f"{prefix}.{p}") for p in ("q_proj", "k_proj", "v_proj", "o_proj")}

    def load_ffn_weights(self, layer_idx: int) -> dict:
        prefix = f"model.layers.{layer_idx}.ffn"
        return {p: self.load_tensor(f"{prefix}.{p}") for p in ("gate_proj", "up_proj", "down_proj")}

    def has_tensor(self, name: str) -> bool:
        """quant_loader.rs:297-299."""
        return name in self.gguf.tensors

    def load_norm_weights(self, name: str) -> np.ndarray:
        """quant_loader.rs:278-286: a norm vector as f32 (any stored type, dequantized on
        the GPU bit-identically to the reference's load_tensor)."""
        if name not in self.gguf.tensors:
            raise GgufError(_native.ERR_NOT_FOUND, f"Tensor not found: {name}")
        return self.gguf.get_tensor_data_by_ref(self.gguf.tensors[name])

    def load_layer(self, layer_idx: int) -> "QuantizedLayerWeights":
        """QuantizedModelLoader::load_layer (quant_loader.rs:439-484): the layer's four
        attention and three FFN projections, uploaded quantized, and its two norm vectors
        (model.layers.{i}.input_layernorm, .post_attention_layernorm) as f32.  The
        reference also loads MLA (attention.mla.*) and MoE (moe.*) tensors when present;
        those are outside the quantized linear layer built here, so they are reported as
        present (has_mla / has_moe) and not loaded."""
        return QuantizedLayerWeights(
            attention=self.load_attention_weights(layer_idx),
            ffn=self.load_ffn_weights(layer_idx),
            input_layernorm=self.load_norm_weights(f"model.layers.{layer_idx}.input_layernorm"),
            post_attention_layernorm=self.load_norm_weights(f"model.layers.{layer_idx}.post_attention_layernorm"),
            has_mla=self.has_tensor(f"model.layers.{layer_idx}.attention.mla.q_proj"),
            has_moe=self.has_tensor(f"model.layers.{layer_idx}.moe.router"))


@dataclass
class QuantizedLayerWeights:
    """QuantizedLayerWeights (quant_loader.rs:24-44) with the projections as GPU handles."""
    attention: dict
    ffn: dict
    input_layernorm: np.ndarray
    post_attention_layernorm: np.ndarray
    has_mla: bool = False
    has_moe: bool = False
