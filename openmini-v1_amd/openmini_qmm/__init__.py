"""openmini_qmm: MI355X (gfx950) GGUF quantized linear layer for OpenMini-V1.

The compute path is libopenmini_qmm.so (hand-written HIP, C-ABI in
include/openmini_qmm.h); this package is its host-side mirror of the reference's
operator interface (see ops.py) plus synthetic-input helpers (synth.py).
"""
from ._native import LIB_PATH, Q4_0, Q8_0, QmmError, lib  # noqa: F401
from .layer import (AttentionWeights, FFNWeights, ffn_gate_up, ffn_gate_up_bf16,  # noqa: F401
                    ffn_gate_up_f32, gemv_multi)
from .ops import (GEMM_MIN_ROWS, GEMM_MIN_ROWS_LOW, DeviceBuffer, GgufTensorType, HipQuantGemmEngine, HipQuantOps,  # noqa: F401
                  InsufficientData, InvalidInput, QuantError, QuantizedWeight, Stream,
                  UnsupportedType, convert_to_soa_layout, dequantize, dequantize_simd,
                  get_gemm_engine, init, linear,
                  linear_gemm, safe_dequantize, safe_dequantize_q4_0, safe_dequantize_q4_1,
                  safe_dequantize_q8_0, stream_copy, stream_read,
                  gemm_ceiling, gemm_f32_workspace, weight_device_bytes)
