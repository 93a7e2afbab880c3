"""The projections of one transformer layer on quantized weights.

Mirrors the two places where src/model/inference/model.rs (openmini-server/) runs
several linear layers on one input:
  * FFNWeights::forward (model.rs:713-735): hidden = silu(x . Wg^T) * (x . Wu^T),
    out = hidden . Wd^T, silu(v) = v / (1 + exp(-v)) (model.rs:1187-1189).  The
    engine's fused_gemm_silu (gemm_engine/vulkan_backend.rs:111-131) has the same
    meaning, silu(gate) * up; here gate and up share one launch that writes `hidden` directly;
  * prepare_qkv (model.rs:1379-1410): q, k, v = linear_gemm(x, W_{q,k,v})
    (model.rs:1392-1394), here one launch for the three.  RoPE and the attention
    itself are not part of the quantized linear layer.

The host-array methods are synchronous and mirror the reference's signatures; from
the weight's gemm_min_rows() rows on (prefill: 64-128 rows by the weight's shape)
they run the fp32-activation GEMMs, below it (and for
Q4_1 / Q5_K weights, whose blocks carry a minimum) the decode GEMVs.  The *_device methods take device buffers and a stream and only enqueue
work.
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._native import check, lib
from .ops import DeviceBuffer, InvalidInput, QuantizedWeight, gemm_f32_workspace

MAX_GROUP = 4  # weights per gemv_multi launch


def gemv_multi(weights, d_x: DeviceBuffer, d_ys, batch: int, stream=None) -> None:
    """d_ys[i][batch, N_i] = x[batch, K] . W_i^T for up to 4 weights of one type and K."""
    n = len(weights)
    if n != len(d_ys):
        raise InvalidInput(f"{n} weights but {len(d_ys)} outputs")
    hs = (ctypes.c_void_p * max(n, 1))(*[w.handle.value for w in weights])
    ys = (ctypes.c_void_p * max(n, 1))(*[y.ptr.value for y in d_ys])
    check(lib().openmini_qmm_gemv_multi(hs, n, d_x.ptr, ys, int(batch), stream))


def ffn_gate_up(gate: QuantizedWeight, up: QuantizedWeight, d_x: DeviceBuffer, d_h: DeviceBuffer,
                batch: int, stream=None) -> None:
    """d_h[batch, N] = silu(x . Wg^T) * (x . Wu^T), fp32 activations (decode)."""
    check(lib().openmini_qmm_ffn_gate_up(gate.handle, up.handle, d_x.ptr, d_h.ptr, int(batch), stream))


def ffn_gate_up_bf16(gate: QuantizedWeight, up: QuantizedWeight, d_x: DeviceBuffer,
                     d_h: DeviceBuffer, m: int, stream=None) -> None:
    """The same with bf16 activations (raw bits) on the prefill GEMM."""
    check(lib().openmini_qmm_ffn_gate_up_bf16(gate.handle, up.handle, d_x.ptr, d_h.ptr, int(m), stream))


def ffn_gate_up_f32(gate: QuantizedWeight, up: QuantizedWeight, d_x: DeviceBuffer, d_h: DeviceBuffer,
                    m: int, d_work: DeviceBuffer, stream=None) -> None:
    """The same with fp32 activations on the prefill GEMM (x split once into d_work,
    gemm_f32_workspace(m, K) bytes)."""
    check(lib().openmini_qmm_ffn_gate_up_f32(gate.handle, up.handle, d_x.ptr, d_h.ptr, int(m), d_work.ptr,
                                             d_work.nbytes, stream))


def _rows(x: np.ndarray, k: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim != 2 or x.shape[1] != k or x.shape[0] < 1:
        raise InvalidInput(f"x shape {x.shape} does not match K = {k}")
    return x


class FFNWeights:
    """FFNWeights (model.rs:706-711) holding quantized gate / up / down projections:
    gate_proj, up_proj [intermediate, hidden], down_proj [hidden, intermediate]."""

    def __init__(self, gate_proj: QuantizedWeight, up_proj: QuantizedWeight,
                 down_proj: QuantizedWeight):
        if (gate_proj.n_rows, gate_proj.k_cols) != (up_proj.n_rows, up_proj.k_cols):
            raise InvalidInput("gate_proj and up_proj differ in shape")
        if down_proj.k_cols != gate_proj.n_rows:
            raise InvalidInput(f"down_proj K = {down_proj.k_cols} != intermediate {gate_proj.n_rows}")
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    @property
    def hidden_size(self) -> int:
        return self.gate_proj.k_cols

    @property
    def intermediate_size(self) -> int:
        return self.gate_proj.n_rows

    def forward_device(self, d_x: DeviceBuffer, d_h: DeviceBuffer, d_out: DeviceBuffer, batch: int,
                       stream=None) -> None:
        """out[batch, hidden] = (silu(x . Wg^T) * (x . Wu^T)) . Wd^T with fp32
        activations: one gate/up launch and one down launch per 4 rows; d_h
        [batch, intermediate] fp32 is the caller's scratch."""
        ffn_gate_up(self.gate_proj, self.up_proj, d_x, d_h, batch, stream)
        self.down_proj.gemv(d_h, d_out, batch, stream)

    def forward(self, x: np.ndarray) -> np.ndarray:
        """model.rs:713-735 on host arrays: x [seq, hidden] -> [seq, hidden]."""
        x = _rows(x, self.hidden_size)
        m = x.shape[0]
        d_x = DeviceBuffer.from_numpy(x)
        d_h = DeviceBuffer(m * self.intermediate_size * 4)
        d_out = DeviceBuffer(m * self.down_proj.n_rows * 4)
        pair_gemm, down_gemm = self.gate_proj.prefill_gemm(m), self.down_proj.prefill_gemm(m)
        if not pair_gemm and not down_gemm:
            self.forward_device(d_x, d_h, d_out, m)
        else:
            work = gemm_f32_workspace(m, max(self.hidden_size, self.intermediate_size))
            if pair_gemm:
                ffn_gate_up_f32(self.gate_proj, self.up_proj, d_x, d_h, m, work)
            else:
                ffn_gate_up(self.gate_proj, self.up_proj, d_x, d_h, m)
            if down_gemm:
                self.down_proj.gemm_f32(d_h, d_out, m, work)
            else:
                self.down_proj.gemv(d_h, d_out, m)
        return d_out.download(np.float32, (m, self.down_proj.n_rows))

    def hidden(self, x: np.ndarray) -> np.ndarray:
        """silu(x . Wg^T) * (x . Wu^T), the input of down_proj (model.rs:728-730)."""
        x = _rows(x, self.hidden_size)
        m = x.shape[0]
        d_x = DeviceBuffer.from_numpy(x)
        d_h = DeviceBuffer(m * self.intermediate_size * 4)
        if self.gate_proj.prefill_gemm(m):
            ffn_gate_up_f32(self.gate_proj, self.up_proj, d_x, d_h, m, gemm_f32_workspace(m, self.hidden_size))
        else:
            ffn_gate_up(self.gate_proj, self.up_proj, d_x, d_h, m)
        return d_h.download(np.float32, (m, self.intermediate_size))


class AttentionWeights:
    """AttentionWeights (model.rs:696-703) holding quantized q / k / v / o projections
    (o_proj may be None when only the input projections are needed)."""

    def __init__(self, q_proj: QuantizedWeight, k_proj: QuantizedWeight, v_proj: QuantizedWeight,
                 o_proj: QuantizedWeight | None = None):
        for w in (k_proj, v_proj):
            if w.k_cols != q_proj.k_cols or w.tensor_type != q_proj.tensor_type:
                raise InvalidInput("q/k/v projections must share K and type")
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = q_proj, k_proj, v_proj, o_proj

    def project_qkv_device(self, d_x: DeviceBuffer, d_q: DeviceBuffer, d_k: DeviceBuffer,
                           d_v: DeviceBuffer, batch: int, stream=None) -> None:
        gemv_multi((self.q_proj, self.k_proj, self.v_proj), d_x, (d_q, d_k, d_v), batch, stream)

    def project_qkv(self, x: np.ndarray):
        """The three linear_gemm calls of prepare_qkv (model.rs:1392-1394) before RoPE:
        x [seq, hidden] -> (q [seq, Nq], k [seq, Nk], v [seq, Nv])."""
        x = _rows(x, self.q_proj.k_cols)
        m = x.shape[0]
        d_x = DeviceBuffer.from_numpy(x)
        ws = (self.q_proj, self.k_proj, self.v_proj)
        outs = [DeviceBuffer(m * w.n_rows * 4) for w in ws]
        if self.q_proj.prefill_gemm(m):
            work = gemm_f32_workspace(m, self.q_proj.k_cols)
            for w, o in zip(ws, outs):
                w.gemm_f32(d_x, o, m, work)
        else:
            self.project_qkv_device(d_x, *outs, m)
        return tuple(o.download(np.float32, (m, w.n_rows)) for o, w in zip(outs, ws))

    def project_o(self, attn: np.ndarray) -> np.ndarray:
        """attn [seq, heads * head_dim] . Wo^T."""
        if self.o_proj is None:
            raise InvalidInput("no o_proj")
        attn = _rows(attn, self.o_proj.k_cols)
        m = attn.shape[0]
        d_a = DeviceBuffer.from_numpy(attn)
        d_o = DeviceBuffer(m * self.o_proj.n_rows * 4)
        if self.o_proj.prefill_gemm(m):
            self.o_proj.gemm_f32(d_a, d_o, m)
        else:
            self.o_proj.gemv(d_a, d_o, m)
        return d_o.download(np.float32, (m, self.o_proj.n_rows))


__all__ = ["AttentionWeights", "FFNWeights", "MAX_GROUP", "ffn_gate_up", "ffn_gate_up_bf16",
           "ffn_gate_up_f32", "gemv_multi"]
