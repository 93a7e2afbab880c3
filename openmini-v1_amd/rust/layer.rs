//! One layer's projections with activations resident on the device (FFNWeights::forward,
//! model.rs:713-735; prepare_qkv, model.rs:1379-1410).  A serving loop can capture a
//! layer's launches once in a HIP graph on its stream and replay it per token: none of
//! these calls allocates or sets memory.  Calls of 4+ rows on one weight of at most 8192
//! rows share that weight's K-split workspace, so they must be ordered (one stream, or
//! events between streams); a layer decoded on one stream satisfies that.
use std::os::raw::c_void;

use super::engine::HipQuantWeight;
use super::ffi;

/// Decode step of one layer's FFN: hidden = silu(x . Wg^T) * (x . Wu^T) (model.rs:728-731),
/// out = hidden . Wd^T.
///
/// # Safety
/// Device pointers of batch * K, batch * N_gate and batch * N_down floats on the weights'
/// device, valid until `stream` reaches the calls; d_x 16-byte aligned.
pub unsafe fn ffn_forward_device(g: &HipQuantWeight, u: &HipQuantWeight, d: &HipQuantWeight, d_x: *const f32,
                                 d_h: *mut f32, d_out: *mut f32, batch: usize, stream: *mut c_void)
                                 -> Result<(), String> {
    ffi::check(ffi::openmini_qmm_ffn_gate_up(g.raw, u.raw, d_x, d_h, batch as i64, stream))?;
    ffi::check(ffi::openmini_qmm_gemv(d.raw, d_h, d_out, batch as i64, stream))
}

/// q, k and v of prepare_qkv (model.rs:1392-1394) in one launch; RoPE follows as today.
///
/// # Safety
/// As ffn_forward_device.
pub unsafe fn qkv_device(q: &HipQuantWeight, k: &HipQuantWeight, v: &HipQuantWeight, d_x: *const f32,
                         d_q: *mut f32, d_k: *mut f32, d_v: *mut f32, batch: usize, stream: *mut c_void)
                         -> Result<(), String> {
    let ws = [q.raw as *const ffi::QWeight, k.raw, v.raw];
    let ys = [d_q, d_k, d_v];
    ffi::check(ffi::openmini_qmm_gemv_multi(ws.as_ptr(), 3, d_x, ys.as_ptr(), batch as i64, stream))
}

/// Prefill (bf16 activations, raw bits): the fp32 FFN hidden state of m rows.  The
/// prefill GEMM takes bf16 activations, so the caller converts the hidden state to bf16
/// before the down projection (openmini_qmm_gemm_bf16).
///
/// # Safety
/// As ffn_forward_device, with m rows.
pub unsafe fn ffn_hidden_prefill(g: &HipQuantWeight, u: &HipQuantWeight, d_x_bf16: *const u16, d_h: *mut f32,
                                 m: usize, stream: *mut c_void) -> Result<(), String> {
    ffi::check(ffi::openmini_qmm_ffn_gate_up_bf16(g.raw, u.raw, d_x_bf16, d_h, m as i64, stream))
}
