//! The quantized sibling of GemmEngine (openmini-server/src/model/inference/
//! gemm_engine.rs:37-56) over libopenmini_qmm: the same surface (name, backend_type,
//! matmul, batched_matmul, fused_gemm_relu, fused_gemm_silu, is_available), `Send + Sync`,
//! `&self`, InferenceResult errors, host ndarray in and out, with a device-resident
//! quantized weight W[N, K] in place of the dense right operand.  GemmBackendType
//! (gemm_engine.rs:16-23) gains a `HipQuant` variant.
use std::os::raw::c_void;
use std::sync::OnceLock;

use ndarray::{s, Array1, Array2, Array3};

use super::ffi;
use crate::model::inference::error::{InferenceError, InferenceResult};
use crate::model::inference::gemm_engine::GemmBackendType;
use crate::model::inference::gguf::GgufTensorType;

/// A GGUF Q4_0 / Q4_1 / Q8_0 / Q4_K / Q5_K / Q6_K / Q8_K tensor W[n, k] repacked in HBM; the
/// quantized data is immutable after upload (a weight that splits K in batched calls
/// also holds their scratch, which the library orders for the host-pointer calls this
/// engine makes).
pub struct HipQuantWeight {
    pub(crate) raw: *mut ffi::QWeight,
    pub n: usize,
    pub k: usize,
    /// GGUF type id (Q4_1 = 3 and Q5_K = 13 carry a block minimum: no prefill GEMM)
    pub tensor_type: i32,
}
unsafe impl Send for HipQuantWeight {}
unsafe impl Sync for HipQuantWeight {}
impl Drop for HipQuantWeight {
    fn drop(&mut self) {
        unsafe { ffi::openmini_qmm_free_weight(self.raw) }
    }
}

impl HipQuantWeight {
    /// Replaces dequantize-at-load (quant_loader.rs:76-92): the tensor's raw GGUF blocks
    /// (ggml ne0 = K, ne1 = N) stay quantized and are repacked on the GPU.
    pub fn upload(t: GgufTensorType, blocks: &[u8], n_rows: usize, k_cols: usize) -> Result<Self, String> {
        let mut raw = std::ptr::null_mut();
        ffi::check(unsafe {
            ffi::openmini_qmm_upload(t as i32, blocks.as_ptr().cast(), blocks.len(), n_rows as i64,
                                     k_cols as i64, &mut raw)
        })?;
        Ok(Self { raw, n: n_rows, k: k_cols, tensor_type: t as i32 })
    }

    /// Whether linear() on `m` rows of this weight runs the fp32 prefill GEMM, asked of
    /// the library (openmini_qmm_gemm_min_rows: between GEMM_MIN_ROWS_LOW and
    /// GEMM_MIN_ROWS by the weight's shape, 0 = never for the block-minimum types; a
    /// failed query answers no and the GEMV call that follows reports the error).
    pub fn prefill_gemm(&self, m: usize) -> bool {
        let t = unsafe { ffi::openmini_qmm_gemm_min_rows(self.raw) };
        t > 0 && m as i64 >= t
    }

    pub fn info(&self) -> Result<ffi::WeightInfo, String> {
        let mut info = ffi::WeightInfo::default();
        ffi::check(unsafe { ffi::openmini_qmm_weight_info(self.raw, &mut info) })?;
        Ok(info)
    }
}

/// An owned device allocation (openmini_qmm_malloc / openmini_qmm_free).
struct DeviceBuf(*mut c_void);
impl DeviceBuf {
    fn new(bytes: usize) -> Result<Self, String> {
        let mut p = std::ptr::null_mut();
        ffi::check(unsafe { ffi::openmini_qmm_malloc(&mut p, bytes) })?;
        Ok(Self(p))
    }
}
impl Drop for DeviceBuf {
    fn drop(&mut self) {
        unsafe { ffi::openmini_qmm_free(self.0) };
    }
}

pub trait QuantGemmEngine: Send + Sync {
    fn name(&self) -> &'static str;
    fn backend_type(&self) -> GemmBackendType;
    /// linear(x, W) = x . W^T (model.rs:1050-1064; GemmEngine::matmul on W^T).
    fn matmul(&self, x: &Array2<f32>, w: &HipQuantWeight) -> InferenceResult<Array2<f32>>;
    /// GemmEngine::batched_matmul (gemm_engine.rs:73-96): slice i of x times W_i^T, with
    /// the reference's "Batch dimension mismatch" error.
    fn batched_matmul(&self, x: &Array3<f32>, w: &[&HipQuantWeight]) -> InferenceResult<Array3<f32>>;
    /// GemmEngine::fused_gemm_relu (gemm_engine.rs:98-110): relu(x . W^T + bias).
    fn fused_gemm_relu(&self, x: &Array2<f32>, w: &HipQuantWeight, bias: Option<&Array1<f32>>)
        -> InferenceResult<Array2<f32>>;
    /// FFNWeights::forward's hidden state (model.rs:728-731): silu(x . Wg^T) * (x . Wu^T)
    /// (+ bias), gate and up in one launch (openmini_qmm_ffn_gate_up).  The ndarray
    /// fallback's fused_gemm_silu (gemm_engine.rs:112-130) computes gate * silu(up) on
    /// untransposed weights instead; the unfused branch of FFNWeights::forward is the one
    /// followed here.
    fn fused_gemm_silu(&self, x: &Array2<f32>, gate: &HipQuantWeight, up: &HipQuantWeight,
                       bias: Option<&Array1<f32>>) -> InferenceResult<Array2<f32>>;
    fn is_available(&self) -> bool;
}

pub struct HipQuantGemmEngine;

/// Rows from which the host calls run the fp32 prefill GEMM instead of the decode GEMVs
/// (openmini_qmm_linear_host makes the same choice): per weight,
/// HipQuantWeight::prefill_gemm, between GEMM_MIN_ROWS_LOW and GEMM_MIN_ROWS.
pub const GEMM_MIN_ROWS: usize = 128;
pub const GEMM_MIN_ROWS_LOW: usize = 64;

fn gen_err(e: String) -> InferenceError {
    InferenceError::generation(e)
}

impl QuantGemmEngine for HipQuantGemmEngine {
    fn name(&self) -> &'static str {
        "hip_quant"
    }

    fn backend_type(&self) -> GemmBackendType {
        GemmBackendType::HipQuant
    }

    fn matmul(&self, x: &Array2<f32>, w: &HipQuantWeight) -> InferenceResult<Array2<f32>> {
        let x = x.as_standard_layout();
        let (m, k) = x.dim();
        if k != w.k {
            return Err(InferenceError::config(format!("x has {k} columns, W has {}", w.k)));
        }
        let mut y = Array2::<f32>::zeros((m, w.n));
        if m > 0 {
            ffi::check(unsafe { ffi::openmini_qmm_linear_host(w.raw, x.as_ptr(), y.as_mut_ptr(), m as i64) })
                .map_err(gen_err)?;
        }
        Ok(y)
    }

    fn batched_matmul(&self, x: &Array3<f32>, w: &[&HipQuantWeight]) -> InferenceResult<Array3<f32>> {
        if x.shape()[0] != w.len() {
            return Err(InferenceError::config(format!("Batch dimension mismatch: {} vs {}", x.shape()[0],
                                                      w.len())));
        }
        let (b, m) = (x.shape()[0], x.shape()[1]);
        let n = w.first().map(|w| w.n).unwrap_or(0);
        if w.iter().any(|wi| wi.n != n) {
            return Err(InferenceError::config("batched weights differ in N".to_string()));
        }
        let mut y = Array3::<f32>::zeros((b, m, n));
        for (i, wi) in w.iter().enumerate() {
            let yi = self.matmul(&x.slice(s![i, .., ..]).to_owned(), wi)?;
            y.slice_mut(s![i, .., ..]).assign(&yi);
        }
        Ok(y)
    }

    fn fused_gemm_relu(&self, x: &Array2<f32>, w: &HipQuantWeight, bias: Option<&Array1<f32>>)
        -> InferenceResult<Array2<f32>> {
        let mut y = self.matmul(x, w)?;
        if let Some(b) = bias {
            y += b;
        }
        y.mapv_inplace(|v| v.max(0.0));
        Ok(y)
    }

    fn fused_gemm_silu(&self, x: &Array2<f32>, gate: &HipQuantWeight, up: &HipQuantWeight,
                       bias: Option<&Array1<f32>>) -> InferenceResult<Array2<f32>> {
        let x = x.as_standard_layout();
        let (m, k) = x.dim();
        if k != gate.k || gate.k != up.k || gate.n != up.n {
            return Err(InferenceError::config(format!(
                "x [_, {k}], gate [{}, {}], up [{}, {}] do not match", gate.n, gate.k, up.n, up.k)));
        }
        let mut h = Array2::<f32>::zeros((m, gate.n));
        if m > 0 {
            let dx = DeviceBuf::new(m * k * 4).map_err(gen_err)?;
            let dh = DeviceBuf::new(m * gate.n * 4).map_err(gen_err)?;
            unsafe {
                ffi::check(ffi::openmini_qmm_memcpy_h2d(dx.0, x.as_ptr().cast(), m * k * 4, std::ptr::null_mut()))
                    .map_err(gen_err)?;
                if gate.prefill_gemm(m) {
                    // prefill: the fp32 GEMM pair on one split of x
                    let wb = ffi::openmini_qmm_gemm_f32_workspace_bytes(m as i64, k as i64);
                    let work = DeviceBuf::new(wb).map_err(gen_err)?;
                    ffi::check(ffi::openmini_qmm_ffn_gate_up_f32(gate.raw, up.raw, dx.0.cast(), dh.0.cast(), m as i64,
                                                                 work.0, wb, std::ptr::null_mut()))
                        .map_err(gen_err)?;
                } else {
                    ffi::check(ffi::openmini_qmm_ffn_gate_up(gate.raw, up.raw, dx.0.cast(), dh.0.cast(), m as i64,
                                                             std::ptr::null_mut()))
                        .map_err(gen_err)?;
                }
                ffi::check(ffi::openmini_qmm_memcpy_d2h(h.as_mut_ptr().cast(), dh.0, m * gate.n * 4,
                                                        std::ptr::null_mut()))
                    .map_err(gen_err)?;
            }
        }
        if let Some(b) = bias {
            h += b;
        }
        Ok(h)
    }

    fn is_available(&self) -> bool {
        unsafe { ffi::openmini_qmm_is_available() == 1 }
    }
}

/// The process-wide engine, chosen once like get_gemm_engine_manager()
/// (gemm_engine.rs:373-384, 471-475): None when no gfx950 device is usable.
pub fn hip_engine() -> Option<&'static HipQuantGemmEngine> {
    static ENGINE: OnceLock<Option<HipQuantGemmEngine>> = OnceLock::new();
    ENGINE
        .get_or_init(|| {
            if unsafe { ffi::openmini_qmm_is_available() } == 1 && unsafe { ffi::openmini_qmm_init(0) } == ffi::OK {
                ffi::install_logging();
                Some(HipQuantGemmEngine)
            } else {
                None
            }
        })
        .as_ref()
}
