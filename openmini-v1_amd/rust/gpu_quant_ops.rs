//! GpuQuantOps (openmini-server/src/model/inference/quant_simd.rs:2944-2986) on the
//! GPU: replaces the CudaQuantOps stub (quant_simd.rs:3157-3188).
use super::ffi;
use crate::model::inference::gguf::GgufTensorType;
use crate::model::inference::quant_simd::GpuQuantOps;

pub struct HipQuantOps;

/// quant_simd::safe_dequantize semantics (quant_simd.rs:150-302): n = 0 -> empty;
/// short input -> ERR_INSUFFICIENT_DATA with the expected byte count in the message.
fn deq(t: i32, data: &[u8], n: usize) -> Result<Vec<f32>, String> {
    let mut out = vec![0f32; n];
    let mut expected = 0usize;
    ffi::check(unsafe {
        ffi::openmini_qmm_dequantize(t, data.as_ptr().cast(), data.len(), n, out.as_mut_ptr(), &mut expected)
    })?;
    Ok(out)
}

impl GpuQuantOps for HipQuantOps {
    fn dequantize_q4_0_gpu(&self, data: &[u8], n: usize) -> Result<Vec<f32>, String> {
        deq(ffi::Q4_0, data, n)
    }
    fn dequantize_q8_0_gpu(&self, data: &[u8], n: usize) -> Result<Vec<f32>, String> {
        deq(ffi::Q8_0, data, n)
    }
    fn dequantize_q4_1_gpu(&self, data: &[u8], n: usize) -> Result<Vec<f32>, String> {
        deq(ffi::Q4_1, data, n)
    }
    /// quant_simd.rs:3104-3118 runs dequantize_simd per tensor: every layout, zero tail
    /// on short input, no InsufficientData.
    fn batch_dequantize_gpu(&self, ts: &[(GgufTensorType, &[u8], usize)]) -> Result<Vec<Vec<f32>>, String> {
        ts.iter()
            .map(|(t, d, n)| {
                let mut out = vec![0f32; *n];
                ffi::check(unsafe {
                    ffi::openmini_qmm_dequantize_any(*t as i32, d.as_ptr().cast(), d.len(), *n, out.as_mut_ptr())
                })?;
                Ok(out)
            })
            .collect()
    }
    fn is_available(&self) -> bool {
        unsafe { ffi::openmini_qmm_is_available() == 1 }
    }
    fn device_info(&self) -> String {
        let mut buf = [0 as std::os::raw::c_char; 256];
        unsafe { ffi::openmini_qmm_device_info(buf.as_mut_ptr(), buf.len()) };
        unsafe { std::ffi::CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned()
    }
    fn estimate_memory_usage(&self, n: usize) -> usize {
        unsafe { ffi::openmini_qmm_estimate_memory_usage(ffi::Q4_0, n) }
    }
}

/// quant_simd::convert_to_soa_layout (quant_simd.rs:3245-3397) with the byte permutation
/// on the GPU; byte-identical output.
pub fn convert_to_soa_layout(data: &[u8], tensor_type: GgufTensorType, n: usize, _block_size: usize) -> Vec<u8> {
    let t = tensor_type as i32;
    let mut len = 0usize;
    if unsafe { ffi::openmini_qmm_soa_bytes(t, data.len(), n, &mut len) } != ffi::OK || len == 0 {
        return Vec::new();
    }
    let mut out = vec![0u8; len];
    let rc = unsafe {
        ffi::openmini_qmm_convert_to_soa(t, data.as_ptr().cast(), data.len(), n, out.as_mut_ptr().cast())
    };
    if let Err(e) = ffi::check(rc) {
        panic!("convert_to_soa_layout: {e}");
    }
    out
}
