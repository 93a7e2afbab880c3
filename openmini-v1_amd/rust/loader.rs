//! The loader's raw-block path: GgufFile (openmini-server/src/model/inference/
//! gguf.rs:1357-2110) and QuantizedWeightLoader (quant_loader.rs:54-138) without
//! dequantize-at-load.  Projections stay quantized on the GPU; other tensors (norms,
//! embeddings) come back as f32 through get_tensor_data_by_ref, bit-identical.
use std::collections::HashMap;
use std::ffi::CString;

use super::engine::HipQuantWeight;
use super::ffi;

pub struct HipGguf(*mut ffi::Gguf);
unsafe impl Send for HipGguf {}
unsafe impl Sync for HipGguf {}
impl Drop for HipGguf {
    fn drop(&mut self) {
        unsafe { ffi::openmini_qmm_gguf_close(self.0) }
    }
}

fn cstr(s: &str) -> Result<CString, String> {
    CString::new(s).map_err(|e| e.to_string())
}

impl HipGguf {
    /// GgufFile::open (gguf.rs:1357-1364): the reference's own dialect or standard GGUF.
    pub fn open(path: &str) -> Result<Self, String> {
        let c = cstr(path)?;
        let mut g = std::ptr::null_mut();
        ffi::check(unsafe { ffi::openmini_qmm_gguf_open(c.as_ptr(), ffi::GGUF_AUTO, &mut g) })?;
        Ok(Self(g))
    }

    pub fn tensor_info(&self, name: &str) -> Result<ffi::GgufTensorInfo, String> {
        let c = cstr(name)?;
        let mut info = ffi::GgufTensorInfo::default();
        ffi::check(unsafe { ffi::openmini_qmm_gguf_tensor_info(self.0, c.as_ptr(), &mut info) })?;
        Ok(info)
    }

    /// load_tensor (quant_loader.rs:66-92) for a projection: raw blocks -> GPU chunks.
    /// ggml ne0 is K, so dims[0] is k_cols and dims[1] is n_rows.
    pub fn load_projection(&self, name: &str) -> Result<HipQuantWeight, String> {
        let info = self.tensor_info(name)?;
        let c = cstr(name)?;
        let mut raw = std::ptr::null_mut();
        ffi::check(unsafe {
            ffi::openmini_qmm_gguf_upload_weight(self.0, c.as_ptr(), std::ptr::null_mut(), &mut raw)
        })?;
        Ok(HipQuantWeight { raw, n: info.dims[1] as usize, k: info.dims[0] as usize, tensor_type: info.tensor_type })
    }

    /// get_tensor_data_by_ref (gguf.rs:2062-2110) for a non-projection tensor: f32 on the
    /// host, dequantized on the GPU.
    pub fn tensor_f32(&self, name: &str) -> Result<Vec<f32>, String> {
        let info = self.tensor_info(name)?;
        let n = info.n_elements as usize;
        let mut d: *mut std::os::raw::c_void = std::ptr::null_mut();
        ffi::check(unsafe { ffi::openmini_qmm_malloc(&mut d, n.max(1) * 4) })?;
        let c = cstr(name)?;
        let mut out = vec![0f32; n];
        let r = unsafe { ffi::openmini_qmm_gguf_dequantize_tensor(self.0, c.as_ptr(), d.cast(), std::ptr::null_mut()) };
        let r = ffi::check(r).and_then(|_| {
            ffi::check(unsafe { ffi::openmini_qmm_memcpy_d2h(out.as_mut_ptr().cast(), d, n * 4, std::ptr::null_mut()) })
        });
        unsafe { ffi::openmini_qmm_free(d) };
        r.map(|_| out)
    }

    /// QuantizedWeightLoader::load_attention_weights (quant_loader.rs:95-115): the four
    /// attention projections of layer `layer`, by the reference's tensor names.
    pub fn load_attention_weights(&self, layer: usize) -> Result<HashMap<&'static str, HipQuantWeight>, String> {
        let mut m = HashMap::new();
        for p in ["q_proj", "k_proj", "v_proj", "o_proj"] {
            m.insert(p, self.load_projection(&format!("model.layers.{layer}.attention.{p}"))?);
        }
        Ok(m)
    }

    /// QuantizedWeightLoader::load_ffn_weights (quant_loader.rs:117-138).
    pub fn load_ffn_weights(&self, layer: usize) -> Result<HashMap<&'static str, HipQuantWeight>, String> {
        let mut m = HashMap::new();
        for p in ["gate_proj", "up_proj", "down_proj"] {
            m.insert(p, self.load_projection(&format!("model.layers.{layer}.ffn.{p}"))?);
        }
        Ok(m)
    }

    /// QuantizedWeightLoader::has_tensor (quant_loader.rs:297-299).
    pub fn has_tensor(&self, name: &str) -> bool {
        self.tensor_info(name).is_ok()
    }

    /// QuantizedModelLoader::load_layer (quant_loader.rs:439-484): the seven projections
    /// uploaded quantized and the two norm vectors as f32 (load_norm_weights,
    /// quant_loader.rs:278-286).  MLA / MoE tensors, which the reference also loads when
    /// present, are outside the quantized linear layer: reported, not loaded.
    pub fn load_layer(&self, layer: usize) -> Result<HipLayerWeights, String> {
        Ok(HipLayerWeights {
            attention: self.load_attention_weights(layer)?,
            ffn: self.load_ffn_weights(layer)?,
            input_layernorm: self.tensor_f32(&format!("model.layers.{layer}.input_layernorm"))?,
            post_attention_layernorm: self.tensor_f32(&format!("model.layers.{layer}.post_attention_layernorm"))?,
            has_mla: self.has_tensor(&format!("model.layers.{layer}.attention.mla.q_proj")),
            has_moe: self.has_tensor(&format!("model.layers.{layer}.moe.router")),
        })
    }
}

/// QuantizedLayerWeights (quant_loader.rs:24-44) with the projections on the GPU.
pub struct HipLayerWeights {
    pub attention: HashMap<&'static str, HipQuantWeight>,
    pub ffn: HashMap<&'static str, HipQuantWeight>,
    pub input_layernorm: Vec<f32>,
    pub post_attention_layernorm: Vec<f32>,
    pub has_mla: bool,
    pub has_moe: bool,
}
