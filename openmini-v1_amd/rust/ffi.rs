//! FFI to libopenmini_qmm.so: a line-for-line transcription of include/openmini_qmm.h
//! (C types only).  Lives in openmini-server as src/model/inference/hip_quant/ffi.rs and
//! links through build.rs (see build.rs in this directory).  tests/test_rust_ffi.py
//! checks every declaration here against the header.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

// openmini_qmm_status_t (values shared with openmini_error_t, native/include/openmini.h:20-31)
pub const OK: c_int = 0;
pub const ERR_MEMORY: c_int = -1;
pub const ERR_INVALID_PARAM: c_int = -2;
pub const ERR_MODEL_LOAD: c_int = -3;
pub const ERR_INFERENCE: c_int = -4;
pub const ERR_UNSUPPORTED: c_int = -5;
pub const ERR_HIP: c_int = -10;
pub const ERR_INSUFFICIENT_DATA: c_int = -11;
pub const ERR_NOT_FOUND: c_int = -12;

// GgufTensorType ids (src/model/inference/gguf.rs:219-240)
pub const F32: c_int = 0;
pub const F16: c_int = 1;
pub const Q4_0: c_int = 2;
pub const Q4_1: c_int = 3;
pub const Q8_0: c_int = 7;
pub const Q2_K: c_int = 10;
pub const Q3_K: c_int = 11;
pub const Q4_K: c_int = 12;
pub const Q5_K: c_int = 13;
pub const Q6_K: c_int = 14;
pub const Q8_K: c_int = 15;

// openmini_qmm_gguf_dialect_t
pub const GGUF_AUTO: c_int = 0;
pub const GGUF_REFERENCE: c_int = 1;
pub const GGUF_STANDARD: c_int = 2;

pub const LOG_ERROR: c_int = 3;

#[repr(C)]
pub struct QWeight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct Gguf {
    _p: [u8; 0],
}

#[repr(C)]
#[derive(Default, Debug, Clone, Copy)]
pub struct WeightInfo {
    pub tensor_type: i32,
    pub device: i32,
    pub n_rows: i64,
    pub k_cols: i64,
    pub blocks_per_row: i64,
    pub gguf_bytes: usize,
    pub device_bytes: usize,
}

#[repr(C)]
#[derive(Default, Debug, Clone, Copy)]
pub struct GgufHeader {
    pub version: u32,
    pub dialect: i32,
    pub tensor_count: u64,
    pub metadata_kv_count: u64,
    pub distinct_tensors: u64,
    pub distinct_keys: u64,
    pub alignment: u32,
    pub file_size: u64,
}

#[repr(C)]
#[derive(Default, Debug, Clone, Copy)]
pub struct GgufTensorInfo {
    pub tensor_type: i32,
    pub n_dims: u32,
    pub dims: [u64; 8],
    pub offset: u64,
    pub n_elements: u64,
    pub data_size: u64,
}

pub type LogCallback = extern "C" fn(level: c_int, text: *const c_char, user_data: *mut c_void);

extern "C" {
    pub fn openmini_qmm_version() -> *const c_char;
    pub fn openmini_qmm_init(device: c_int) -> c_int;
    pub fn openmini_qmm_last_error() -> *const c_char;
    pub fn openmini_qmm_set_log_callback(callback: Option<LogCallback>, user_data: *mut c_void) -> c_int;
    pub fn openmini_qmm_is_available() -> c_int;
    pub fn openmini_qmm_device_info(buf: *mut c_char, buf_len: usize) -> c_int;
    pub fn openmini_qmm_required_bytes(tensor_type: c_int, n_elements: usize, out_bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_estimate_memory_usage(tensor_type: c_int, n_elements: usize) -> usize;
    pub fn openmini_qmm_upload(tensor_type: c_int, gguf_blocks: *const c_void, gguf_bytes: usize, n_rows: i64, k_cols: i64, out_weight: *mut *mut QWeight) -> c_int;
    pub fn openmini_qmm_upload_device(tensor_type: c_int, d_gguf_blocks: *const c_void, gguf_bytes: usize, n_rows: i64, k_cols: i64, stream: *mut c_void, out_weight: *mut *mut QWeight) -> c_int;
    pub fn openmini_qmm_weight_device_bytes(tensor_type: c_int, n_rows: i64, k_cols: i64, out_bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_upload_device_into(tensor_type: c_int, d_gguf_blocks: *const c_void, gguf_bytes: usize, n_rows: i64, k_cols: i64, d_weight_mem: *mut c_void, weight_mem_bytes: usize, stream: *mut c_void, out_weight: *mut *mut QWeight) -> c_int;
    pub fn openmini_qmm_free_weight(weight: *mut QWeight);
    pub fn openmini_qmm_weight_info(weight: *const QWeight, info: *mut WeightInfo) -> c_int;
    pub fn openmini_qmm_gemv(weight: *const QWeight, d_x: *const f32, d_y: *mut f32, batch: i64, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_gemm_bf16(weight: *const QWeight, d_x: *const u16, d_y: *mut f32, m: i64, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_gemm_f32_workspace_bytes(m: i64, k_cols: i64) -> usize;
    pub fn openmini_qmm_gemm_launch_shape(weight: *const QWeight, m: i64, split_x: c_int) -> c_int;
    pub fn openmini_qmm_gemm_min_rows(weight: *const QWeight) -> i64;
    pub fn openmini_qmm_gemm_f32(weight: *const QWeight, d_x: *const f32, d_y: *mut f32, m: i64, d_work: *mut c_void, work_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_gemv_multi(weights: *const *const QWeight, count: c_int, d_x: *const f32, d_ys: *const *mut f32, batch: i64, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_ffn_gate_up(gate: *const QWeight, up: *const QWeight, d_x: *const f32, d_h: *mut f32, batch: i64, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_ffn_gate_up_bf16(gate: *const QWeight, up: *const QWeight, d_x: *const u16, d_h: *mut f32, m: i64, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_ffn_gate_up_f32(gate: *const QWeight, up: *const QWeight, d_x: *const f32, d_h: *mut f32, m: i64, d_work: *mut c_void, work_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_linear_host(weight: *const QWeight, x: *const f32, y: *mut f32, m: i64) -> c_int;
    pub fn openmini_qmm_linear_host_noalloc(weight: *const QWeight, x: *const f32, y: *mut f32, m: i64) -> c_int;
    pub fn openmini_qmm_dequant_weight(weight: *const QWeight, d_out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_dequantize_device(tensor_type: c_int, d_gguf: *const c_void, gguf_bytes: usize, n: usize, d_out: *mut f32, stream: *mut c_void, expected_bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_dequantize(tensor_type: c_int, gguf: *const c_void, gguf_bytes: usize, n: usize, out: *mut f32, expected_bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_dequantize_any_device(tensor_type: c_int, d_gguf: *const c_void, gguf_bytes: usize, n: usize, d_out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_dequantize_any(tensor_type: c_int, gguf: *const c_void, gguf_bytes: usize, n: usize, out: *mut f32) -> c_int;
    pub fn openmini_qmm_soa_bytes(tensor_type: c_int, len: usize, n: usize, out_bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_convert_to_soa_device(tensor_type: c_int, d_data: *const c_void, len: usize, n: usize, d_out: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_convert_to_soa(tensor_type: c_int, data: *const c_void, len: usize, n: usize, out: *mut c_void) -> c_int;
    pub fn openmini_qmm_gguf_open(path: *const c_char, dialect: c_int, out_gguf: *mut *mut Gguf) -> c_int;
    pub fn openmini_qmm_gguf_close(gguf: *mut Gguf);
    pub fn openmini_qmm_gguf_header(gguf: *const Gguf, header: *mut GgufHeader) -> c_int;
    pub fn openmini_qmm_gguf_tensor_name(gguf: *const Gguf, index: usize, buf: *mut c_char, buf_len: usize) -> c_int;
    pub fn openmini_qmm_gguf_tensor_info(gguf: *const Gguf, name: *const c_char, info: *mut GgufTensorInfo) -> c_int;
    pub fn openmini_qmm_gguf_tensor_data(gguf: *const Gguf, name: *const c_char, data: *mut *const c_void, bytes: *mut usize) -> c_int;
    pub fn openmini_qmm_gguf_meta_key(gguf: *const Gguf, index: usize, buf: *mut c_char, buf_len: usize) -> c_int;
    pub fn openmini_qmm_gguf_meta_type(gguf: *const Gguf, key: *const c_char, value_type: *mut c_int, array_len: *mut u64) -> c_int;
    pub fn openmini_qmm_gguf_get_u32(gguf: *const Gguf, key: *const c_char, out: *mut u32) -> c_int;
    pub fn openmini_qmm_gguf_get_u64(gguf: *const Gguf, key: *const c_char, out: *mut u64) -> c_int;
    pub fn openmini_qmm_gguf_get_f32(gguf: *const Gguf, key: *const c_char, out: *mut f32) -> c_int;
    pub fn openmini_qmm_gguf_get_string(gguf: *const Gguf, key: *const c_char, buf: *mut c_char, buf_len: usize, out_len: *mut usize) -> c_int;
    pub fn openmini_qmm_gguf_upload_weight(gguf: *const Gguf, name: *const c_char, stream: *mut c_void, out_weight: *mut *mut QWeight) -> c_int;
    pub fn openmini_qmm_gguf_dequantize_tensor(gguf: *const Gguf, name: *const c_char, d_out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_malloc(d_ptr: *mut *mut c_void, bytes: usize) -> c_int;
    pub fn openmini_qmm_free(d_ptr: *mut c_void) -> c_int;
    pub fn openmini_qmm_memcpy_h2d(d_dst: *mut c_void, src: *const c_void, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_memcpy_d2h(dst: *mut c_void, d_src: *const c_void, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_memset(d_dst: *mut c_void, value: c_int, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_stream_create(out_stream: *mut *mut c_void) -> c_int;
    pub fn openmini_qmm_stream_destroy(stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_stream_synchronize(stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_stream_copy(d_dst: *mut c_void, d_src: *const c_void, bytes: usize, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_stream_read(d_src: *const c_void, bytes: usize, d_sink: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn openmini_qmm_gemm_ceiling(tensor_type: c_int, m: i64, n: i64, k: i64, d_sink: *mut c_void, stream: *mut c_void) -> c_int;
}

/// Status -> Result with the calling thread's openmini_qmm_last_error() message.
pub fn check(status: c_int) -> Result<(), String> {
    if status == OK {
        return Ok(());
    }
    let msg = unsafe { std::ffi::CStr::from_ptr(openmini_qmm_last_error()) };
    Err(format!("openmini_qmm status {status}: {}", msg.to_string_lossy()))
}

/// Library failures into the server's `log` crate, as openmini_set_log_callback does for
/// the reference's native layer (native/include/openmini.h:151-155).
extern "C" fn to_log(level: c_int, text: *const c_char, _user: *mut c_void) {
    let msg = unsafe { std::ffi::CStr::from_ptr(text) }.to_string_lossy();
    if level >= LOG_ERROR {
        log::error!("openmini_qmm: {msg}")
    } else {
        log::info!("openmini_qmm: {msg}")
    }
}

pub fn install_logging() {
    unsafe {
        openmini_qmm_set_log_callback(Some(to_log), std::ptr::null_mut());
    }
}
