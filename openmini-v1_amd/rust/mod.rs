//! src/model/inference/hip_quant/: the MI355X quantized linear layer behind the
//! `hip-quant` cargo feature (declared from src/model/inference/mod.rs as
//! `#[cfg(feature = "hip-quant")] pub mod hip_quant;`).
pub mod engine;
pub mod ffi;
pub mod gpu_quant_ops;
pub mod layer;
pub mod loader;

pub use engine::{hip_engine, HipQuantGemmEngine, HipQuantWeight, QuantGemmEngine};
pub use gpu_quant_ops::HipQuantOps;
pub use loader::HipGguf;
