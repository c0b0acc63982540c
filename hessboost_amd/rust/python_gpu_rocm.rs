//! The ROCm arm of the Python package's `GpuModel` (python/src/gpu.rs:29-150):
//! `device="rocm"` / `"rocm:<ordinal>"` for batch prediction from Python.
//!
//! This file is `python/src/gpu_rocm.rs` of hessboost's Python extension,
//! declared in `python/src/lib.rs` as `mod gpu_rocm;`, compiled on every
//! platform (the arms below refuse where the `rocm` feature is off, as the
//! CUDA arms do). The extension's `Cargo.toml` forwards a `rocm` feature to
//! the `hessboost` crate, as it forwards `cuda`.
//!
//! `python/src/gpu.rs` gains one line per match, each calling into this
//! module:
//!
//! - `enum Backend` gains `Rocm { ordinal: usize }`;
//! - `Backend::parse` (`gpu.rs:47-66`): `Ok(Device::Rocm { ordinal }) =>
//!   Ok(Self::Rocm { ordinal })`, and the refusal's list of spellings adds
//!   `"rocm"` and `"rocm:<ordinal>"`;
//! - `Backend::available` (`:71-84`): `Self::Rocm { ordinal } =>
//!   gpu_rocm::available(ordinal)`;
//! - `Backend::device_name` (`:87-100`): `Self::Rocm { ordinal } =>
//!   gpu_rocm::device_name(ordinal)`;
//! - `enum Predictor` gains `Rocm(gpu_rocm::Model)`;
//! - `Predictor::build` (`:106-127`): `Backend::Rocm { ordinal } =>
//!   gpu_rocm::build(py, model, ordinal).map(Self::Rocm)`;
//! - `Predictor::model` / `device` / `predict` (`:129-170`): `Self::Rocm(gpu)
//!   => gpu_rocm::model(gpu)`, `=> "rocm"`, and `=> gpu_rocm::predict(gpu,
//!   data, iterations, margin)`.
//!
//! `GpuModel.predict(data, kind, iteration_range)` then returns the margins or
//! values of a model uploaded to the MI355X, shaped as for the other
//! backends and bit-identical to the CPU's (the objective's transform runs on
//! the CPU, as for CUDA).

use hessboost::error::Result;
use hessboost::model::{BoostedModel, Iterations, Predictions};
use pyo3::prelude::*;

#[cfg(all(target_os = "linux", feature = "rocm"))]
use crate::errors::DetachExt;
#[cfg(not(all(target_os = "linux", feature = "rocm")))]
use crate::errors::refuse;

/// Why an extension built without ROCm refuses it.
#[cfg(not(all(target_os = "linux", feature = "rocm")))]
const WITHOUT_ROCM: &str = "this hessboost extension was built without ROCm (build it on Linux with the \
                            `rocm` feature and libhbrocm.so on HBROCM_LIB_DIR)";

/// A model uploaded to a ROCm device.
#[cfg(all(target_os = "linux", feature = "rocm"))]
pub(crate) type Model = hessboost::backend::rocm::RocmModel;

/// Where the backend is not compiled in no model is ever built; the type
/// keeps `Predictor`'s arm well-formed.
#[cfg(not(all(target_os = "linux", feature = "rocm")))]
pub(crate) enum Model {}

/// Whether `rocm:<ordinal>` predicts here: the library loads and the device
/// exists.
pub(crate) fn available(ordinal: usize) -> bool {
    #[cfg(all(target_os = "linux", feature = "rocm"))]
    {
        hessboost::backend::rocm::available(ordinal)
    }
    #[cfg(not(all(target_os = "linux", feature = "rocm")))]
    {
        let _ = ordinal;
        false
    }
}

/// The device's name and architecture (for diagnostics and benchmarks).
pub(crate) fn device_name(ordinal: usize) -> Option<String> {
    #[cfg(all(target_os = "linux", feature = "rocm"))]
    {
        hessboost::backend::rocm::device_name(ordinal)
    }
    #[cfg(not(all(target_os = "linux", feature = "rocm")))]
    {
        let _ = ordinal;
        None
    }
}

/// `model` uploaded to `rocm:<ordinal>` (`BoostedModel::to_rocm`), without
/// the GIL.
pub(crate) fn build(py: Python<'_>, model: &BoostedModel, ordinal: usize) -> PyResult<Model> {
    #[cfg(all(target_os = "linux", feature = "rocm"))]
    {
        py.detached(|| model.to_rocm(ordinal))
    }
    #[cfg(not(all(target_os = "linux", feature = "rocm")))]
    {
        let _ = (py, model);
        Err(refuse(format!("ROCm GPU prediction (device \"rocm:{ordinal}\") is unavailable: {WITHOUT_ROCM}")))
    }
}

/// The uploaded model.
pub(crate) fn model(gpu: &Model) -> &BoostedModel {
    #[cfg(all(target_os = "linux", feature = "rocm"))]
    {
        gpu.model()
    }
    #[cfg(not(all(target_os = "linux", feature = "rocm")))]
    {
        match *gpu {}
    }
}

/// Raw margins (`margin`) or values of `data` from `iterations`.
pub(crate) fn predict(
    gpu: &Model,
    data: &hessboost::data::DMatrix,
    iterations: Iterations,
    margin: bool,
) -> Result<Predictions> {
    #[cfg(all(target_os = "linux", feature = "rocm"))]
    {
        if margin { gpu.predict_margin(data, iterations) } else { gpu.predict(data, iterations) }
    }
    #[cfg(not(all(target_os = "linux", feature = "rocm")))]
    {
        let _ = (data, iterations, margin);
        match *gpu {}
    }
}
