//! Selecting the backend: the `device = rocm` spellings, the availability
//! check and the histogram backend of a training run.
//!
//! This file is `src/backend/rocm_device.rs` of hessboost's crate, declared
//! in `src/backend/mod.rs` on every platform (`pub(crate) mod rocm_device;`)
//! so that `device = rocm` parses everywhere and is refused by validation
//! where the backend is not compiled in, as `cuda` is.
//!
//! hessboost's `Device` enum (src/config/params.rs:170-197) gains the
//! variant `Rocm { ordinal: usize }`, serialized as `rocm` (ordinal 0) or
//! `rocm:<ordinal>`. Its arms call into this module:
//!
//! - `Device::SPELLINGS` (params.rs:202-210) appends [`SPELLINGS`];
//! - `Device::parse` (params.rs:212-229) tries [`parse`] before the CUDA
//!   prefixes: `if let Some(ordinal) = rocm::device::parse(value) { return
//!   Some(Device::Rocm { ordinal }) }`;
//! - `Device::is_compiled_in` (params.rs:231-240) answers [`COMPILED_IN`]
//!   for `Rocm`, and `TrainingParams::validate` calls [`validate`];
//! - `hist_backend` (src/training/prepare.rs:356-416) gains the arm
//!   `Device::Rocm { ordinal } => rocm_device::hist_backend(params, index, ordinal)`;
//! - `TrainingParams` (src/config/params.rs) gains `rocm_sums: RocmSums`
//!   (`"fixed_point"`, the default, or `"exact"`; parsed with
//!   [`rocm::RocmSums::parse`] beside the other string parameters).
//!
//! Device-resident rounds (`Prepared::device_backend`, prepare.rs:94-103,
//! and `device_round`, src/training/round.rs:105-148) drive the same
//! `RowEngine` calls. With `rocm_sums = fixed_point` they stay on the device
//! past the exact domain (the 10.5M-row logistic workload leaves it from its
//! second round); with `exact` the library refuses there and those rounds
//! run on the host.

use crate::config::TrainingParams;
use crate::data::ghist::GHistIndex;
use crate::error::{HessboostError, Result};
use crate::tree::hist::HistogramBackend;

#[cfg(all(target_os = "linux", feature = "rocm"))]
use crate::backend::rocm;

/// The spellings `Device::parse` accepts for this backend, for its error
/// messages.
pub const SPELLINGS: &[&str] = &["rocm", "rocm:<ordinal>"];

/// Whether this build carries the backend (Linux with the `rocm` feature).
pub const COMPILED_IN: bool = cfg!(all(target_os = "linux", feature = "rocm"));

/// The ordinal of `rocm` (0) or `rocm:<ordinal>` (digits only, as for
/// `cuda:<ordinal>`: `usize::from_str` would also take a leading `+`), or
/// `None` for any other value.
pub fn parse(value: &str) -> Option<usize> {
    if value == "rocm" {
        return Some(0);
    }
    let digits = value.strip_prefix("rocm:")?;
    if digits.is_empty() || !digits.bytes().all(|b| b.is_ascii_digit()) {
        return None;
    }
    digits.parse().ok()
}

/// The serialized spelling of `Device::Rocm { ordinal }`.
pub fn spelling(ordinal: usize) -> String {
    if ordinal == 0 { "rocm".to_owned() } else { format!("rocm:{ordinal}") }
}

/// The parameter validation's check of `device = rocm:<ordinal>` (the tree
/// method, `hist`/`auto`, is checked by the caller as for every GPU device):
/// the device exists.
#[cfg(all(target_os = "linux", feature = "rocm"))]
pub fn validate(ordinal: usize) -> Result<()> {
    if !rocm::available(ordinal) {
        return Err(HessboostError::invalid_param(
            "device",
            format!("no ROCm device {ordinal} ({} visible)", rocm::device_count()),
        ));
    }
    Ok(())
}

/// The same where the backend is not compiled in: always refused.
#[cfg(not(all(target_os = "linux", feature = "rocm")))]
pub fn validate(_ordinal: usize) -> Result<()> {
    Err(HessboostError::invalid_param(
        "device",
        "`rocm` requires building with the `rocm` feature on Linux",
    ))
}

/// The `Device::Rocm { ordinal }` arm of `hist_backend`: the backend in the
/// run's summing mode, its guard checking the run's `gamma`.
#[cfg(all(target_os = "linux", feature = "rocm"))]
pub fn hist_backend(params: &TrainingParams, index: &GHistIndex, ordinal: usize) -> Result<Box<dyn HistogramBackend>> {
    let backend = rocm::RocmHistBackend::new(index, ordinal)?.with_sums(params.rocm_sums, params.gamma)?;
    let backend: Box<dyn HistogramBackend> = Box::new(backend);
    Ok(backend)
}

/// Unreachable in practice where the backend is not compiled in:
/// validation refuses `device = rocm` first, as for `cuda`.
#[cfg(not(all(target_os = "linux", feature = "rocm")))]
pub fn hist_backend(_params: &TrainingParams, _index: &GHistIndex, _ordinal: usize) -> Result<Box<dyn HistogramBackend>> {
    validate(0).map(|()| unreachable!())
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn parses_the_rocm_spellings_only() {
        assert_eq!(parse("rocm"), Some(0));
        assert_eq!(parse("rocm:0"), Some(0));
        assert_eq!(parse("rocm:3"), Some(3));
        for bad in ["rocm:", "rocm:+1", "rocm:-1", "rocm:1a", "ROCM", "rocm 1", "cuda:0", "gpu"] {
            assert_eq!(parse(bad), None, "{bad}");
        }
        assert_eq!(spelling(0), "rocm");
        assert_eq!(spelling(2), "rocm:2");
        assert_eq!(parse(&spelling(7)), Some(7));
    }
}
