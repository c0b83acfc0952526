//! Status + payload of every call, in the shapes of the reference's error
//! enums (LengthMismatch { argument, expected, actual }, NonFiniteInput
//! { index, value }, Int4OutOfRange(u8), InvalidRowCount(usize), DeviceError).
use core::ffi::{c_char, CStr};
use std::fmt;

use nemotron_hip_sys::{nh_error, nh_status};

#[derive(Clone, Debug, PartialEq)]
pub enum HipError {
    /// `*Error::InvalidShape` (the detail names the shape).
    InvalidShape(String),
    LengthMismatch { argument: &'static str, expected: usize, actual: usize },
    /// `QuantizeError::InvalidParams`
    InvalidParams(String),
    /// `QuantizeError::NonFiniteInput`; `argument` is "input", or for a layer's
    /// f32 intermediate "intermediate" (the MoE shared expert's:
    /// "shared_intermediate").
    NonFiniteInput { argument: &'static str, index: usize, value: f32 },
    Int4OutOfRange(u8),
    InvalidRowCount(usize),
    /// Outside the device envelope: the caller runs the host path instead.
    Unsupported(String),
    DeviceError(String),
    Io(String),
    InvalidHeader(String),
    TensorNotFound(String),
}

/// The library's argument names are static C strings.
fn static_str(p: *const c_char) -> &'static str {
    if p.is_null() {
        return "";
    }
    // SAFETY: nh_error.argument points at a string literal of the library.
    unsafe { CStr::from_ptr(p) }.to_str().unwrap_or("")
}

fn message(err: &nh_error) -> String {
    // SAFETY: the library always NUL-terminates message (a zeroed nh_error is empty).
    unsafe { CStr::from_ptr(err.message.as_ptr()) }.to_string_lossy().into_owned()
}

/// `Ok(())` for NH_OK, else the error the status and payload describe.
pub fn check(status: nh_status, err: &nh_error) -> Result<(), HipError> {
    let msg = || message(err);
    Err(match status {
        nh_status::OK => return Ok(()),
        nh_status::INVALID_SHAPE => HipError::InvalidShape(msg()),
        nh_status::LENGTH_MISMATCH => HipError::LengthMismatch {
            argument: static_str(err.argument),
            expected: err.expected as usize,
            actual: err.actual as usize,
        },
        nh_status::INVALID_PARAMS => HipError::InvalidParams(msg()),
        nh_status::NON_FINITE_INPUT => HipError::NonFiniteInput {
            argument: static_str(err.argument),
            index: err.index as usize,
            value: err.value,
        },
        nh_status::OUT_OF_RANGE => HipError::Int4OutOfRange(err.byte as u8),
        nh_status::INVALID_ROW_COUNT => HipError::InvalidRowCount(err.actual as usize),
        nh_status::UNSUPPORTED => HipError::Unsupported(msg()),
        nh_status::IO_ERROR => HipError::Io(msg()),
        nh_status::INVALID_HEADER => HipError::InvalidHeader(msg()),
        nh_status::TENSOR_NOT_FOUND => HipError::TensorNotFound(msg()),
        _ => HipError::DeviceError(msg()),
    })
}

/// Runs one library call with a fresh error payload and maps its status.
pub(crate) fn call(f: impl FnOnce(*mut nh_error) -> nh_status) -> Result<(), HipError> {
    let mut err = nh_error::default();
    let st = f(&mut err);
    check(st, &err)
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            Self::InvalidShape(m) => write!(f, "invalid shape: {m}"),
            Self::LengthMismatch { argument, expected, actual } => {
                write!(f, "{argument} length mismatch: expected {expected}, got {actual}")
            }
            Self::InvalidParams(m) => write!(f, "invalid quantization parameters: {m}"),
            Self::NonFiniteInput { argument, index, value } => {
                write!(f, "non-finite {argument} value {value} at index {index}")
            }
            Self::Int4OutOfRange(b) => write!(f, "int4 value {b} out of range"),
            Self::InvalidRowCount(r) => write!(f, "row_count must be non-zero, got {r}"),
            Self::Unsupported(m) => write!(f, "outside the device envelope: {m}"),
            Self::DeviceError(m) => write!(f, "device error: {m}"),
            Self::Io(m) => write!(f, "io error: {m}"),
            Self::InvalidHeader(m) => write!(f, "invalid safetensors header: {m}"),
            Self::TensorNotFound(m) => write!(f, "{m}"),
        }
    }
}

impl std::error::Error for HipError {}
