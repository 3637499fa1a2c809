//! Status codes of the C ABI back into `OrcaError` (orca-core/src/error.rs:5-31), all five
//! variants with their fields (orca_hip_last_error_info).
use std::collections::HashMap;
use std::ffi::CStr;
use std::os::raw::{c_char, c_int};
use std::sync::{Mutex, OnceLock};

use orca_core::{DType, Device, OrcaError, Result};

use crate::ffi;

/// DType in orca_core's order (orca-core/src/dtype.rs:5-22), as the ABI numbers it.
pub fn dtype_code(d: DType) -> c_int {
    match d {
        DType::F32 => 0,
        DType::F64 => 1,
        DType::F16 => 2,
        DType::BF16 => 3,
        DType::I32 => 4,
        DType::I64 => 5,
        DType::U8 => 6,
        DType::Bool => 7,
    }
}

fn dtype_of(code: c_int) -> DType {
    match code {
        1 => DType::F64,
        2 => DType::F16,
        3 => DType::BF16,
        4 => DType::I32,
        5 => DType::I64,
        6 => DType::U8,
        7 => DType::Bool,
        _ => DType::F32,
    }
}

fn device_of(kind: c_int, index: c_int) -> Device {
    let i = index.max(0) as usize;
    match kind {
        0 => Device::Cpu,
        1 => Device::Cuda(i),
        _ => Device::Gpu(i),
    }
}

fn text(p: *const c_char) -> String {
    if p.is_null() {
        String::new()
    } else {
        unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
    }
}

/// OrcaError's `op` is a `&'static str`: each distinct operation name is kept once.
fn intern(op: String) -> &'static str {
    static NAMES: OnceLock<Mutex<HashMap<String, &'static str>>> = OnceLock::new();
    let mut names = NAMES.get_or_init(|| Mutex::new(HashMap::new())).lock().unwrap_or_else(|e| e.into_inner());
    if let Some(s) = names.get(&op) {
        return s;
    }
    let s: &'static str = Box::leak(op.clone().into_boxed_str());
    names.insert(op, s);
    s
}

/// Ok(()) for ORCA_HIP_OK, else the calling thread's last failure as its OrcaError variant.
pub fn check(rc: c_int) -> Result<()> {
    if rc == ffi::ORCA_HIP_OK {
        return Ok(());
    }
    let mut info = ffi::ErrorInfo {
        code: rc,
        op: std::ptr::null(),
        expected: std::ptr::null(),
        got: std::ptr::null(),
        dtype: -1,
        dtype_got: -1,
        device_kind: [-1, -1],
        device_index: [-1, -1],
        message: std::ptr::null(),
    };
    if unsafe { ffi::orca_hip_last_error_info(&mut info) } != ffi::ORCA_HIP_OK {
        return Err(OrcaError::InternalError(text(unsafe { ffi::orca_hip_last_error() })));
    }
    let op = intern(text(info.op));
    Err(match rc {
        ffi::ORCA_HIP_ERR_SHAPE => OrcaError::ShapeMismatch { op, expected: text(info.expected), got: text(info.got) },
        ffi::ORCA_HIP_ERR_UNSUPPORTED_DTYPE => OrcaError::UnsupportedDType { op, dtype: dtype_of(info.dtype) },
        ffi::ORCA_HIP_ERR_DTYPE_MISMATCH => OrcaError::DTypeMismatch {
            op,
            expected: dtype_of(info.dtype),
            got: dtype_of(info.dtype_got),
        },
        ffi::ORCA_HIP_ERR_DEVICE_MISMATCH => OrcaError::DeviceMismatch(
            device_of(info.device_kind[0], info.device_index[0]),
            device_of(info.device_kind[1], info.device_index[1]),
        ),
        _ => OrcaError::InternalError(text(info.message)),
    })
}
