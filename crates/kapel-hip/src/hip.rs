//! The few functions of the HIP runtime (libamdhip64) the backend calls:
//! device selection, memory, copies and one stream. Default stream
//! priority only.

use core::ffi::{c_char, c_int, c_void};

pub type HipError = c_int;
pub const HIP_SUCCESS: HipError = 0;

/// `hipMemcpyKind`.
pub const HOST_TO_DEVICE: c_int = 1;
pub const DEVICE_TO_HOST: c_int = 2;
pub const DEVICE_TO_DEVICE: c_int = 3;

#[cfg(feature = "hip")]
#[link(name = "amdhip64")]
unsafe extern "C" {
    pub fn hipSetDevice(device: c_int) -> HipError;
    pub fn hipGetDeviceCount(count: *mut c_int) -> HipError;
    pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> HipError;
    pub fn hipFree(ptr: *mut c_void) -> HipError;
    pub fn hipMemset(dst: *mut c_void, value: c_int, size: usize) -> HipError;
    pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> HipError;
    pub fn hipMemcpyAsync(
        dst: *mut c_void,
        src: *const c_void,
        size: usize,
        kind: c_int,
        stream: *mut c_void,
    ) -> HipError;
    pub fn hipStreamCreate(stream: *mut *mut c_void) -> HipError;
    pub fn hipStreamDestroy(stream: *mut c_void) -> HipError;
    pub fn hipStreamSynchronize(stream: *mut c_void) -> HipError;
    pub fn hipGetErrorString(error: HipError) -> *const c_char;
}
