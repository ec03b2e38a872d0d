//! The C ABI of libkapel_hip (`include/kapel_hip.h`), declared for Rust.
//!
//! Every declaration mirrors one of the header, in the header's order, with
//! the same names, argument order and widths (`uint32_t` → `u32`, `uint64_t` →
//! `u64`, `int` → `c_int`, pointers to device memory as raw pointers, the
//! stream as `*mut c_void`). The test `tests/test_rust_abi.py` of the
//! kapel-hip checkout compares this file with the header.

use core::ffi::{c_char, c_int, c_void};

// Formats: the codes of kapel-cuda-abi (crates/kapel-cuda-abi/src/lib.rs:152-194),
// with Q2_K and Q3_K added.
pub const KH_INT8: u32 = 0;
pub const KH_INT4: u32 = 1;
pub const KH_Q8_0: u32 = 2;
pub const KH_Q4_0: u32 = 3;
pub const KH_Q4_1: u32 = 4;
pub const KH_Q5_0: u32 = 5;
pub const KH_Q5_1: u32 = 6;
pub const KH_Q4K: u32 = 7;
pub const KH_Q5K: u32 = 8;
pub const KH_Q6K: u32 = 9;
pub const KH_IQ4_NL: u32 = 10;
pub const KH_IQ4_XS: u32 = 11;
pub const KH_IQ3_S: u32 = 12;
pub const KH_Q2K: u32 = 13;
pub const KH_Q3K: u32 = 14;

// Activation and output types.
pub const KH_F32: u32 = 0;
pub const KH_BF16: u32 = 1;
pub const KH_F16: u32 = 2;

// Status codes.
pub const KH_OK: c_int = 0;
pub const KH_ERR_ARITY: c_int = 1;
pub const KH_ERR_DTYPE: c_int = 2;
pub const KH_ERR_SHAPE: c_int = 3;
pub const KH_ERR_MISALIGNED: c_int = 4;
pub const KH_ERR_OVERFLOW: c_int = 5;
pub const KH_ERR_WORKSPACE: c_int = 6;
pub const KH_ERR_HIP: c_int = 7;
pub const KH_ERR_NULL: c_int = 8;

// Flags of the products.
pub const KH_BYTE_ACTIVATIONS: u32 = 1;
pub const KH_REUSE_ACTIVATIONS: u32 = 2;
pub const KH_BYTE_ACTIVATIONS_ALL_ROWS: u32 = 4;

/// Workspace bytes of the device array `kh_qmatmul_static` uses.
pub const KH_STATIC_SCRATCH_BYTES: u64 = 32 << 20;

/// One weight matrix on the device: `n` rows of whole blocks of `format`.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct KhWeight {
    pub format: u32,
    pub group: u32,
    pub data: *const c_void,
    pub bytes: u64,
    pub n: u64,
}

#[cfg(feature = "hip")]
#[link(name = "kapel_hip")]
unsafe extern "C" {
    pub fn kh_version() -> *const c_char;
    pub fn kh_error_string(status: c_int) -> *const c_char;

    pub fn kh_block_len(format: u32, group: u32) -> u32;
    pub fn kh_block_bytes(format: u32, group: u32) -> u32;

    pub fn kh_qmatmul_workspace(weights: *const KhWeight, count: u32, k: u64, rows: u64, flags: u32) -> u64;
    pub fn kh_qmatmul(
        weights: *const KhWeight,
        count: u32,
        k: u64,
        x_kind: u32,
        x: *const c_void,
        rows: u64,
        out_kind: u32,
        out: *mut c_void,
        flags: u32,
        workspace: *mut c_void,
        workspace_bytes: u64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn kh_qmatmul_static(
        weights: *const KhWeight,
        count: u32,
        k: u64,
        x_kind: u32,
        x: *const c_void,
        rows: u64,
        out_kind: u32,
        out: *mut c_void,
        flags: u32,
        stream: *mut c_void,
    ) -> c_int;

    pub fn kh_quantize_x(
        x_kind: u32,
        x: *const c_void,
        rows: u64,
        k: u64,
        q: *mut i8,
        scale: *mut f32,
        sums32: *mut f32,
        stream: *mut c_void,
    ) -> c_int;
    pub fn kh_block_dots(
        weight: *const KhWeight,
        k: u64,
        q: *const i8,
        rows: u64,
        dots: *mut i32,
        workspace: *mut c_void,
        workspace_bytes: u64,
        stream: *mut c_void,
    ) -> c_int;
    pub fn kh_dequantize(
        weight: *const KhWeight,
        k: u64,
        first: u64,
        count: u64,
        out_kind: u32,
        out: *mut c_void,
        stream: *mut c_void,
    ) -> c_int;
    pub fn kh_dequantize_rows(
        weight: *const KhWeight,
        k: u64,
        indices: *const u32,
        count: u64,
        out_kind: u32,
        out: *mut c_void,
        stream: *mut c_void,
    ) -> c_int;

    pub fn kh_expert_matmul_workspace(
        weight: *const KhWeight,
        experts: u32,
        k: u64,
        tokens: u64,
        topk: u32,
        per_route: u32,
        x_kind: u32,
        flags: u32,
    ) -> u64;
    pub fn kh_expert_matmul(
        weight: *const KhWeight,
        experts: u32,
        k: u64,
        x_kind: u32,
        x: *const c_void,
        tokens: u64,
        topk: u32,
        per_route: u32,
        idx: *const u32,
        out_kind: u32,
        out: *mut c_void,
        flags: u32,
        workspace: *mut c_void,
        workspace_bytes: u64,
        stream: *mut c_void,
    ) -> c_int;

    pub fn kh_quantize_host(
        format: u32,
        group: u32,
        values: *const f32,
        count: u64,
        out: *mut u8,
        threads: c_int,
    ) -> i64;
}
