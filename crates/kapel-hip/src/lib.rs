//! The HIP backend: Kapel on AMD Instinct MI355X (gfx950).
//!
//! The products by quantized weights (`QuantizedMatmul`, `ExpertMatmul`) run
//! in libkapel_hip, through its C ABI ([`abi`]), on the backend's stream; every
//! other operation runs on the host with `kapel_cpu::Cpu` (its inputs
//! downloaded, its outputs uploaded), as kapel-cuda does for the formats it
//! has no kernels for (crates/kapel-cuda/src/ops.rs:1293-1326). So the whole
//! catalogue is there (`Backend`), and the hot path of generation is on the
//! device.
//!
//! Shaped as `kapel_cuda::Cuda` (crates/kapel-cuda/src/device.rs:185-240): one
//! backend per device ordinal, one stream, a workspace kept between calls and
//! grown when a call needs more. Tensors on the device hold a [`HipStorage`].
//!
//! Without the `hip` feature only [`abi`] and the code tables are compiled.

pub mod abi;
mod hip;

#[cfg(feature = "hip")]
mod backend;
#[cfg(feature = "hip")]
pub use backend::{Hip, HipStorage};

use kapel_core::{DType, QuantFormat};

/// The library's code and group of a quantized format; `None` for a format
/// the library does not read (it then runs on the host).
pub fn format_code(dtype: DType) -> Option<(u32, u32)> {
    let DType::Quantized(format) = dtype else {
        return None;
    };
    Some(match format {
        QuantFormat::Int8 { group } => (abi::KH_INT8, u32::from(group)),
        QuantFormat::Int4 { group } => (abi::KH_INT4, u32::from(group)),
        QuantFormat::Q8_0 => (abi::KH_Q8_0, 0),
        QuantFormat::Q4_0 => (abi::KH_Q4_0, 0),
        QuantFormat::Q4_1 => (abi::KH_Q4_1, 0),
        QuantFormat::Q5_0 => (abi::KH_Q5_0, 0),
        QuantFormat::Q5_1 => (abi::KH_Q5_1, 0),
        QuantFormat::Q2K => (abi::KH_Q2K, 0),
        QuantFormat::Q3K => (abi::KH_Q3K, 0),
        QuantFormat::Q4K => (abi::KH_Q4K, 0),
        QuantFormat::Q5K => (abi::KH_Q5K, 0),
        QuantFormat::Q6K => (abi::KH_Q6K, 0),
        QuantFormat::Iq4Nl => (abi::KH_IQ4_NL, 0),
        QuantFormat::Iq4Xs => (abi::KH_IQ4_XS, 0),
        QuantFormat::Iq3S => (abi::KH_IQ3_S, 0),
        _ => return None,
    })
}

/// The library's code of an activation or output type: f32, bf16 or f16.
pub fn float_code(dtype: DType) -> Option<u32> {
    match dtype {
        DType::F32 => Some(abi::KH_F32),
        DType::BF16 => Some(abi::KH_BF16),
        DType::F16 => Some(abi::KH_F16),
        _ => None,
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn codes_are_those_of_the_cuda_abi() {
        // crates/kapel-cuda-abi/src/lib.rs:152-194 numbers the formats the
        // same way up to IQ3_S.
        assert_eq!(format_code(DType::Quantized(QuantFormat::Q4K)), Some((7, 0)));
        assert_eq!(format_code(DType::Quantized(QuantFormat::Iq3S)), Some((12, 0)));
        assert_eq!(format_code(DType::Quantized(QuantFormat::Int4 { group: 64 })), Some((1, 64)));
        assert_eq!(format_code(DType::F32), None);
        assert_eq!(float_code(DType::BF16), Some(1));
        assert_eq!(float_code(DType::F64), None);
    }
}
