//! `GpuContext` on the MI355X build (replaces src/io/device.rs:22-272).
//!
//! The reference's context owns a cudarc context, a stream, a PTX module and
//! the 34 kernel handles it launches by name with positional arguments.  Here
//! it owns one `skl_ctx` of the C ABI (include/soklyn_hip.h): the library
//! resolves and launches its own gfx950 kernels, and each crate-internal
//! method (ffn_device.rs, util_device.rs) is one C call.  `new` /
//! `with_device_index` / `download` keep their public signatures.
mod ffn_device;
pub(crate) mod hip_ffi;
mod util_device;

use std::ffi::CStr;

use hip_ffi::*;

use crate::util::device_buffer::DeviceBuffer;
use crate::util::log::Error;
use crate::util::r#type::Precision;

/// Carries the connection to one GPU: the C ABI's context.
pub struct GpuContext {
    ctx: *mut SklCtx,
    tile_dim: u32,
}

// The context serialises its calls on one stream (every call synchronises by
// default, as the reference does after each launch).
unsafe impl Send for GpuContext {}
unsafe impl Sync for GpuContext {}

/// A C-ABI status as the crate's `Error` (one variant per negative code; a
/// positive code is a HIP runtime error, the variant that takes the place of
/// `DriverError(#[from] DriverError)`, log.rs:23-24).
pub(crate) fn check(status: i32) -> Result<(), Error> {
    const FROM_DEVICE: &str = "rejected by the device layer";
    match status {
        SKL_OK => Ok(()),
        s if s > 0 => Err(Error::HipError {
            code: s,
            message: unsafe { CStr::from_ptr(skl_status_string(s)) }.to_string_lossy().into_owned(),
        }),
        SKL_ERR_INVALID_CONFIGURATION => Err(Error::InvalidConfiguration { reason: FROM_DEVICE.to_string() }),
        SKL_ERR_TRAINING_MODE_REQUIRED => Err(Error::TrainingModeRequired { reason: FROM_DEVICE }),
        SKL_ERR_ALLOCATION_LIMIT => {
            Err(Error::AllocationLimitExceeded { received: 0, max: 0, reason: FROM_DEVICE })
        }
        SKL_ERR_MISMATCHED_DIMENSIONS => {
            Err(Error::MismatchedDimensions { reason: FROM_DEVICE, expected: 0, found: 0 })
        }
        SKL_ERR_INVALID_BATCH_SIZE => Err(Error::InvalidBatchSize { reason: FROM_DEVICE }),
        SKL_ERR_HARDWARE_CONSTRAINT => {
            Err(Error::HardwareConstraintViolation { precision: Precision::FP16, expected: 16, found: 0 })
        }
        SKL_ERR_UNSUPPORTED_CAST => Err(Error::UnsupportedTypeCast { from: Precision::FP32, to: Precision::FP32 }),
        s => Err(Error::HipError {
            code: s,
            message: unsafe { CStr::from_ptr(skl_status_string(s)) }.to_string_lossy().into_owned(),
        }),
    }
}

impl GpuContext {
    /// device.rs:164-167: the first GPU.
    pub fn new(tile_dim: u32) -> Self {
        Self::with_device_index(0, tile_dim)
    }

    /// device.rs:180-183.  Context creation failures panic, as in the reference.
    pub fn with_device_index(ordinal: usize, tile_dim: u32) -> Self {
        let mut ctx: *mut SklCtx = std::ptr::null_mut();
        let ordinal = i32::try_from(ordinal).expect("device ordinal");
        check(unsafe { skl_ctx_create(ordinal, tile_dim, &mut ctx) })
            .unwrap_or_else(|e| panic!("cannot create the MI355X context on device {ordinal}: {e}"));
        Self { ctx, tile_dim }
    }

    /// device.rs:203-209.
    pub fn download<K: Copy>(&self, buffer: &DeviceBuffer<K>) -> Result<Vec<K>, Error> {
        buffer.to_host(self)
    }

    pub(crate) fn get_tile_dim(&self) -> u32 {
        self.tile_dim
    }

    pub(crate) fn raw(&self) -> *mut SklCtx {
        self.ctx
    }
}

impl Drop for GpuContext {
    fn drop(&mut self) {
        unsafe {
            skl_ctx_destroy(self.ctx);
        }
    }
}
