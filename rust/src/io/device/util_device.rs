//! The utility methods of `GpuContext` on the MI355X build (replaces
//! src/io/device/util_device.rs:7-78).  `gpu_matrix_mul` / `gpu_matrix_add`
//! (util_device.rs:81-140) drive the gemm / geam kernels that no DenseBlock
//! path calls; they are not part of this build.
use std::os::raw::c_void;

use super::hip_ffi::*;
use super::{check, GpuContext};
use crate::log::Error;
use crate::util::device_buffer::DeviceBuffer;
use crate::{Precision, PrecisionType};

fn dtype<T: PrecisionType>() -> u32 {
    if T::precision() == Precision::FP16 { SKL_F16 } else { SKL_F32 }
}

impl GpuContext {
    /// util_device.rs:7-47: f32 -> f16 (round to nearest even) or f16 -> f32 into a
    /// new buffer; any other pairing is UnsupportedTypeCast, as in the reference.
    pub(crate) fn gpu_cast_t<T: PrecisionType, U: PrecisionType>(
        &self,
        data: &DeviceBuffer<T>,
    ) -> Result<DeviceBuffer<U>, Error> {
        let out = DeviceBuffer::<U>::alloc(self, data.len())?;
        check(unsafe {
            skl_cast(self.raw(), data.as_ptr() as *const c_void, dtype::<T>(), out.as_ptr(), dtype::<U>(), data.len())
        })?;
        Ok(out)
    }

    /// util_device.rs:49-78: every element of `data` set to `value`.
    pub(crate) fn gpu_broadcast<T: PrecisionType>(&self, data: &DeviceBuffer<T>, value: f32) -> Result<(), Error> {
        check(unsafe { skl_fill(self.raw(), data.as_ptr(), dtype::<T>(), value, data.len()) })
    }
}
