//! Device memory owned by a `Tensor` on the MI355X build: the reference keeps a
//! cudarc `CudaSlice<T>` in `Tensor::data` (core.rs:414-693); here it is a
//! `DeviceBuffer<T>` allocated and freed through the C ABI (skl_malloc /
//! skl_free), so no CUDA or HIP runtime type appears in the crate.  `Tensor`'s
//! `get_data()` returns `&DeviceBuffer<T>`; the rest of core.rs keeps its
//! shapes, ids (TENSOR_ID_COUNTER, core.rs:84-88) and methods, with the copies
//! of from_cpu_vector / download / clone going through skl_memcpy_*.
use std::marker::PhantomData;
use std::os::raw::c_void;

use crate::io::device::hip_ffi::*;
use crate::io::device::{check, GpuContext};
use crate::log::Error;

pub struct DeviceBuffer<T> {
    ptr: *mut c_void,
    len: usize,
    ctx: *mut SklCtx,
    _elem: PhantomData<T>,
}

impl<T: Copy> DeviceBuffer<T> {
    /// `len` elements, uninitialised.
    pub(crate) fn alloc(context: &GpuContext, len: usize) -> Result<Self, Error> {
        let mut ptr: *mut c_void = std::ptr::null_mut();
        check(unsafe { skl_malloc(context.raw(), &mut ptr, len * std::mem::size_of::<T>()) })?;
        Ok(Self { ptr, len, ctx: context.raw(), _elem: PhantomData })
    }

    pub(crate) fn from_host(context: &GpuContext, host: &[T]) -> Result<Self, Error> {
        let buf = Self::alloc(context, host.len())?;
        check(unsafe {
            skl_memcpy_h2d(context.raw(), buf.ptr, host.as_ptr() as *const c_void, std::mem::size_of_val(host))
        })?;
        Ok(buf)
    }

    pub(crate) fn to_host(&self, context: &GpuContext) -> Result<Vec<T>, Error> {
        let mut host = Vec::with_capacity(self.len);
        check(unsafe {
            skl_memcpy_d2h(context.raw(), host.as_mut_ptr() as *mut c_void, self.ptr,
                           self.len * std::mem::size_of::<T>())
        })?;
        unsafe { host.set_len(self.len) };
        Ok(host)
    }

    pub(crate) fn clone_on(&self, context: &GpuContext) -> Result<Self, Error> {
        let buf = Self::alloc(context, self.len)?;
        check(unsafe { skl_memcpy_d2d(context.raw(), buf.ptr, self.ptr, self.len * std::mem::size_of::<T>()) })?;
        Ok(buf)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    /// The device address, for a descriptor field or a C-ABI argument.
    pub(crate) fn as_ptr(&self) -> *mut c_void {
        self.ptr
    }
}

impl<T> Drop for DeviceBuffer<T> {
    fn drop(&mut self) {
        // skl_free synchronises the context's stream before it frees
        unsafe {
            skl_free(self.ctx, self.ptr);
        }
    }
}
