//! One GPU's context, owned device buffers and streams (the roles of
//! GpuDevice and GpuTensor, device.rs:117-153, tensor.rs:259-446).
use core::ffi::c_void;
use core::marker::PhantomData;
use std::ffi::CString;
use std::sync::Arc;

use nemotron_hip_sys as sys;

use crate::error::{call, HipError};

/// A device and the loaded gfx950 code object.  Immutable once created; the
/// library allows sharing it across threads.
pub struct Context {
    raw: *mut sys::nh_context,
}

// SAFETY: the C context is immutable after nh_context_create and every entry
// point binds its device per call (the header's contract).
unsafe impl Send for Context {}
unsafe impl Sync for Context {}

impl Context {
    /// Device `device` with the code object embedded in the library.
    pub fn new(device: i32) -> Result<Arc<Self>, HipError> {
        Self::with_code_object(device, None)
    }

    /// Device `device` with the code object at `path` (None: the embedded one).
    pub fn with_code_object(device: i32, path: Option<&str>) -> Result<Arc<Self>, HipError> {
        let path_c = match path {
            Some(p) => Some(CString::new(p).map_err(|_| HipError::Io("path holds a NUL byte".into()))?),
            None => None,
        };
        let mut raw = core::ptr::null_mut();
        call(|e| unsafe {
            sys::nh_context_create(device, path_c.as_ref().map_or(core::ptr::null(), |c| c.as_ptr()), &mut raw, e)
        })?;
        Ok(Arc::new(Self { raw }))
    }

    pub fn device_count() -> i32 {
        unsafe { sys::nh_device_count() }
    }

    pub fn as_raw(&self) -> *mut sys::nh_context {
        self.raw
    }

    pub fn device(&self) -> i32 {
        unsafe { sys::nh_context_device(self.raw) }
    }

    /// Waits for all work on `stream` (None: the null stream).
    pub fn synchronize(&self, stream: Option<&Stream>) -> Result<(), HipError> {
        call(|e| unsafe { sys::nh_stream_synchronize(self.raw, Stream::raw_or_null(stream), e) })
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe { sys::nh_context_destroy(self.raw) }
    }
}

/// A HIP stream of one context (default priority).
pub struct Stream {
    ctx: Arc<Context>,
    raw: sys::nh_stream,
}

unsafe impl Send for Stream {}

impl Stream {
    pub fn new(ctx: &Arc<Context>) -> Result<Self, HipError> {
        let mut raw = core::ptr::null_mut();
        call(|e| unsafe { sys::nh_stream_create(ctx.raw, &mut raw, e) })?;
        Ok(Self { ctx: ctx.clone(), raw })
    }

    pub fn as_raw(&self) -> sys::nh_stream {
        self.raw
    }

    pub(crate) fn raw_or_null(s: Option<&Stream>) -> sys::nh_stream {
        s.map_or(core::ptr::null_mut(), |s| s.raw)
    }
}

impl Drop for Stream {
    fn drop(&mut self) {
        let _ = call(|e| unsafe { sys::nh_stream_destroy(self.ctx.raw, self.raw, e) });
    }
}

/// `len` elements of `T` in device memory, freed on drop.
pub struct DeviceBuffer<T: Copy> {
    ctx: Arc<Context>,
    ptr: *mut c_void,
    len: usize,
    _t: PhantomData<T>,
}

// SAFETY: a device allocation is not tied to a host thread.
unsafe impl<T: Copy + Send> Send for DeviceBuffer<T> {}
unsafe impl<T: Copy + Sync> Sync for DeviceBuffer<T> {}

impl<T: Copy> DeviceBuffer<T> {
    /// Uninitialised device memory for `len` elements (at least one byte is
    /// allocated, so the pointer is always a valid device address).
    pub fn new(ctx: &Arc<Context>, len: usize) -> Result<Self, HipError> {
        let bytes = len
            .checked_mul(core::mem::size_of::<T>())
            .ok_or_else(|| HipError::InvalidShape(format!("{len} elements overflow")))?;
        let mut ptr = core::ptr::null_mut();
        call(|e| unsafe { sys::nh_malloc(ctx.raw, bytes.max(1), &mut ptr, e) })?;
        Ok(Self { ctx: ctx.clone(), ptr, len, _t: PhantomData })
    }

    /// A device copy of `host` (synchronous).
    pub fn from_host(ctx: &Arc<Context>, host: &[T]) -> Result<Self, HipError> {
        let b = Self::new(ctx, host.len())?;
        b.copy_from_host(host)?;
        Ok(b)
    }

    /// Zero-filled device memory (synchronous).
    pub fn zeroed(ctx: &Arc<Context>, len: usize) -> Result<Self, HipError> {
        let b = Self::new(ctx, len)?;
        call(|e| unsafe { sys::nh_memset_d8(ctx.raw, b.ptr, 0, b.bytes(), e) })?;
        Ok(b)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub fn bytes(&self) -> usize {
        self.len * core::mem::size_of::<T>()
    }

    pub fn as_ptr(&self) -> *const T {
        self.ptr as *const T
    }

    pub fn as_mut_ptr(&mut self) -> *mut T {
        self.ptr as *mut T
    }

    pub fn context(&self) -> &Arc<Context> {
        &self.ctx
    }

    pub fn copy_from_host(&self, host: &[T]) -> Result<(), HipError> {
        if host.len() != self.len {
            return Err(HipError::LengthMismatch { argument: "host", expected: self.len, actual: host.len() });
        }
        call(|e| unsafe { sys::nh_memcpy_htod(self.ctx.raw, self.ptr, host.as_ptr().cast(), self.bytes(), e) })
    }

    pub fn copy_to_host(&self, host: &mut [T]) -> Result<(), HipError> {
        if host.len() != self.len {
            return Err(HipError::LengthMismatch { argument: "host", expected: self.len, actual: host.len() });
        }
        call(|e| unsafe { sys::nh_memcpy_dtoh(self.ctx.raw, host.as_mut_ptr().cast(), self.ptr, self.bytes(), e) })
    }
}

impl<T: Copy> Drop for DeviceBuffer<T> {
    fn drop(&mut self) {
        let _ = call(|e| unsafe { sys::nh_free(self.ctx.raw, self.ptr, e) });
    }
}
