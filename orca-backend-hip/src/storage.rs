//! `HipStorage`: the trait's storage (orca-tensor/src/backend.rs:7-15) as one reference to a
//! storage handle of the library.  Clones share it (an `Arc`), the last drop releases it: the
//! library then frees the device memory stream-ordered, and decides which pending values are
//! still held from these references, so a storage must not outlive its last Rust holder.
use std::fmt;
use std::sync::Arc;

use orca_tensor::Storage;

use crate::ffi;

struct Handle(*mut ffi::OrcaHipStorage);

// The library's handles are reference counted atomically and used under its own lock.
unsafe impl Send for Handle {}
unsafe impl Sync for Handle {}

impl Drop for Handle {
    fn drop(&mut self) {
        unsafe {
            ffi::orca_hip_storage_release(self.0);
        }
    }
}

#[derive(Clone)]
pub struct HipStorage {
    handle: Arc<Handle>,
    len: usize,
}

impl HipStorage {
    /// Takes over one reference returned by the library (null only on failure, never adopted).
    pub(crate) fn adopt(raw: *mut ffi::OrcaHipStorage) -> Self {
        let mut len = 0usize;
        unsafe {
            ffi::orca_hip_storage_len(raw, &mut len);
        }
        HipStorage { handle: Arc::new(Handle(raw)), len }
    }

    pub(crate) fn raw(&self) -> *mut ffi::OrcaHipStorage {
        self.handle.0
    }

    pub(crate) fn len_elements(&self) -> usize {
        self.len
    }
}

impl fmt::Debug for HipStorage {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "HipStorage({} elements)", self.len)
    }
}

impl Storage for HipStorage {
    fn len(&self) -> usize {
        self.len
    }
}
