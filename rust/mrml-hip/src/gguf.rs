//! `GgufFile` (crates/mrml-tensor/src/gguf.rs:71-184) over the library's
//! reader: header, metadata and tensor directory parsed at open, tensor bytes
//! read on demand.

use std::ffi::{c_char, CStr, CString};

use crate::ffi::{self, Gguf};
use crate::{load_error, Error, Result};

/// One tensor of the directory.
#[derive(Clone, Debug)]
pub struct GgufTensor {
    pub name: String,
    pub type_id: i32,
    pub dims: Vec<u64>,
    pub offset: u64,
    pub size_bytes: u64,
}

pub struct GgufFile {
    api: &'static ffi::Api,
    handle: Gguf,
    pub version: u32,
    pub data_offset: u64,
    pub n_tensors: usize,
    pub n_meta: usize,
}

unsafe impl Send for GgufFile {}

impl GgufFile {
    fn error(api: &ffi::Api, status: i32) -> Error {
        let m = unsafe { (api.gguf_last_error)() };
        let message = if m.is_null() { String::new() } else { unsafe { CStr::from_ptr(m) }.to_string_lossy().into_owned() };
        Error { status, message }
    }

    fn check(&self, status: i32) -> Result<()> {
        if status == 0 { Ok(()) } else { Err(Self::error(self.api, status)) }
    }

    /// `GgufFile::open` (gguf.rs:80-171).
    pub fn open(path: &str) -> Result<Self> {
        let api = ffi::api().map_err(load_error)?;
        let c = CString::new(path).map_err(|e| Error { status: ffi::MRML_HIP_E_INVALID, message: e.to_string() })?;
        let mut handle: Gguf = std::ptr::null_mut();
        let st = unsafe { (api.gguf_open)(c.as_ptr(), &mut handle) };
        if st != 0 {
            return Err(Self::error(api, st));
        }
        let mut f = Self { api, handle, version: 0, data_offset: 0, n_tensors: 0, n_meta: 0 };
        let (mut v, mut off, mut nt, mut nm) = (0u32, 0u64, 0i64, 0i64);
        f.check(unsafe { (api.gguf_header)(handle, &mut v, &mut off, &mut nt, &mut nm) })?;
        f.version = v;
        f.data_offset = off;
        f.n_tensors = nt as usize;
        f.n_meta = nm as usize;
        Ok(f)
    }

    pub fn tensor(&self, index: usize) -> Result<GgufTensor> {
        let mut i = std::mem::MaybeUninit::<ffi::MrmlGgufTensorInfo>::zeroed();
        self.check(unsafe { (self.api.gguf_tensor)(self.handle, index as i64, i.as_mut_ptr()) })?;
        let i = unsafe { i.assume_init() };
        Ok(GgufTensor {
            name: unsafe { CStr::from_ptr(i.name) }.to_string_lossy().into_owned(),
            type_id: i.type_id,
            dims: i.dims[..i.n_dims.clamp(0, 4) as usize].to_vec(),
            offset: i.offset,
            size_bytes: i.size_bytes,
        })
    }

    pub fn find_tensor(&self, name: &str) -> Result<usize> {
        let c = CString::new(name).map_err(|e| Error { status: ffi::MRML_HIP_E_INVALID, message: e.to_string() })?;
        let mut index = 0i64;
        self.check(unsafe { (self.api.gguf_find_tensor)(self.handle, c.as_ptr(), &mut index) })?;
        Ok(index as usize)
    }

    /// `GgufFile::read_tensor_bytes`: the tensor's stored bytes.
    pub fn read_tensor_bytes(&self, index: usize) -> Result<Vec<u8>> {
        let t = self.tensor(index)?;
        let mut out = vec![0u8; t.size_bytes as usize];
        self.check(unsafe {
            (self.api.gguf_read_tensor)(self.handle, index as i64, out.as_mut_ptr() as *mut std::ffi::c_void, t.size_bytes)
        })?;
        Ok(out)
    }

    pub fn meta_u32(&self, key: &str) -> Result<u32> {
        let c = CString::new(key).unwrap();
        let mut v = 0u32;
        self.check(unsafe { (self.api.gguf_meta_u32)(self.handle, c.as_ptr(), &mut v) })?;
        Ok(v)
    }

    pub fn meta_f32(&self, key: &str) -> Result<f32> {
        let c = CString::new(key).unwrap();
        let mut v = 0f32;
        self.check(unsafe { (self.api.gguf_meta_f32)(self.handle, c.as_ptr(), &mut v) })?;
        Ok(v)
    }

    pub fn meta_str(&self, key: &str) -> Result<String> {
        let c = CString::new(key).unwrap();
        let (mut p, mut n): (*const c_char, u64) = (std::ptr::null(), 0);
        self.check(unsafe { (self.api.gguf_meta_str)(self.handle, c.as_ptr(), &mut p, &mut n) })?;
        let bytes = unsafe { std::slice::from_raw_parts(p as *const u8, n as usize) };
        Ok(String::from_utf8_lossy(bytes).into_owned())
    }

    /// (item type, length) of an array value.
    pub fn meta_array(&self, key: &str) -> Result<(i32, u64)> {
        let c = CString::new(key).unwrap();
        let (mut t, mut n) = (0i32, 0u64);
        self.check(unsafe { (self.api.gguf_meta_array)(self.handle, c.as_ptr(), &mut t, &mut n) })?;
        Ok((t, n))
    }

    /// Key `index` of the metadata (key-byte order) and its value type.
    pub fn meta_key(&self, index: usize) -> Result<(String, i32)> {
        let (mut k, mut t): (*const c_char, i32) = (std::ptr::null(), 0);
        self.check(unsafe { (self.api.gguf_meta_key)(self.handle, index as i64, &mut k, &mut t) })?;
        Ok((unsafe { CStr::from_ptr(k) }.to_string_lossy().into_owned(), t))
    }
}

impl Drop for GgufFile {
    fn drop(&mut self) {
        unsafe { (self.api.gguf_close)(self.handle) };
    }
}
