//! `CudaDevice` / `CudaBuffer` / `CudaGraphExec` over `libmrml_hip.so`.

use std::ffi::{c_void, CStr};
use std::marker::PhantomData;
use std::sync::atomic::{AtomicUsize, Ordering};
use std::sync::Arc;

use crate::ffi::{self, Api, Ctx};
use crate::{load_error, Error, Result};

/// The context shared by a device and everything allocated on it: the last
/// owner destroys it (after the buffers and graphs that hold it are gone).
pub(crate) struct Inner {
    pub(crate) api: &'static Api,
    pub(crate) ctx: Ctx,
}

unsafe impl Send for Inner {}
unsafe impl Sync for Inner {}

impl Inner {
    pub(crate) fn error(&self, status: i32) -> Error {
        let msg = unsafe { (self.api.last_error)(self.ctx) };
        let message = if msg.is_null() { String::new() } else { unsafe { CStr::from_ptr(msg) }.to_string_lossy().into_owned() };
        Error { status, message }
    }

    pub(crate) fn check(&self, status: i32) -> Result<()> {
        if status == 0 { Ok(()) } else { Err(self.error(status)) }
    }

    /// The reference's launch contract (`.expect(...)`, cuda.rs:2304): a
    /// failed operator launch panics.
    pub(crate) fn expect(&self, status: i32, what: &str) {
        if status != 0 {
            panic!("{what} failed: {}", self.error(status));
        }
    }
}

impl Drop for Inner {
    fn drop(&mut self) {
        unsafe { (self.api.destroy)(self.ctx) };
    }
}

/// `CudaDeviceInfo` (cuda.rs:1860-1878) with the AMD fields.
#[derive(Clone, Debug)]
pub struct DeviceInfo {
    pub name: String,
    pub compute_units: i32,
    pub clock_khz: i32,
    pub runtime_version: i32,
    pub abi_version: i32,
    pub total_memory: u64,
    pub l2_bytes: u64,
}

/// One gfx950 device and its stream (`CudaDevice`, cuda.rs:1516-1535).
#[derive(Clone)]
pub struct HipDevice {
    pub(crate) inner: Arc<Inner>,
    device_id: i32,
}

/// A device allocation of `len` elements (`CudaBuffer<T>`, cuda.rs:1243-1513).
pub struct HipBuffer<T> {
    inner: Arc<Inner>,
    ptr: *mut T,
    len: usize,
    allocation: Allocation,
    _t: PhantomData<T>,
}

/// Who frees a buffer's memory (`CudaAllocation`, cuda.rs:1251-1255): the
/// buffer itself, or the arena it was cut from (kept alive by the buffer).
enum Allocation {
    Owned,
    Arena(Arc<ArenaAllocation>),
}

struct ArenaAllocation {
    inner: Arc<Inner>,
    ptr: *mut c_void,
    bytes: usize,
}

unsafe impl Send for ArenaAllocation {}
unsafe impl Sync for ArenaAllocation {}

impl Drop for ArenaAllocation {
    fn drop(&mut self) {
        unsafe { (self.inner.api.free)(self.inner.ctx, self.ptr) };
    }
}

/// `CudaArena` (cuda.rs:1274-1331): one device allocation handed out in
/// 256-byte-aligned pieces; the pieces free nothing, the allocation goes
/// when the arena and every piece are gone.
#[derive(Clone)]
pub struct HipArena {
    allocation: Arc<ArenaAllocation>,
    next: Arc<AtomicUsize>,
}

impl HipArena {
    pub fn new(device: &HipDevice, bytes: usize) -> Result<Self> {
        let mut p = std::ptr::null_mut();
        device.inner.check(unsafe { (device.inner.api.malloc)(device.inner.ctx, bytes.max(1), &mut p) })?;
        Ok(Self {
            allocation: Arc::new(ArenaAllocation { inner: device.inner.clone(), ptr: p, bytes }),
            next: Arc::new(AtomicUsize::new(0)),
        })
    }

    /// `len` elements from the arena; `MRML_HIP_E_ALLOC` when it is exhausted.
    pub fn alloc<T>(&self, len: usize) -> Result<HipBuffer<T>> {
        let bytes = len.checked_mul(std::mem::size_of::<T>()).ok_or_else(|| Error {
            status: ffi::MRML_HIP_E_ALLOC,
            message: "arena allocation size overflows".into(),
        })?;
        let aligned = (bytes + 255) & !255;
        let offset = self.next.fetch_add(aligned, Ordering::Relaxed);
        if offset + aligned > self.allocation.bytes {
            self.next.fetch_sub(aligned, Ordering::Relaxed);
            return Err(Error {
                status: ffi::MRML_HIP_E_ALLOC,
                message: format!("arena exhausted: requested {bytes} bytes, {} remain",
                                 self.allocation.bytes.saturating_sub(offset)),
            });
        }
        Ok(HipBuffer {
            inner: self.allocation.inner.clone(),
            ptr: unsafe { (self.allocation.ptr as *mut u8).add(offset) } as *mut T,
            len,
            allocation: Allocation::Arena(self.allocation.clone()),
            _t: PhantomData,
        })
    }

    pub fn used_bytes(&self) -> usize {
        self.next.load(Ordering::Relaxed)
    }

    pub fn capacity_bytes(&self) -> usize {
        self.allocation.bytes
    }
}

unsafe impl<T: Send> Send for HipBuffer<T> {}
unsafe impl<T: Sync> Sync for HipBuffer<T> {}

/// An instantiated graph of captured launches (`CudaGraphExec`, cuda.rs:1841-1858).
pub struct HipGraph {
    inner: Arc<Inner>,
    exec: *mut c_void,
}

impl Drop for HipGraph {
    fn drop(&mut self) {
        unsafe { (self.inner.api.graph_destroy)(self.inner.ctx, self.exec) };
    }
}

fn i32_of(v: usize, what: &str) -> i32 {
    i32::try_from(v).unwrap_or_else(|_| panic!("{what} = {v} does not fit the ABI's i32"))
}

impl HipDevice {
    /// `CudaDevice::new` (cuda.rs:2068-2087).
    pub fn new(device_id: i32) -> Result<Self> {
        let api = ffi::api().map_err(load_error)?;
        let mut ctx: Ctx = std::ptr::null_mut();
        let st = unsafe { (api.create)(device_id, &mut ctx) };
        if st != 0 {
            let msg = unsafe { (api.status_string)(st) };
            let message = if msg.is_null() { String::new() } else { unsafe { CStr::from_ptr(msg) }.to_string_lossy().into_owned() };
            return Err(Error { status: st, message });
        }
        Ok(Self { inner: Arc::new(Inner { api, ctx }), device_id })
    }

    /// `CudaDevice::count` (cuda.rs:2041-2049): 0 when the library or a
    /// gfx950 device is missing.
    pub fn count() -> usize {
        let Ok(api) = ffi::api() else { return 0 };
        let mut n = 0i32;
        if unsafe { (api.device_count)(&mut n) } != 0 { 0 } else { n.max(0) as usize }
    }

    /// `CudaDevice::is_available` (cuda.rs:2051-2053).
    pub fn is_available() -> bool {
        Self::count() > 0
    }

    pub fn device_id(&self) -> i32 {
        self.device_id
    }

    /// `CudaDevice::sync` (cuda.rs:2089-2100); also reports a bounded wait
    /// that gave up since the last synchronisation.
    pub fn sync(&self) -> Result<()> {
        self.inner.check(unsafe { (self.inner.api.sync)(self.inner.ctx) })
    }

    pub fn device_info(&self) -> Result<DeviceInfo> {
        let mut i = std::mem::MaybeUninit::<ffi::MrmlHipDeviceInfo>::zeroed();
        self.inner.check(unsafe { (self.inner.api.device_info_get)(self.inner.ctx, i.as_mut_ptr()) })?;
        let i = unsafe { i.assume_init() };
        let name = unsafe { CStr::from_ptr(i.name.as_ptr()) }.to_string_lossy().into_owned();
        Ok(DeviceInfo {
            name,
            compute_units: i.compute_units,
            clock_khz: i.clock_khz,
            runtime_version: i.runtime_version,
            abi_version: i.abi_version,
            total_memory: i.total_memory,
            l2_bytes: i.l2_bytes,
        })
    }

    /// `CudaDevice::get_memory_info` (cuda.rs:2055-2066): (free, total) bytes.
    pub fn get_memory_info(&self) -> Result<(usize, usize)> {
        let (mut free, mut total) = (0u64, 0u64);
        self.inner.check(unsafe { (self.inner.api.memory_info)(self.inner.ctx, &mut free, &mut total) })?;
        Ok((free as usize, total as usize))
    }

    /// Sizes the context workspace once, ahead of a capture.
    pub fn reserve_workspace(&self, bytes: usize) -> Result<()> {
        self.inner.check(unsafe { (self.inner.api.reserve_workspace)(self.inner.ctx, bytes) })
    }

    /// Current size of the internal scratch (no `CudaDevice` counterpart).
    pub fn workspace_bytes(&self) -> Result<usize> {
        let mut n = 0usize;
        self.inner.check(unsafe { (self.inner.api.workspace_bytes)(self.inner.ctx, &mut n) })?;
        Ok(n)
    }

    /// `CudaDevice::capture` (cuda.rs:1957-1994): every launch `launches`
    /// issues on this device becomes one replayable graph.
    pub fn capture<F: FnOnce()>(&self, launches: F) -> Result<HipGraph> {
        self.inner.check(unsafe { (self.inner.api.graph_begin)(self.inner.ctx) })?;
        launches();
        let mut exec = std::ptr::null_mut();
        self.inner.check(unsafe { (self.inner.api.graph_end)(self.inner.ctx, &mut exec) })?;
        Ok(HipGraph { inner: self.inner.clone(), exec })
    }

    /// `CudaDevice::launch_graph` (cuda.rs:1996-2003).
    pub fn launch_graph(&self, graph: &HipGraph) -> Result<()> {
        self.inner.check(unsafe { (self.inner.api.graph_launch)(self.inner.ctx, graph.exec) })
    }

    /// `CudaDevice::copy_from_host_async` (cuda.rs:2334-2350).
    pub fn copy_from_host_async<T: Copy>(&self, dst: &mut HipBuffer<T>, src: &[T]) -> Result<()> {
        assert!(src.len() <= dst.len, "copy_from_host_async: {} elements into {}", src.len(), dst.len);
        self.inner.check(unsafe {
            (self.inner.api.memcpy_h2d_async)(self.inner.ctx, dst.ptr as *mut c_void, src.as_ptr() as *const c_void,
                                              std::mem::size_of_val(src))
        })
    }

    /// `CudaDevice::copy_from_host_at_async` (cuda.rs:2352-2376): `src` into
    /// elements offset.. of `dst`, ordered on the stream (model.rs:1525-1526
    /// writes KV rows this way).
    pub fn copy_from_host_at_async<T: Copy>(&self, dst: &mut HipBuffer<T>, offset: usize, src: &[T]) -> Result<()> {
        assert!(offset + src.len() <= dst.len, "copy_from_host_at_async: {}+{} elements into {}", offset, src.len(),
                dst.len);
        self.inner.check(unsafe {
            (self.inner.api.memcpy_h2d_async)(self.inner.ctx, dst.ptr.add(offset) as *mut c_void,
                                              src.as_ptr() as *const c_void, std::mem::size_of_val(src))
        })
    }

    /// `CudaDevice::add` (cuda.rs:2579-2593): out = a + b elementwise.
    pub fn add(&self, d_a: &HipBuffer<f32>, d_b: &HipBuffer<f32>, d_out: &mut HipBuffer<f32>) {
        assert_eq!(d_a.len, d_b.len);
        assert_eq!(d_a.len, d_out.len);
        let st = unsafe { (self.inner.api.add)(self.inner.ctx, d_a.ptr, d_b.ptr, d_out.ptr, i32_of(d_a.len, "len")) };
        self.inner.expect(st, "add");
    }

    /// `CudaDevice::embedding` (cuda.rs:2595-2623): row `token` of an f32
    /// table, a device-to-device copy on the stream.
    pub fn embedding(&self, d_table: &HipBuffer<f32>, d_out: &mut HipBuffer<f32>, token: usize, dim: usize) {
        assert!((token + 1) * dim <= d_table.len && dim <= d_out.len, "embedding: row {token} of {dim} outside the table");
        let st = unsafe {
            (self.inner.api.memcpy_d2d_async)(self.inner.ctx, d_out.ptr as *mut c_void,
                                              d_table.ptr.add(token * dim) as *const c_void, dim * 4)
        };
        self.inner.expect(st, "embedding");
    }

    // ---- weights: GGUF blocks in, backend layouts out ----------------------------

    fn upload(&self, gguf: &[u8], rows: usize, cols: usize,
              repack: unsafe extern "C" fn(Ctx, *const c_void, *mut c_void, i32, i32) -> i32) -> Result<HipBuffer<u8>> {
        let raw = HipBuffer::from_host_on(self, gguf)?;
        let out = HipBuffer::<u8>::alloc_on(self, gguf.len())?;
        self.inner.check(unsafe {
            repack(self.inner.ctx, raw.ptr as *const c_void, out.ptr as *mut c_void, i32_of(rows, "rows"), i32_of(cols, "cols"))
        })?;
        self.sync()?;
        Ok(out)
    }

    /// A Q4_0 matrix (rows x cols, GGUF blocks as in model.rs:651-705) in the
    /// layout of the Q4_0 products.
    pub fn upload_q4_0(&self, gguf: &[u8], rows: usize, cols: usize) -> Result<HipBuffer<u8>> {
        self.upload(gguf, rows, cols, self.inner.api.repack_q4_0)
    }

    pub fn upload_q8_0(&self, gguf: &[u8], rows: usize, cols: usize) -> Result<HipBuffer<u8>> {
        self.upload(gguf, rows, cols, self.inner.api.repack_q8_0)
    }

    pub fn upload_q4_k(&self, gguf: &[u8], rows: usize, cols: usize) -> Result<HipBuffer<u8>> {
        self.upload(gguf, rows, cols, self.inner.api.repack_q4_k)
    }

    // ---- the operators (cuda.rs:2102-3111), same names and arguments ----------------

    /// `CudaDevice::rms_norm` (cuda.rs:2102-2137): dim = `d_x.len()`.
    pub fn rms_norm(&self, d_x: &HipBuffer<f32>, d_weight: Option<&HipBuffer<f32>>, d_out: &mut HipBuffer<f32>, eps: f32) {
        let w = d_weight.map_or(std::ptr::null(), |w| w.ptr as *const f32);
        let st = unsafe {
            (self.inner.api.rms_norm)(self.inner.ctx, d_x.ptr, w, d_out.ptr, std::ptr::null_mut(), i32_of(d_x.len, "dim"), eps)
        };
        self.inner.expect(st, "rms_norm");
    }

    /// `CudaDevice::rms_norm_batch` (cuda.rs:2139-2180).
    pub fn rms_norm_batch(&self, d_x: &HipBuffer<f32>, d_weight: Option<&HipBuffer<f32>>, d_out: &mut HipBuffer<f32>,
                          dim: usize, batch: usize, eps: f32) {
        let w = d_weight.map_or(std::ptr::null(), |w| w.ptr as *const f32);
        let st = unsafe {
            (self.inner.api.rms_norm_batch)(self.inner.ctx, d_x.ptr, w, d_out.ptr, i32_of(dim, "dim"), i32_of(batch, "batch"), eps)
        };
        self.inner.expect(st, "rms_norm_batch");
    }

    /// `CudaDevice::gemv_q4_0` (cuda.rs:2286-2306).
    pub fn gemv_q4_0(&self, d_w_q4: &HipBuffer<u8>, d_x: &HipBuffer<f32>, d_y: &mut HipBuffer<f32>, n_rows: usize, n_cols: usize) {
        let st = unsafe {
            (self.inner.api.gemv_q4_0)(self.inner.ctx, d_w_q4.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(n_rows, "n_rows"),
                                       i32_of(n_cols, "n_cols"))
        };
        self.inner.expect(st, "gemv_q4_0");
    }

    /// `CudaDevice::gemm_q4_0` (cuda.rs:2308-2332): x [batch][n_cols] -> y [batch][n_rows].
    pub fn gemm_q4_0(&self, d_w_q4: &HipBuffer<u8>, d_x: &HipBuffer<f32>, d_y: &mut HipBuffer<f32>, n_rows: usize,
                     n_cols: usize, batch: usize) {
        let st = unsafe {
            (self.inner.api.gemm_q4_0)(self.inner.ctx, d_w_q4.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(n_rows, "n_rows"),
                                       i32_of(n_cols, "n_cols"), i32_of(batch, "batch"))
        };
        self.inner.expect(st, "gemm_q4_0");
    }

    /// `CudaDevice::gemv_q4_0_qkv` (cuda.rs:2378-2404): y = [q | k | v].
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_q4_0_qkv(&self, d_w_q: &HipBuffer<u8>, d_w_k: &HipBuffer<u8>, d_w_v: &HipBuffer<u8>, d_x: &HipBuffer<f32>,
                         d_y: &mut HipBuffer<f32>, q_rows: usize, kv_rows: usize, n_cols: usize) {
        let st = unsafe {
            (self.inner.api.gemv_q4_0_qkv)(self.inner.ctx, d_w_q.ptr as *const c_void, d_w_k.ptr as *const c_void,
                                           d_w_v.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(q_rows, "q_rows"),
                                           i32_of(kv_rows, "kv_rows"), i32_of(n_cols, "n_cols"))
        };
        self.inner.expect(st, "gemv_q4_0_qkv");
    }

    /// `CudaDevice::gemm_q4_0_qkv` (cuda.rs:2406-2436): per token, y row = [q | k | v].
    #[allow(clippy::too_many_arguments)]
    pub fn gemm_q4_0_qkv(&self, d_w_q: &HipBuffer<u8>, d_w_k: &HipBuffer<u8>, d_w_v: &HipBuffer<u8>, d_x: &HipBuffer<f32>,
                         d_y: &mut HipBuffer<f32>, q_rows: usize, kv_rows: usize, n_cols: usize, batch: usize) {
        let st = unsafe {
            (self.inner.api.gemm_q4_0_qkv)(self.inner.ctx, d_w_q.ptr as *const c_void, d_w_k.ptr as *const c_void,
                                           d_w_v.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(q_rows, "q_rows"),
                                           i32_of(kv_rows, "kv_rows"), i32_of(n_cols, "n_cols"), i32_of(batch, "batch"))
        };
        self.inner.expect(st, "gemm_q4_0_qkv");
    }

    /// `CudaDevice::gemv_q4_0_geglu` (cuda.rs:2521-2544): act = gelu(Wg x) * (Wu x).
    pub fn gemv_q4_0_geglu(&self, d_w_gate: &HipBuffer<u8>, d_w_up: &HipBuffer<u8>, d_x: &HipBuffer<f32>,
                           d_act: &mut HipBuffer<f32>, n_rows: usize, n_cols: usize) {
        let st = unsafe {
            (self.inner.api.gemv_q4_0_geglu)(self.inner.ctx, d_w_gate.ptr as *const c_void, d_w_up.ptr as *const c_void,
                                             d_x.ptr, d_act.ptr, i32_of(n_rows, "n_rows"), i32_of(n_cols, "n_cols"))
        };
        self.inner.expect(st, "gemv_q4_0_geglu");
    }

    /// `CudaDevice::gemm_q4_0_geglu` (cuda.rs:2699-2725).
    #[allow(clippy::too_many_arguments)]
    pub fn gemm_q4_0_geglu(&self, d_w_gate: &HipBuffer<u8>, d_w_up: &HipBuffer<u8>, d_x: &HipBuffer<f32>,
                           d_act: &mut HipBuffer<f32>, n_rows: usize, n_cols: usize, batch: usize) {
        let st = unsafe {
            (self.inner.api.gemm_q4_0_geglu)(self.inner.ctx, d_w_gate.ptr as *const c_void, d_w_up.ptr as *const c_void,
                                             d_x.ptr, d_act.ptr, i32_of(n_rows, "n_rows"), i32_of(n_cols, "n_cols"),
                                             i32_of(batch, "batch"))
        };
        self.inner.expect(st, "gemm_q4_0_geglu");
    }

    /// `CudaDevice::gemv_q8_0` (cuda.rs:2546-2577): the LM head, 30*tanh(y/30)
    /// as the device path applies it (kernels.rs:552-595).
    pub fn gemv_q8_0(&self, d_w_q8: &HipBuffer<u8>, d_x: &HipBuffer<f32>, d_y: &mut HipBuffer<f32>, n_rows: usize, n_cols: usize) {
        self.gemv_q8_0_softcap(d_w_q8, d_x, d_y, n_rows, n_cols, true);
    }

    /// The Q8_0 product with or without the softcap (the CPU path softcaps in
    /// its vocabulary loop instead, model.rs:2851-2853).
    pub fn gemv_q8_0_softcap(&self, d_w_q8: &HipBuffer<u8>, d_x: &HipBuffer<f32>, d_y: &mut HipBuffer<f32>, n_rows: usize,
                             n_cols: usize, softcap: bool) {
        let st = unsafe {
            (self.inner.api.gemv_q8_0)(self.inner.ctx, d_w_q8.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(n_rows, "n_rows"),
                                       i32_of(n_cols, "n_cols"), softcap as i32)
        };
        self.inner.expect(st, "gemv_q8_0");
    }

    /// The GGUF Q4_K product (no reference counterpart; GGUF semantics).
    pub fn gemv_q4_k(&self, d_w: &HipBuffer<u8>, d_x: &HipBuffer<f32>, d_y: &mut HipBuffer<f32>, n_rows: usize, n_cols: usize) {
        let st = unsafe {
            (self.inner.api.gemv_q4_k)(self.inner.ctx, d_w.ptr as *const c_void, d_x.ptr, d_y.ptr, i32_of(n_rows, "n_rows"),
                                       i32_of(n_cols, "n_cols"))
        };
        self.inner.expect(st, "gemv_q4_k");
    }

    /// `CudaDevice::embedding_q8_0` (cuda.rs:2625-2656): row `token` of a Q8_0
    /// table times `output_scale`.
    pub fn embedding_q8_0(&self, d_table: &HipBuffer<u8>, d_out: &mut HipBuffer<f32>, token: usize, dim: usize, output_scale: f32) {
        let vocab = d_table.len / (dim / 32 * 34);
        let st = unsafe {
            (self.inner.api.embedding)(self.inner.ctx, d_table.ptr as *const c_void, ffi::MRML_HIP_Q8_0, i32_of(token, "token"),
                                       std::ptr::null(), d_out.ptr, i32_of(dim, "dim"), i32_of(vocab, "vocab"), output_scale)
        };
        self.inner.expect(st, "embedding_q8_0");
    }

    /// `CudaDevice::attention_causal` (cuda.rs:2658-2697) for one token, with
    /// the reference's arguments: the cache is a ring of `cache_capacity`
    /// positions, `sliding_window` limits the window below it, and the cache
    /// formats must be 0 (f16 rows, `KvCacheFormat::cuda_code`).
    #[allow(clippy::too_many_arguments)]
    pub fn attention_causal(&self, d_q: &HipBuffer<f32>, d_k_cache: &HipBuffer<u16>, d_v_cache: &HipBuffer<u16>,
                            d_out: &mut HipBuffer<f32>, n_past: usize, n_heads: usize, n_kv_heads: usize, head_dim: usize,
                            scale: f32, sliding_window: Option<usize>, cache_capacity: usize, k_format: i32,
                            v_format: i32) {
        let sw = sliding_window.map(|w| i32_of(w, "sliding_window")).unwrap_or(-1);
        let st = unsafe {
            (self.inner.api.attention_causal)(self.inner.ctx, d_q.ptr, d_k_cache.ptr, d_v_cache.ptr, d_out.ptr,
                                              i32_of(n_past, "n_past"), i32_of(n_heads, "n_heads"),
                                              i32_of(n_kv_heads, "n_kv_heads"), i32_of(head_dim, "head_dim"), scale, sw,
                                              i32_of(cache_capacity, "cache_capacity"), k_format, v_format)
        };
        self.inner.expect(st, "attention_causal");
    }

    /// `CudaDevice::attention_prefill` (cuda.rs:2727-2770): `batch` queries at
    /// positions `cache_start + i`, query rows `d_q.len / batch` floats apart;
    /// row i equals `attention_causal` at `n_past = cache_start + i`.
    #[allow(clippy::too_many_arguments)]
    pub fn attention_prefill(&self, d_q: &HipBuffer<f32>, d_k_cache: &HipBuffer<u16>, d_v_cache: &HipBuffer<u16>,
                             d_out: &mut HipBuffer<f32>, cache_start: usize, batch: usize, n_heads: usize,
                             n_kv_heads: usize, head_dim: usize, scale: f32, sliding_window: Option<usize>,
                             cache_capacity: usize, k_format: i32, v_format: i32) {
        let q_stride = d_q.len / batch;
        assert!(q_stride >= n_heads * head_dim);
        assert_eq!(d_out.len, batch * n_heads * head_dim);
        let sw = sliding_window.map(|w| i32_of(w, "sliding_window")).unwrap_or(-1);
        let st = unsafe {
            (self.inner.api.attention_prefill)(self.inner.ctx, d_q.ptr, i32_of(q_stride, "q_stride"), d_k_cache.ptr,
                                               d_v_cache.ptr, d_out.ptr, i32_of(cache_start, "cache_start"),
                                               i32_of(batch, "batch"), i32_of(n_heads, "n_heads"),
                                               i32_of(n_kv_heads, "n_kv_heads"), i32_of(head_dim, "head_dim"), scale, sw,
                                               i32_of(cache_capacity, "cache_capacity"), k_format, v_format)
        };
        self.inner.expect(st, "attention_prefill");
    }

    /// `CudaDevice::qkv_postprocess_batch` (cuda.rs:2478-2519) without the
    /// Gemma-4 head norms: RoPE of `batch` stacked q|k|v rows at `start_pos + i`
    /// and their k/v to cache rows `(cache_start + i) % cache_capacity`.
    #[allow(clippy::too_many_arguments)]
    pub fn rope_kv_append_f16_batch(&self, qkv: &mut HipBuffer<f32>, k_cache: &mut HipBuffer<u16>,
                                    v_cache: &mut HipBuffer<u16>, start_pos: usize, cache_start: usize, n_heads: usize,
                                    n_kv_heads: usize, head_dim: usize, freq_base: f32, batch: usize,
                                    cache_capacity: usize, k_format: i32, v_format: i32) {
        assert_eq!(qkv.len, batch * (n_heads + 2 * n_kv_heads) * head_dim);
        let st = unsafe {
            (self.inner.api.rope_kv_append_f16_batch)(self.inner.ctx, qkv.ptr, k_cache.ptr, v_cache.ptr,
                                                      i32_of(start_pos, "start_pos"), i32_of(cache_start, "cache_start"),
                                                      i32_of(batch, "batch"), i32_of(n_heads, "n_heads"),
                                                      i32_of(n_kv_heads, "n_kv_heads"), i32_of(head_dim, "head_dim"),
                                                      freq_base, 1.0, i32_of(cache_capacity, "cache_capacity"),
                                                      k_format, v_format, std::ptr::null(), 0)
        };
        self.inner.expect(st, "rope_kv_append_f16_batch");
    }

    /// `CudaDevice::rope_256k` (cuda.rs:2248-2285): RoPE of `n_heads` heads of
    /// `d_vec` in place at position `pos`.
    pub fn rope_256k(&self, d_vec: &mut HipBuffer<f32>, pos: usize, head_dim: usize, n_heads: usize, freq_base: f32,
                     freq_scale: f32) {
        let st = unsafe {
            (self.inner.api.rope)(self.inner.ctx, d_vec.ptr, i32_of(pos, "pos"), i32_of(head_dim, "head_dim"),
                                  i32_of(n_heads, "n_heads"), freq_base, freq_scale, std::ptr::null(), 0)
        };
        self.inner.expect(st, "rope_256k");
    }

    /// `CudaDevice::geglu` (cuda.rs:2215-2246): out = gelu_tanh(gate) * up.
    pub fn geglu(&self, d_gate: &HipBuffer<f32>, d_up: &HipBuffer<f32>, d_out: &mut HipBuffer<f32>) {
        assert_eq!(d_gate.len, d_up.len);
        assert_eq!(d_gate.len, d_out.len);
        let st = unsafe { (self.inner.api.geglu)(self.inner.ctx, d_gate.ptr, d_up.ptr, d_out.ptr, i32_of(d_gate.len, "len")) };
        self.inner.expect(st, "geglu");
    }

    /// `CudaDevice::swiglu` (cuda.rs:2182-2213): out = silu(gate) * up.
    pub fn swiglu(&self, d_gate: &HipBuffer<f32>, d_up: &HipBuffer<f32>, d_out: &mut HipBuffer<f32>) {
        assert_eq!(d_gate.len, d_up.len);
        assert_eq!(d_gate.len, d_out.len);
        let st = unsafe { (self.inner.api.swiglu)(self.inner.ctx, d_gate.ptr, d_up.ptr, d_out.ptr, i32_of(d_gate.len, "len")) };
        self.inner.expect(st, "swiglu");
    }

    /// Greedy pick over `n` scores: lowest index on ties, NaN never wins.
    pub fn argmax_f32(&self, d_x: &HipBuffer<f32>, n: usize, d_out: &mut HipBuffer<i32>) {
        let st = unsafe { (self.inner.api.argmax_f32)(self.inner.ctx, d_x.ptr, i32_of(n, "n"), d_out.ptr) };
        self.inner.expect(st, "argmax_f32");
    }

    /// `CudaDevice::vocab_topk` (cuda.rs:3052-3111): each partition's `k` best
    /// (score, id), (-inf, -1) past its candidates.
    #[allow(clippy::too_many_arguments)]
    pub fn vocab_topk(&self, logits: &HipBuffer<f32>, valid: &HipBuffer<u8>, recent: &HipBuffer<i32>,
                      scores: &mut HipBuffer<f32>, ids: &mut HipBuffer<i32>, vocab_size: usize, n_recent: usize,
                      generated_count: usize, k: usize, partitions: usize) {
        assert!(valid.len >= vocab_size && recent.len >= n_recent);
        assert!(scores.len >= k * partitions && ids.len >= k * partitions);
        let st = unsafe {
            (self.inner.api.vocab_topk)(self.inner.ctx, logits.ptr, valid.ptr, recent.ptr, scores.ptr, ids.ptr,
                                        i32_of(vocab_size, "vocab_size"), i32_of(n_recent, "n_recent"),
                                        i32_of(generated_count, "generated_count"), i32_of(k, "k"),
                                        i32_of(partitions, "partitions"))
        };
        self.inner.expect(st, "vocab_topk");
    }

    /// The whole next-token pick of step_generation (model.rs:2842-2907) on
    /// the device: scoring `ffi::MRML_HIP_SCORE_CPU` (softcap, -3.5 once) or
    /// `_DEVICE` (-1.8 per occurrence), the `k` best, then greedy
    /// (temperature <= 0) or the reference's draw at `pos`.
    #[allow(clippy::too_many_arguments)]
    pub fn vocab_select(&self, logits: &HipBuffer<f32>, vocab_size: usize, valid: Option<&HipBuffer<u8>>,
                        recent: Option<&HipBuffer<i32>>, n_recent: usize, generated_count: usize, scoring: i32,
                        temperature: f32, pos: u64, k: usize, token: &mut HipBuffer<i32>,
                        scores: Option<&mut HipBuffer<f32>>, ids: Option<&mut HipBuffer<i32>>) {
        let st = unsafe {
            (self.inner.api.vocab_select)(self.inner.ctx, logits.ptr, i32_of(vocab_size, "vocab_size"),
                                          valid.map_or(std::ptr::null(), |v| v.ptr as *const u8),
                                          recent.map_or(std::ptr::null(), |r| r.ptr as *const i32),
                                          i32_of(n_recent, "n_recent"), i32_of(generated_count, "generated_count"), scoring,
                                          temperature, pos, i32_of(k, "k"), token.ptr,
                                          scores.map_or(std::ptr::null_mut(), |s| s.ptr),
                                          ids.map_or(std::ptr::null_mut(), |i| i.ptr))
        };
        self.inner.expect(st, "vocab_select");
    }
}

impl<T> HipBuffer<T> {
    /// `CudaBuffer::alloc_on` (cuda.rs:1350-1370): `len` elements, contents undefined.
    pub fn alloc_on(device: &HipDevice, len: usize) -> Result<Self> {
        let bytes = len.checked_mul(std::mem::size_of::<T>()).expect("allocation size overflows");
        let mut p = std::ptr::null_mut();
        device.inner.check(unsafe { (device.inner.api.malloc)(device.inner.ctx, bytes.max(1), &mut p) })?;
        Ok(Self { inner: device.inner.clone(), ptr: p as *mut T, len, allocation: Allocation::Owned, _t: PhantomData })
    }

    /// `CudaBuffer::alloc_pooled_on` (cuda.rs:1372-1390).  The library keeps
    /// no free-list of its own, so this is `alloc_on`; a caller that wants
    /// reuse without allocation cuts buffers from a `HipArena`.
    pub fn alloc_pooled_on(device: &HipDevice, len: usize) -> Result<Self> {
        Self::alloc_on(device, len)
    }

    /// `CudaBuffer::copy_from_host_at` (cuda.rs:1424-1441): `slice` into
    /// elements offset.., synchronous.
    pub fn copy_from_host_at(&mut self, offset: usize, slice: &[T]) -> Result<()>
    where
        T: Copy,
    {
        assert!(offset + slice.len() <= self.len, "copy_from_host_at: {}+{} elements into {}", offset, slice.len(),
                self.len);
        self.inner.check(unsafe {
            (self.inner.api.memcpy_h2d)(self.inner.ctx, self.ptr.add(offset) as *mut c_void,
                                        slice.as_ptr() as *const c_void, std::mem::size_of_val(slice))
        })
    }

    /// `CudaBuffer::from_host_on` (cuda.rs:1400-1404).
    pub fn from_host_on(device: &HipDevice, slice: &[T]) -> Result<Self>
    where
        T: Copy,
    {
        let mut b = Self::alloc_on(device, slice.len())?;
        b.copy_from_host(slice)?;
        Ok(b)
    }

    /// `CudaBuffer::copy_from_host` (cuda.rs:1406-1422): synchronous.
    pub fn copy_from_host(&mut self, slice: &[T]) -> Result<()>
    where
        T: Copy,
    {
        assert!(slice.len() <= self.len, "copy_from_host: {} elements into {}", slice.len(), self.len);
        self.inner.check(unsafe {
            (self.inner.api.memcpy_h2d)(self.inner.ctx, self.ptr as *mut c_void, slice.as_ptr() as *const c_void,
                                        std::mem::size_of_val(slice))
        })
    }

    /// `CudaBuffer::copy_to_host` (cuda.rs:1443-1446): the whole buffer.
    pub fn copy_to_host(&self, slice: &mut [T]) -> Result<()>
    where
        T: Copy,
    {
        assert_eq!(slice.len(), self.len, "copy_to_host: {} elements from {}", slice.len(), self.len);
        self.copy_prefix_to_host(slice)
    }

    /// `CudaBuffer::copy_prefix_to_host` (cuda.rs:1448-1465).
    pub fn copy_prefix_to_host(&self, slice: &mut [T]) -> Result<()>
    where
        T: Copy,
    {
        assert!(slice.len() <= self.len, "copy_prefix_to_host: {} elements from {}", slice.len(), self.len);
        self.inner.check(unsafe {
            (self.inner.api.memcpy_d2h)(self.inner.ctx, slice.as_mut_ptr() as *mut c_void, self.ptr as *const c_void,
                                        std::mem::size_of_val(slice))
        })
    }

    pub fn as_ptr(&self) -> *const T {
        self.ptr
    }

    pub fn as_mut_ptr(&mut self) -> *mut T {
        self.ptr
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
}

impl<T> Drop for HipBuffer<T> {
    fn drop(&mut self) {
        if let Allocation::Owned = self.allocation {
            unsafe { (self.inner.api.free)(self.inner.ctx, self.ptr as *mut c_void) };
        }
    }
}
