//! Raw C ABI of `libmrml_hip.so` (`include/mrml_hip.h`): the structs and one
//! table of function pointers, resolved with `dlsym` when the library is
//! first used.  Every entry below names its C symbol; the argument types are
//! the header's (`int32_t` -> `i32`, `size_t` -> `usize`, `T *` -> `*mut T`,
//! `const T *` -> `*const T`, opaque handles -> `*mut c_void`).

use std::ffi::{c_char, c_int, c_void, CStr, CString};
use std::sync::OnceLock;

pub const MRML_HIP_ABI_VERSION: i32 = 2;

pub const MRML_HIP_OK: i32 = 0;
pub const MRML_HIP_E_INVALID: i32 = -1;
pub const MRML_HIP_E_ALLOC: i32 = -2;
pub const MRML_HIP_E_HIP: i32 = -3;
pub const MRML_HIP_E_UNSUPPORTED: i32 = -4;
pub const MRML_HIP_E_NODEVICE: i32 = -5;
pub const MRML_HIP_E_FORMAT: i32 = -6;
pub const MRML_HIP_E_IO: i32 = -7;
pub const MRML_HIP_E_NOTFOUND: i32 = -8;

/// GGUF type ids of the repacked matrix layouts.
pub const MRML_HIP_Q4_0: i32 = 2;
pub const MRML_HIP_Q8_0: i32 = 8;
pub const MRML_HIP_Q4_K: i32 = 12;

pub const MRML_HIP_SCORE_CPU: i32 = 0;
pub const MRML_HIP_SCORE_DEVICE: i32 = 1;
pub const MRML_HIP_NUMERICS_EXACT: i32 = 0;
pub const MRML_HIP_NUMERICS_FAST: i32 = 1;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MrmlHipDeviceInfo {
    pub name: [c_char; 64],
    pub compute_units: i32,
    pub clock_khz: i32,
    pub runtime_version: i32,
    pub abi_version: i32,
    pub total_memory: u64,
    pub l2_bytes: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct MrmlHipGemma2Config {
    pub n_layers: i32,
    pub dim: i32,
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub ffn_dim: i32,
    pub vocab: i32,
    pub ctx_len: i32,
    pub rope_base: f32,
    pub eps: f32,
    pub attn_scale: f32,
    pub tie_type: i32,
    pub numerics: i32,
    pub sliding_window: i32,
    pub swa_period: i32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MrmlHipGemma2Layer {
    pub wq: *const c_void,
    pub wk: *const c_void,
    pub wv: *const c_void,
    pub wo: *const c_void,
    pub w_gate: *const c_void,
    pub w_up: *const c_void,
    pub w_down: *const c_void,
    pub attn_norm: *const f32,
    pub post_attn_norm: *const f32,
    pub ffn_norm: *const f32,
    pub post_ffw_norm: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MrmlHipSampler {
    pub d_valid: *const u8,
    pub temperature: f32,
    pub top_k: i32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct MrmlGgufTensorInfo {
    pub name: *const c_char,
    pub type_id: i32,
    pub n_dims: i32,
    pub dims: [u64; 4],
    pub offset: u64,
    pub size_bytes: u64,
}

pub type Ctx = *mut c_void;
pub type Model = *mut c_void;
pub type Gguf = *mut c_void;

extern "C" {
    fn dlopen(filename: *const c_char, flag: c_int) -> *mut c_void;
    fn dlsym(handle: *mut c_void, symbol: *const c_char) -> *mut c_void;
    fn dlerror() -> *const c_char;
}
const RTLD_NOW: c_int = 2;

macro_rules! api {
    ($($field:ident: fn($($arg:ty),*) -> $ret:ty = $sym:literal;)*) => {
        /// The library's entry points.
        pub struct Api {
            $(pub $field: unsafe extern "C" fn($($arg),*) -> $ret,)*
        }
        impl Api {
            unsafe fn resolve(lib: *mut c_void) -> Result<Api, String> {
                Ok(Api {
                    $($field: {
                        let p = dlsym(lib, concat!($sym, "\0").as_ptr() as *const c_char);
                        if p.is_null() {
                            return Err(format!("libmrml_hip.so has no symbol {}", $sym));
                        }
                        std::mem::transmute::<*mut c_void, unsafe extern "C" fn($($arg),*) -> $ret>(p)
                    },)*
                })
            }
        }
    };
}

api! {
    device_count: fn(*mut i32) -> c_int = "mrml_hip_device_count";
    create: fn(i32, *mut Ctx) -> c_int = "mrml_hip_create";
    destroy: fn(Ctx) -> c_int = "mrml_hip_destroy";
    last_error: fn(Ctx) -> *const c_char = "mrml_hip_last_error";
    status_string: fn(c_int) -> *const c_char = "mrml_hip_status_string";
    sync: fn(Ctx) -> c_int = "mrml_hip_sync";
    set_wait_limit: fn(Ctx, i32) -> c_int = "mrml_hip_set_wait_limit";
    device_info_get: fn(Ctx, *mut MrmlHipDeviceInfo) -> c_int = "mrml_hip_device_info_get";
    memory_info: fn(Ctx, *mut u64, *mut u64) -> c_int = "mrml_hip_memory_info";
    stream: fn(Ctx) -> *mut c_void = "mrml_hip_stream";
    reserve_workspace: fn(Ctx, usize) -> c_int = "mrml_hip_reserve_workspace";
    workspace_bytes: fn(Ctx, *mut usize) -> c_int = "mrml_hip_workspace_bytes";
    graph_begin: fn(Ctx) -> c_int = "mrml_hip_graph_begin";
    graph_end: fn(Ctx, *mut *mut c_void) -> c_int = "mrml_hip_graph_end";
    graph_launch: fn(Ctx, *mut c_void) -> c_int = "mrml_hip_graph_launch";
    graph_destroy: fn(Ctx, *mut c_void) -> c_int = "mrml_hip_graph_destroy";
    malloc: fn(Ctx, usize, *mut *mut c_void) -> c_int = "mrml_hip_malloc";
    free: fn(Ctx, *mut c_void) -> c_int = "mrml_hip_free";
    memcpy_h2d: fn(Ctx, *mut c_void, *const c_void, usize) -> c_int = "mrml_hip_memcpy_h2d";
    memcpy_d2h: fn(Ctx, *mut c_void, *const c_void, usize) -> c_int = "mrml_hip_memcpy_d2h";
    memcpy_h2d_async: fn(Ctx, *mut c_void, *const c_void, usize) -> c_int = "mrml_hip_memcpy_h2d_async";
    memcpy_d2d_async: fn(Ctx, *mut c_void, *const c_void, usize) -> c_int = "mrml_hip_memcpy_d2d_async";
    zero_async: fn(Ctx, *mut c_void, usize) -> c_int = "mrml_hip_zero_async";
    copy_kernel: fn(Ctx, *mut c_void, *const c_void, usize) -> c_int = "mrml_hip_copy_kernel";
    read_kernel: fn(Ctx, *const c_void, usize, *mut c_void) -> c_int = "mrml_hip_read_kernel";
    repack_q4_0: fn(Ctx, *const c_void, *mut c_void, i32, i32) -> c_int = "mrml_hip_repack_q4_0";
    repack_q8_0: fn(Ctx, *const c_void, *mut c_void, i32, i32) -> c_int = "mrml_hip_repack_q8_0";
    repack_q4_k: fn(Ctx, *const c_void, *mut c_void, i32, i32) -> c_int = "mrml_hip_repack_q4_k";
    quantize_q8_0: fn(Ctx, *const f32, *mut c_void, *mut c_void, i32) -> c_int = "mrml_hip_quantize_q8_0";
    q8_0_pack_bytes: fn(i32) -> usize = "mrml_hip_q8_0_pack_bytes";
    gemv_q4_0: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0";
    gemv_q4_0_q8: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_q8";
    gemv_q4_0_q8_relaxed: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_q8_relaxed";
    gemv_q4_0_gguf: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_gguf";
    gemv_q4_0_geglu: fn(Ctx, *const c_void, *const c_void, *const f32, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_geglu";
    ffn_geglu_q4_0: fn(Ctx, *const c_void, *const c_void, *const c_void, *const f32, *mut f32, *mut f32, i32, i32) -> c_int = "mrml_hip_ffn_geglu_q4_0";
    ffn_split_geglu: fn(Ctx, *const c_void, *const c_void, *const f32, *mut f32, *mut c_void, *const c_void, i32, i32) -> c_int = "mrml_hip_ffn_split_geglu";
    ffn_split_down: fn(Ctx, *const c_void, *const c_void, *const f32, *mut f32, i32, i32) -> c_int = "mrml_hip_ffn_split_down";
    gemv_q4_0_geglu_pack: fn(Ctx, *const c_void, *const c_void, *const f32, *mut f32, *mut c_void, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_geglu_pack";
    gemv_q4_0_geglu_q8: fn(Ctx, *const c_void, *const c_void, *const c_void, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_geglu_q8";
    gemv_q4_0_qkv: fn(Ctx, *const c_void, *const c_void, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_qkv";
    gemv_q4_0_qkv_q8: fn(Ctx, *const c_void, *const c_void, *const c_void, *const c_void, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemv_q4_0_qkv_q8";
    gemv_q8_0: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemv_q8_0";
    gemv_q8_0_q8: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemv_q8_0_q8";
    gemv_q4_k: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_k";
    gemv_q4_k_q8: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32) -> c_int = "mrml_hip_gemv_q4_k_q8";
    gemm_q4_0: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0";
    gemm_q4_0_q8: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_q8";
    gemm_pack_bytes: fn(i32, i32) -> usize = "mrml_hip_gemm_pack_bytes";
    quantize_q8_0_gemm: fn(Ctx, *const f32, *mut c_void, i32, i32) -> c_int = "mrml_hip_quantize_q8_0_gemm";
    gemm_q4_0_gpack: fn(Ctx, *const c_void, *const c_void, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_gpack";
    gemm_q4_0_qkv: fn(Ctx, *const c_void, *const c_void, *const c_void, *const f32, *mut f32, i32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_qkv";
    gemm_q4_0_geglu: fn(Ctx, *const c_void, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_geglu";
    gemm_q4_0_relaxed: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_relaxed";
    gemm_q4_0_noalloc: fn(Ctx, *const c_void, *const f32, *mut f32, i32, i32, i32) -> c_int = "mrml_hip_gemm_q4_0_noalloc";
    gemm_q4_0_noalloc_max_pack_bytes: fn() -> usize = "mrml_hip_gemm_q4_0_noalloc_max_pack_bytes";
    argmax_f32: fn(Ctx, *const f32, i32, *mut i32) -> c_int = "mrml_hip_argmax_f32";
    vocab_topk: fn(Ctx, *const f32, *const u8, *const i32, *mut f32, *mut i32, i32, i32, i32, i32, i32) -> c_int = "mrml_hip_vocab_topk";
    vocab_select: fn(Ctx, *const f32, i32, *const u8, *const i32, i32, i32, i32, f32, u64, i32, *mut i32, *mut f32, *mut i32) -> c_int = "mrml_hip_vocab_select";
    rms_norm: fn(Ctx, *const f32, *const f32, *mut f32, *mut c_void, i32, f32) -> c_int = "mrml_hip_rms_norm";
    rms_norm_batch: fn(Ctx, *const f32, *const f32, *mut f32, i32, i32, f32) -> c_int = "mrml_hip_rms_norm_batch";
    residual_rms_norm: fn(Ctx, *const f32, *const f32, *mut f32, *const f32, *mut f32, *mut c_void, i32, f32) -> c_int = "mrml_hip_residual_rms_norm";
    embedding: fn(Ctx, *const c_void, i32, i32, *const i32, *mut f32, i32, i32, f32) -> c_int = "mrml_hip_embedding";
    rope_table: fn(Ctx, *mut f32, i32, i32, f32, f32) -> c_int = "mrml_hip_rope_table";
    rope_kv_append_f16: fn(Ctx, *mut f32, *mut u16, *mut u16, i32, *const i32, i32, i32, i32, f32, f32, i32, *const f32, i32) -> c_int = "mrml_hip_rope_kv_append_f16";
    attn_decode_f16: fn(Ctx, *const f32, *const u16, *const u16, *mut f32, *mut c_void, i32, *const i32, i32, i32, i32, f32, i32) -> c_int = "mrml_hip_attn_decode_f16";
    attn_decode_f16_split: fn(Ctx, *const f32, *const u16, *const u16, *mut f32, *mut c_void, i32, *const i32, i32, i32, i32, f32, i32) -> c_int = "mrml_hip_attn_decode_f16_split";
    rope_kv_append_f16_batch: fn(Ctx, *mut f32, *mut u16, *mut u16, i32, i32, i32, i32, i32, i32, f32, f32, i32, i32, i32, *const f32, i32) -> c_int = "mrml_hip_rope_kv_append_f16_batch";
    rope: fn(Ctx, *mut f32, i32, i32, i32, f32, f32, *const f32, i32) -> c_int = "mrml_hip_rope";
    geglu: fn(Ctx, *const f32, *const f32, *mut f32, i32) -> c_int = "mrml_hip_geglu";
    swiglu: fn(Ctx, *const f32, *const f32, *mut f32, i32) -> c_int = "mrml_hip_swiglu";
    add: fn(Ctx, *const f32, *const f32, *mut f32, i32) -> c_int = "mrml_hip_add";
    attention_prefill: fn(Ctx, *const f32, i32, *const u16, *const u16, *mut f32, i32, i32, i32, i32, i32, f32, i32, i32, i32, i32) -> c_int = "mrml_hip_attention_prefill";
    attention_causal: fn(Ctx, *const f32, *const u16, *const u16, *mut f32, i32, i32, i32, i32, f32, i32, i32, i32, i32) -> c_int = "mrml_hip_attention_causal";
    attention_causal_split: fn(Ctx, *const f32, *const u16, *const u16, *mut f32, i32, i32, i32, i32, f32, i32, i32, i32, i32) -> c_int = "mrml_hip_attention_causal_split";
    gemma2_create: fn(Ctx, *const MrmlHipGemma2Config, *const c_void, *const f32, *const MrmlHipGemma2Layer, *mut Model) -> c_int = "mrml_hip_gemma2_create";
    gemma2_destroy: fn(Ctx, Model) -> c_int = "mrml_hip_gemma2_destroy";
    gemma2_step: fn(Ctx, Model, *mut i32, *mut u16, *mut u16, *mut f32, *mut i32, *mut i32, i32, *const i32, i32) -> c_int = "mrml_hip_gemma2_step";
    gemma2_prefill: fn(Ctx, Model, *const i32, i32, i32, *mut u16, *mut u16, *mut f32, *mut i32) -> c_int = "mrml_hip_gemma2_prefill";
    gemma2_set_sampler: fn(Ctx, Model, *const MrmlHipSampler) -> c_int = "mrml_hip_gemma2_set_sampler";
    gemma2_reserve_prefill: fn(Ctx, Model) -> c_int = "mrml_hip_gemma2_reserve_prefill";
    gemma2_activations: fn(Ctx, Model, *mut *mut f32, *mut *mut f32) -> c_int = "mrml_hip_gemma2_activations";
    gguf_open: fn(*const c_char, *mut Gguf) -> c_int = "mrml_gguf_open";
    gguf_close: fn(Gguf) -> c_int = "mrml_gguf_close";
    gguf_last_error: fn() -> *const c_char = "mrml_gguf_last_error";
    gguf_header: fn(Gguf, *mut u32, *mut u64, *mut i64, *mut i64) -> c_int = "mrml_gguf_header";
    gguf_tensor: fn(Gguf, i64, *mut MrmlGgufTensorInfo) -> c_int = "mrml_gguf_tensor";
    gguf_find_tensor: fn(Gguf, *const c_char, *mut i64) -> c_int = "mrml_gguf_find_tensor";
    gguf_read_tensor: fn(Gguf, i64, *mut c_void, u64) -> c_int = "mrml_gguf_read_tensor";
    gguf_meta_key: fn(Gguf, i64, *mut *const c_char, *mut i32) -> c_int = "mrml_gguf_meta_key";
    gguf_meta_u32: fn(Gguf, *const c_char, *mut u32) -> c_int = "mrml_gguf_meta_u32";
    gguf_meta_f32: fn(Gguf, *const c_char, *mut f32) -> c_int = "mrml_gguf_meta_f32";
    gguf_meta_str: fn(Gguf, *const c_char, *mut *const c_char, *mut u64) -> c_int = "mrml_gguf_meta_str";
    gguf_meta_array: fn(Gguf, *const c_char, *mut i32, *mut u64) -> c_int = "mrml_gguf_meta_array";
}

/// The library, opened once: `$MRML_HIP_LIB` if set, else `libmrml_hip.so`
/// from the loader path.
pub fn api() -> Result<&'static Api, String> {
    static API: OnceLock<Result<Api, String>> = OnceLock::new();
    API.get_or_init(|| unsafe {
        let path = std::env::var("MRML_HIP_LIB").unwrap_or_else(|_| "libmrml_hip.so".to_string());
        let c = CString::new(path.clone()).map_err(|e| e.to_string())?;
        let lib = dlopen(c.as_ptr(), RTLD_NOW);
        if lib.is_null() {
            let why = dlerror();
            let why = if why.is_null() { "unknown".into() } else { CStr::from_ptr(why).to_string_lossy().into_owned() };
            return Err(format!("cannot open {path}: {why}"));
        }
        Api::resolve(lib)
    })
    .as_ref()
    .map_err(|e| e.clone())
}
