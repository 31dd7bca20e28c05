//! The Gemma-2-shape token step and prefill (`forward_token` +
//! `step_generation`, model.rs:1185-2260, 2713-2930; `prefill_cuda`,
//! model.rs:2395-2638) as device-resident calls.

use std::ffi::c_void;
use std::sync::Arc;

use crate::device::{HipBuffer, HipDevice, Inner};
use crate::ffi::{self, Model};
use crate::Result;

/// The step's numerics: `Exact` keeps every op in the CPU path's order
/// (logits bit-identical); `Fast` uses tree-order norm sums and split-K
/// attention (within 1e-5 of the CPU path per op).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Numerics {
    Exact,
    Fast,
}

/// `mrml_hip_gemma2_config`.
#[derive(Clone, Copy, Debug)]
pub struct Gemma2Config {
    pub n_layers: usize,
    pub dim: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub head_dim: usize,
    pub ffn_dim: usize,
    pub vocab: usize,
    pub ctx_len: usize,
    pub rope_base: f32,
    pub eps: f32,
    pub attn_scale: f32,
    /// GGUF type of the tied embedding / LM-head table: `ffi::MRML_HIP_Q4_0` or `_Q8_0`.
    pub tie_type: i32,
    pub numerics: Numerics,
    /// Per-layer windows (model.rs:590, 1465-1467): with both > 0, layer l
    /// attends the last `sliding_window` positions unless
    /// `l % swa_period == swa_period - 1`.  0 and 0: every layer global.
    pub sliding_window: usize,
    pub swa_period: usize,
}

/// One layer's weights: matrices uploaded with `HipDevice::upload_q4_0`,
/// norm weights f32[dim].
pub struct Gemma2Layer<'a> {
    pub wq: &'a HipBuffer<u8>,
    pub wk: &'a HipBuffer<u8>,
    pub wv: &'a HipBuffer<u8>,
    pub wo: &'a HipBuffer<u8>,
    pub w_gate: &'a HipBuffer<u8>,
    pub w_up: &'a HipBuffer<u8>,
    pub w_down: &'a HipBuffer<u8>,
    pub attn_norm: &'a HipBuffer<f32>,
    pub post_attn_norm: &'a HipBuffer<f32>,
    pub ffn_norm: &'a HipBuffer<f32>,
    pub post_ffw_norm: &'a HipBuffer<f32>,
}

/// The pick of the step: the reference's scoring (valid mask, early ids,
/// 30*tanh softcap, -3.5 for the last 32 tokens) and its draw over the
/// `top_k` best at `temperature` (greedy when <= 0).
pub struct Sampler<'a> {
    pub valid: Option<&'a HipBuffer<u8>>,
    pub temperature: f32,
    pub top_k: usize,
}

/// A model bound to device weights.  The weights are not copied: they must
/// outlive the model (the borrow in `create` is the caller's promise).
pub struct Gemma2Model {
    inner: Arc<Inner>,
    handle: Model,
    cfg: Gemma2Config,
}

unsafe impl Send for Gemma2Model {}

impl Gemma2Model {
    pub fn create(device: &HipDevice, cfg: &Gemma2Config, tok_embd: &HipBuffer<u8>, output_norm: &HipBuffer<f32>,
                  layers: &[Gemma2Layer<'_>]) -> Result<Self> {
        assert_eq!(layers.len(), cfg.n_layers, "one Gemma2Layer per layer");
        let c = ffi::MrmlHipGemma2Config {
            n_layers: cfg.n_layers as i32,
            dim: cfg.dim as i32,
            n_heads: cfg.n_heads as i32,
            n_kv_heads: cfg.n_kv_heads as i32,
            head_dim: cfg.head_dim as i32,
            ffn_dim: cfg.ffn_dim as i32,
            vocab: cfg.vocab as i32,
            ctx_len: cfg.ctx_len as i32,
            rope_base: cfg.rope_base,
            eps: cfg.eps,
            attn_scale: cfg.attn_scale,
            tie_type: cfg.tie_type,
            numerics: match cfg.numerics {
                Numerics::Exact => ffi::MRML_HIP_NUMERICS_EXACT,
                Numerics::Fast => ffi::MRML_HIP_NUMERICS_FAST,
            },
            sliding_window: cfg.sliding_window as i32,
            swa_period: cfg.swa_period as i32,
        };
        let ls: Vec<ffi::MrmlHipGemma2Layer> = layers
            .iter()
            .map(|l| ffi::MrmlHipGemma2Layer {
                wq: l.wq.as_ptr() as *const c_void,
                wk: l.wk.as_ptr() as *const c_void,
                wv: l.wv.as_ptr() as *const c_void,
                wo: l.wo.as_ptr() as *const c_void,
                w_gate: l.w_gate.as_ptr() as *const c_void,
                w_up: l.w_up.as_ptr() as *const c_void,
                w_down: l.w_down.as_ptr() as *const c_void,
                attn_norm: l.attn_norm.as_ptr(),
                post_attn_norm: l.post_attn_norm.as_ptr(),
                ffn_norm: l.ffn_norm.as_ptr(),
                post_ffw_norm: l.post_ffw_norm.as_ptr(),
            })
            .collect();
        let inner = device.inner.clone();
        let mut handle: Model = std::ptr::null_mut();
        inner.check(unsafe {
            (inner.api.gemma2_create)(inner.ctx, &c, tok_embd.as_ptr() as *const c_void, output_norm.as_ptr(), ls.as_ptr(),
                                      &mut handle)
        })?;
        Ok(Self { inner, handle, cfg: *cfg })
    }

    pub fn config(&self) -> &Gemma2Config {
        &self.cfg
    }

    /// f16 elements of one KV cache: [n_layers][ctx_len][n_kv_heads][head_dim].
    pub fn cache_elems(&self) -> usize {
        self.cfg.n_layers * self.cfg.ctx_len * self.cfg.n_kv_heads * self.cfg.head_dim
    }

    /// Enqueue one token step (`mrml_hip_gemma2_step`).  `state` = {token, pos}
    /// on the device is read when the step runs and advanced by it: the pick
    /// goes to `pick` and `hist[pos]`, and the next token is `prompt[pos+1]`
    /// while the prompt lasts, else the pick.  One captured graph of this call
    /// replays for every token.
    #[allow(clippy::too_many_arguments)]
    pub fn step(&self, state: &mut HipBuffer<i32>, k_cache: &mut HipBuffer<u16>, v_cache: &mut HipBuffer<u16>,
                logits: Option<&mut HipBuffer<f32>>, pick: Option<&mut HipBuffer<i32>>, hist: Option<&mut HipBuffer<i32>>,
                prompt: Option<&HipBuffer<i32>>) {
        let (hist_p, hist_cap) = hist.map_or((std::ptr::null_mut(), 0), |h| (h.as_mut_ptr(), h.len() as i32));
        let (prompt_p, prompt_len) = prompt.map_or((std::ptr::null(), 0), |p| (p.as_ptr(), p.len() as i32));
        let st = unsafe {
            (self.inner.api.gemma2_step)(self.inner.ctx, self.handle, state.as_mut_ptr(), k_cache.as_mut_ptr(),
                                         v_cache.as_mut_ptr(), logits.map_or(std::ptr::null_mut(), |l| l.as_mut_ptr()),
                                         pick.map_or(std::ptr::null_mut(), |p| p.as_mut_ptr()), hist_p, hist_cap, prompt_p,
                                         prompt_len)
        };
        self.inner.expect(st, "gemma2_step");
    }

    /// `prefill_cuda` (model.rs:2395-2638): the steps of positions
    /// pos0..pos0+n for `tokens`, through the batched products; the caches
    /// end bit-identical to n token steps.  `pick` receives the first
    /// generated token.
    pub fn prefill(&self, tokens: &HipBuffer<i32>, pos0: usize, k_cache: &mut HipBuffer<u16>, v_cache: &mut HipBuffer<u16>,
                   logits: Option<&mut HipBuffer<f32>>, pick: Option<&mut HipBuffer<i32>>) -> Result<()> {
        self.inner.check(unsafe {
            (self.inner.api.gemma2_prefill)(self.inner.ctx, self.handle, tokens.as_ptr(), tokens.len() as i32, pos0 as i32,
                                            k_cache.as_mut_ptr(), v_cache.as_mut_ptr(),
                                            logits.map_or(std::ptr::null_mut(), |l| l.as_mut_ptr()),
                                            pick.map_or(std::ptr::null_mut(), |p| p.as_mut_ptr()))
        })
    }

    /// Allocate the prefill's chunk buffers now, so that a later `prefill`
    /// can be captured into a graph.
    pub fn reserve_prefill(&self) -> Result<()> {
        self.inner.check(unsafe { (self.inner.api.gemma2_reserve_prefill)(self.inner.ctx, self.handle) })
    }

    /// The pick of later steps and prefills: `None` for the plain argmax.
    pub fn set_sampler(&self, sampler: Option<&Sampler<'_>>) -> Result<()> {
        let s = sampler.map(|s| ffi::MrmlHipSampler {
            d_valid: s.valid.map_or(std::ptr::null(), |v| v.as_ptr()),
            temperature: s.temperature,
            top_k: s.top_k as i32,
        });
        let p = s.as_ref().map_or(std::ptr::null(), |s| s as *const ffi::MrmlHipSampler);
        self.inner.check(unsafe { (self.inner.api.gemma2_set_sampler)(self.inner.ctx, self.handle, p) })
    }
}

impl Drop for Gemma2Model {
    fn drop(&mut self) {
        unsafe { (self.inner.api.gemma2_destroy)(self.inner.ctx, self.handle) };
    }
}
