//! src/compute/hip_backend.rs — the MI355X (gfx950) compute plane for Bramha.
//!
//! `HipComputePlane` is the counterpart of `WgpuComputePlane` (src/compute/wgpu_backend.rs:100-117):
//! a process-wide plane behind a `OnceLock` (`get_hip_plane`, like `get_wgpu_plane` at :1707-1728)
//! whose `matvec_mul*` methods keep the wgpu methods' signatures and `Result<Vec<f32>, String>`
//! contract (:734-741, :906-914, :1083-1091), so `matvec_mul` in cpu_engine.rs (:397-446) can try it
//! first and fall back to the CPU loop on `Err` exactly as it does for wgpu. `HipModel` wraps the
//! device decoder (`bh_model_*`) that replaces the per-op CPU calls and the host KV cache of
//! `generate_cpu_inner_logits` (cpu_engine.rs:2290-3064).
//!
//! Not compiled in this repository (no Rust toolchain in its build image); the declarations it
//! calls are checked against include/bramha_hip.h by tests/test_rust_binding.py.

use std::ffi::{CStr, CString};
use std::os::raw::{c_int, c_void};
use std::ptr;
use std::sync::{Mutex, OnceLock};

use bramha_hip_sys as sys;

fn cstr(s: Option<&str>) -> Result<Option<CString>, String> {
    s.map(|v| CString::new(v).map_err(|e| e.to_string())).transpose()
}

fn opt_ptr(s: &Option<CString>) -> *const std::os::raw::c_char {
    s.as_ref().map_or(ptr::null(), |c| c.as_ptr())
}

/// One context on one device: a stream and a registry of device-resident weights keyed
/// "model:layer" with LRU eviction under a byte cap (ModelBuffers, wgpu_backend.rs:25-82).
pub struct HipComputePlane {
    ctx: *mut sys::bh_ctx,
    // the reference guards its registry with a Mutex (wgpu_backend.rs:111); the context also
    // serialises internally, this lock keeps the error text paired with the failing call
    lock: Mutex<()>,
}

// The context is used only under `lock`; the library serialises calls on one context.
unsafe impl Send for HipComputePlane {}
unsafe impl Sync for HipComputePlane {}

impl HipComputePlane {
    /// Opens `device`; `Err` when it is not a gfx950 device (the caller stays on CPU).
    pub fn new(device: i32) -> Result<Self, String> {
        let mut ctx = ptr::null_mut();
        let st = unsafe { sys::bh_init(device as c_int, &mut ctx) };
        if st != sys::BH_OK {
            let msg = unsafe { CStr::from_ptr(sys::bh_status_str(st)) };
            return Err(msg.to_string_lossy().into_owned());
        }
        Ok(Self { ctx, lock: Mutex::new(()) })
    }

    fn last_error(&self) -> String {
        unsafe { CStr::from_ptr(sys::bh_last_error(self.ctx)) }.to_string_lossy().into_owned()
    }

    fn status(&self, st: c_int) -> Result<(), String> {
        if st == sys::BH_OK { Ok(()) } else { Err(self.last_error()) }
    }

    /// y = W h, W f32 [out_features][h.len()] (WgpuComputePlane::matvec_mul, :734-741).
    pub fn matvec_mul(&self, h: &[f32], weight: &[f32], out_features: usize, model_name: Option<&str>,
                      layer_name: Option<&str>) -> Result<Vec<f32>, String> {
        let (m, l) = (cstr(model_name)?, cstr(layer_name)?);
        let mut out = vec![0.0f32; out_features];
        let _g = self.lock.lock().unwrap();
        let st = unsafe {
            sys::bh_matvec_mul(self.ctx, h.as_ptr(), h.len(), weight.as_ptr(), weight.len(), out_features,
                               opt_ptr(&m), opt_ptr(&l), out.as_mut_ptr())
        };
        self.status(st).map(|_| out)
    }

    /// int8 per-row weights (WgpuComputePlane::matvec_mul_int8, :906-914).
    pub fn matvec_mul_int8(&self, h: &[f32], q_weight: &[i8], scales: &[f32], out_features: usize,
                           model_name: Option<&str>, layer_name: Option<&str>) -> Result<Vec<f32>, String> {
        let (m, l) = (cstr(model_name)?, cstr(layer_name)?);
        let mut out = vec![0.0f32; out_features];
        let _g = self.lock.lock().unwrap();
        let st = unsafe {
            sys::bh_matvec_mul_int8(self.ctx, h.as_ptr(), h.len(), q_weight.as_ptr(), q_weight.len(),
                                    scales.as_ptr(), scales.len(), out_features, opt_ptr(&m), opt_ptr(&l),
                                    out.as_mut_ptr())
        };
        self.status(st).map(|_| out)
    }

    /// packed 4-bit per-row weights, high nibble first (WgpuComputePlane::matvec_mul_int4, :1083-1091).
    pub fn matvec_mul_int4(&self, h: &[f32], q_weight: &[u8], scales: &[f32], out_features: usize,
                           model_name: Option<&str>, layer_name: Option<&str>) -> Result<Vec<f32>, String> {
        let (m, l) = (cstr(model_name)?, cstr(layer_name)?);
        let mut out = vec![0.0f32; out_features];
        let _g = self.lock.lock().unwrap();
        let st = unsafe {
            sys::bh_matvec_mul_int4(self.ctx, h.as_ptr(), h.len(), q_weight.as_ptr(), q_weight.len(),
                                    scales.as_ptr(), scales.len(), out_features, opt_ptr(&m), opt_ptr(&l),
                                    out.as_mut_ptr())
        };
        self.status(st).map(|_| out)
    }

    /// Drops every registry entry (WgpuComputePlane::clear_persistent_buffers, :724-731).
    pub fn clear_persistent_buffers(&self) {
        let _g = self.lock.lock().unwrap();
        unsafe { sys::bh_clear_persistent_buffers(self.ctx) };
    }

    /// The registry's byte cap (ModelBuffers::max_vram_bytes, :40-56).
    pub fn set_vram_cap(&self, bytes: usize) -> Result<(), String> {
        let _g = self.lock.lock().unwrap();
        let st = unsafe { sys::bh_set_vram_cap(self.ctx, bytes) };
        self.status(st)
    }

    /// A device decoder on this plane (see `HipModel`).
    pub fn model(&self, cfg: &sys::bh_model_config) -> Result<HipModel<'_>, String> {
        let mut m = ptr::null_mut();
        let _g = self.lock.lock().unwrap();
        let st = unsafe { sys::bh_model_create(self.ctx, cfg, &mut m) };
        self.status(st).map(|_| HipModel { plane: self, m, vocab: cfg.vocab as usize, batch: 0 })
    }
}

impl Drop for HipComputePlane {
    fn drop(&mut self) {
        unsafe { sys::bh_destroy(self.ctx) };
    }
}

/// Global plane, initialised on first use; `None` in CPU-only mode or without a gfx950 device,
/// after which the caller stays on its CPU path (get_wgpu_plane, wgpu_backend.rs:1707-1728).
pub static HIP_PLANE: OnceLock<Option<HipComputePlane>> = OnceLock::new();

pub fn get_hip_plane() -> Option<&'static HipComputePlane> {
    if crate::inference::is_cpu_only() {
        return None;
    }
    HIP_PLANE
        .get_or_init(|| match HipComputePlane::new(0) {
            Ok(p) => Some(p),
            Err(e) => {
                eprintln!("[HIP] compute plane unavailable: {}. Staying on the CPU path.", e);
                None
            }
        })
        .as_ref()
}

/// The dense Qwen2/Llama decoder on the device: weights uploaded once by their Hugging Face
/// names, a packed KV cache with one region per sequence slot, prefill, and graph-replayed greedy
/// decode steps over a (ragged) batch of slots.
pub struct HipModel<'p> {
    plane: &'p HipComputePlane,
    m: *mut sys::bh_model,
    vocab: usize,
    batch: usize,
}

impl<'p> HipModel<'p> {
    fn status(&self, st: c_int) -> Result<(), String> {
        self.plane.status(st)
    }

    /// One tensor by its Hugging Face name, in its reference layout (`scales` for the quantized
    /// formats: f32 per row, or fp16 bits per 32 weights).
    pub fn set_weight(&mut self, name: &str, data: &[u8], scales: Option<&[u8]>) -> Result<(), String> {
        let n = CString::new(name).map_err(|e| e.to_string())?;
        let (sp, sl) = scales.map_or((ptr::null(), 0), |s| (s.as_ptr() as *const c_void, s.len()));
        let st = unsafe {
            sys::bh_model_set_weight(self.m, n.as_ptr(), data.as_ptr() as *const c_void, data.len(), sp, sl)
        };
        self.status(st)
    }

    /// A model directory in the reference's on-disk format (manifest.json + shards).
    pub fn load_dir(&mut self, dir: &str) -> Result<usize, String> {
        let d = CString::new(dir).map_err(|e| e.to_string())?;
        let mut n: c_int = 0;
        let st = unsafe { sys::bh_model_load_dir(self.m, d.as_ptr(), &mut n) };
        self.status(st).map(|_| n as usize)
    }

    /// The reference's generate loop at temperature 0 for one sequence (prefill of all prompt
    /// tokens but the last, then greedy steps until max_new ids or an EOS id).
    pub fn generate(&mut self, slot: i32, prompt: &[u32], max_new: usize) -> Result<Vec<u32>, String> {
        let mut ids = vec![0u32; max_new.max(1)];
        let mut n: c_int = 0;
        let st = unsafe {
            sys::bh_model_generate(self.m, slot, prompt.as_ptr(), prompt.len() as c_int, max_new as c_int,
                                   ids.as_mut_ptr(), &mut n, ptr::null_mut())
        };
        self.status(st).map(|_| {
            ids.truncate(n as usize);
            ids
        })
    }

    pub fn seq_open(&mut self, slot: i32, capacity: i64) -> Result<(), String> {
        let st = unsafe { sys::bh_model_seq_open(self.m, slot, capacity) };
        self.status(st)
    }

    pub fn prefill(&mut self, slot: i32, tokens: &[u32]) -> Result<(), String> {
        let st = unsafe { sys::bh_model_prefill(self.m, slot, tokens.as_ptr(), tokens.len() as c_int) };
        self.status(st)
    }

    /// Several prompts in one pass: `prompts[i]` into `slots[i]` (a ragged batch refilling the
    /// entries that ended at the same step).
    pub fn prefill_batch(&mut self, slots: &[i32], prompts: &[&[u32]]) -> Result<(), String> {
        if slots.len() != prompts.len() {
            return Err("slots and prompts differ in length".into());
        }
        let counts: Vec<i32> = prompts.iter().map(|p| p.len() as i32).collect();
        let tokens: Vec<u32> = prompts.iter().flat_map(|p| p.iter().copied()).collect();
        let st = unsafe {
            sys::bh_model_prefill_batch(self.m, slots.len() as c_int, slots.as_ptr(), tokens.as_ptr(), counts.as_ptr())
        };
        self.status(st)
    }

    /// The decode batch: entry b decodes `slots[b]` starting from `first_tokens[b]`.
    pub fn decode_setup(&mut self, slots: &[i32], first_tokens: &[u32]) -> Result<(), String> {
        if slots.len() != first_tokens.len() {
            return Err("slots and first_tokens differ in length".into());
        }
        let st = unsafe {
            sys::bh_model_decode_setup(self.m, slots.len() as c_int, slots.as_ptr(), first_tokens.as_ptr())
        };
        self.status(st).map(|_| self.batch = slots.len())
    }

    /// Swap batch entry b for a new sequence (ragged refill).
    pub fn decode_replace(&mut self, b: usize, slot: i32, first_token: u32) -> Result<(), String> {
        let st = unsafe { sys::bh_model_decode_replace(self.m, b as c_int, slot, first_token) };
        self.status(st)
    }

    /// n_steps greedy steps of the batch: ids [n_steps][batch].
    pub fn decode(&mut self, n_steps: usize) -> Result<Vec<u32>, String> {
        let mut ids = vec![0u32; n_steps * self.batch];
        let st = unsafe { sys::bh_model_decode(self.m, n_steps as c_int, ids.as_mut_ptr(), ptr::null_mut()) };
        self.status(st).map(|_| ids)
    }

    /// Raw (pre-penalty) logits of each step as well: [n_steps][batch][vocab].
    pub fn decode_with_logits(&mut self, n_steps: usize) -> Result<(Vec<u32>, Vec<f32>), String> {
        let mut ids = vec![0u32; n_steps * self.batch];
        let mut lg = vec![0f32; n_steps * self.batch * self.vocab];
        let st = unsafe { sys::bh_model_decode(self.m, n_steps as c_int, ids.as_mut_ptr(), lg.as_mut_ptr()) };
        self.status(st).map(|_| (ids, lg))
    }

    /// KV rows of a slot as the prefix cache stores them: per layer [n][n_kv * head_dim] f32.
    pub fn kv_read(&mut self, slot: i32, row0: i64, n: i64, k: &mut [f32], v: &mut [f32]) -> Result<(), String> {
        let st = unsafe { sys::bh_model_kv_read(self.m, slot, row0, n, k.as_mut_ptr(), v.as_mut_ptr()) };
        self.status(st)
    }

    /// Write cached rows (a prefix-cache hit); the slot's length becomes row0 + n.
    pub fn kv_write(&mut self, slot: i32, row0: i64, n: i64, k: &[f32], v: &[f32]) -> Result<(), String> {
        let st = unsafe { sys::bh_model_kv_write(self.m, slot, row0, n, k.as_ptr(), v.as_ptr()) };
        self.status(st)
    }

    /// temperature 0: greedy (default); > 0: the reference's top-k sampling on the device.
    pub fn set_sampling(&mut self, temperature: f32, top_k: i32, seed: u64) -> Result<(), String> {
        let st = unsafe { sys::bh_model_set_sampling(self.m, temperature, top_k, seed) };
        self.status(st)
    }
}

impl Drop for HipModel<'_> {
    fn drop(&mut self) {
        unsafe { sys::bh_model_destroy(self.m) };
    }
}
