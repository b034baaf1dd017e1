//! Raw FFI declarations of the MI355X (gfx950) backend: one `extern "C"` item per function of
//! `include/bramha_hip.h`, argument for argument. Safe wrappers live in the backend module
//! (`src/compute/hip_backend.rs`). Every function returns a `bh_status` (0 = `BH_OK`); the text of
//! a failure is `bh_last_error(ctx)`.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

#[repr(C)]
pub struct bh_ctx {
    _private: [u8; 0],
}
#[repr(C)]
pub struct bh_weight {
    _private: [u8; 0],
}
#[repr(C)]
pub struct bh_model {
    _private: [u8; 0],
}

/// The decoder configuration (`bh_model_config`, field for field).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct bh_model_config {
    pub n_layers: i32,
    pub hidden: i32,
    pub n_heads: i32,
    pub n_kv_heads: i32,
    pub head_dim: i32,
    pub ffn: i32,
    pub vocab: i32,
    pub rope_theta: f32,
    pub rms_eps: f32,
    pub attn_bias: i32,
    pub o_bias: i32,
    pub wfmt: i32,
    pub head_fmt: i32,
    pub max_context: i32,
    pub sink_tokens: i32,
    pub kv_f16: i32,
    pub max_seqs: i32,
    pub kv_rows: i64,
    pub max_tokens: i32,
}

// bh_status
pub const BH_OK: c_int = 0;
pub const BH_ERR_INVALID: c_int = -1;
pub const BH_ERR_NO_DEVICE: c_int = -2;
pub const BH_ERR_HIP: c_int = -3;
pub const BH_ERR_OOM: c_int = -4;
pub const BH_ERR_NOT_FOUND: c_int = -5;
pub const BH_ERR_INJECTED: c_int = -6;
pub const BH_ERR_UNSUPPORTED: c_int = -7;
pub const BH_ERR_CAPACITY: c_int = -8;

// bh_qfmt
pub const BH_F32: c_int = 0;
pub const BH_Q8_ROW: c_int = 1;
pub const BH_Q4_ROW: c_int = 2;
pub const BH_Q4_G32: c_int = 3;

// op ids of bh_debug_inject_fault
pub const BH_OP_ANY: c_int = 0;
pub const BH_OP_MATVEC: c_int = 1;
pub const BH_OP_UPLOAD: c_int = 2;
pub const BH_OP_GEMV: c_int = 3;
pub const BH_OP_DECODE: c_int = 4;

// kernel classes of bh_model_time_kernels / bh_model_kernel_bytes
pub const BH_K_GEMV_QKV: c_int = 0;
pub const BH_K_ATTN: c_int = 1;
pub const BH_K_GEMV_O: c_int = 2;
pub const BH_K_GEMV_GATEUP: c_int = 3;
pub const BH_K_GEMV_DOWN: c_int = 4;
pub const BH_K_LM_HEAD: c_int = 5;
pub const BH_K_NORM: c_int = 6;
pub const BH_K_OTHER: c_int = 7;
pub const BH_K_ATTN_O: c_int = 8;
pub const BH_K_COUNT: usize = 9;

#[link(name = "bramha_hip")]
extern "C" {
    // ---- context (bh_init replaces WgpuComputePlane::new behind get_wgpu_plane's OnceLock, wgpu_backend.rs:1707-1728)
    pub fn bh_init(device: c_int, out: *mut *mut bh_ctx) -> c_int;
    pub fn bh_destroy(ctx: *mut bh_ctx);
    pub fn bh_last_error(ctx: *const bh_ctx) -> *const c_char;
    pub fn bh_status_str(status: c_int) -> *const c_char;
    pub fn bh_set_vram_cap(ctx: *mut bh_ctx, bytes: usize) -> c_int;
    pub fn bh_registry_stats(ctx: *mut bh_ctx, n_entries: *mut usize, bytes: *mut usize) -> c_int;
    pub fn bh_debug_inject_fault(ctx: *mut bh_ctx, op: c_int, status: c_int, count: c_int) -> c_int;
    // ---- device memory
    pub fn bh_dev_alloc(ctx: *mut bh_ctx, bytes: usize, out: *mut *mut c_void) -> c_int;
    pub fn bh_dev_free(ctx: *mut bh_ctx, p: *mut c_void) -> c_int;
    pub fn bh_memcpy_h2d(ctx: *mut bh_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn bh_memcpy_d2h(ctx: *mut bh_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> c_int;
    pub fn bh_synchronize(ctx: *mut bh_ctx) -> c_int;
    // ---- the WgpuComputePlane GEMV mirrors (wgpu_backend.rs:724-1104): host slices in, host vector out
    pub fn bh_matvec_mul(ctx: *mut bh_ctx, h: *const f32, in_features: usize, weight: *const f32, weight_len: usize,
        out_features: usize, model_name: *const c_char, layer_name: *const c_char, out: *mut f32) -> c_int;
    pub fn bh_matvec_mul_int8(ctx: *mut bh_ctx, h: *const f32, in_features: usize, q_weight: *const i8, q_len: usize,
        scales: *const f32, s_len: usize, out_features: usize, model_name: *const c_char, layer_name: *const c_char,
        out: *mut f32) -> c_int;
    pub fn bh_matvec_mul_int4(ctx: *mut bh_ctx, h: *const f32, in_features: usize, q_weight: *const u8, q_len: usize,
        scales: *const f32, s_len: usize, out_features: usize, model_name: *const c_char, layer_name: *const c_char,
        out: *mut f32) -> c_int;
    pub fn bh_clear_persistent_buffers(ctx: *mut bh_ctx) -> c_int;
    // ---- device-resident weights and single ops (device pointers, stream-ordered)
    pub fn bh_weight_upload(ctx: *mut bh_ctx, fmt: c_int, n_out: i64, k_in: i64, q: *const c_void, q_bytes: usize,
        scales: *const c_void, s_bytes: usize, out: *mut *mut bh_weight) -> c_int;
    pub fn bh_weight_free(ctx: *mut bh_ctx, w: *mut bh_weight);
    pub fn bh_gemv(ctx: *mut bh_ctx, w: *const bh_weight, x: *const f32, y: *mut f32, batch: c_int,
        stream: *mut c_void) -> c_int;
    pub fn bh_dequant(ctx: *mut bh_ctx, w: *const bh_weight, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn bh_rmsnorm(ctx: *mut bh_ctx, x: *const f32, w: *const f32, eps: f32, out: *mut f32, rows: c_int, n: c_int,
        stream: *mut c_void) -> c_int;
    pub fn bh_rope(ctx: *mut bh_ctx, v: *mut f32, pos: *const i32, rows: c_int, n_heads: c_int, head_dim: c_int,
        theta: f32, max_pos: c_int, stream: *mut c_void) -> c_int;
    pub fn bh_silu_mul(ctx: *mut bh_ctx, g: *const f32, u: *const f32, out: *mut f32, n: i64,
        stream: *mut c_void) -> c_int;
    pub fn bh_attn_decode(ctx: *mut bh_ctx, q: *const f32, k: *const c_void, v: *const c_void, kv_f16: c_int,
        kv_rows: i64, seq_off: *const i64, seq_len: *const i32, batch: c_int, n_q: c_int, n_kv: c_int,
        head_dim: c_int, max_len: c_int, out: *mut f32, stream: *mut c_void) -> c_int;
    pub fn bh_attn_decode_noalloc(ctx: *mut bh_ctx, q: *const f32, k: *const c_void, v: *const c_void, kv_f16: c_int,
        kv_rows: i64, seq_off: *const i64, seq_len: *const i32, batch: c_int, n_q: c_int, n_kv: c_int,
        head_dim: c_int, max_len: c_int, out: *mut f32, stream: *mut c_void) -> c_int;
    // ---- measurement helpers
    pub fn bh_time_gemv(ctx: *mut bh_ctx, w: *const bh_weight, x: *const f32, y: *mut f32, batch: c_int,
        iters: c_int, rotate_bytes: usize, us_per_launch: *mut f64) -> c_int;
    pub fn bh_time_attn(ctx: *mut bh_ctx, q: *const f32, k: *const c_void, v: *const c_void, kv_f16: c_int,
        kv_rows: i64, seq_off: *const i64, seq_len: *const i32, batch: c_int, n_q: c_int, n_kv: c_int,
        head_dim: c_int, max_len: c_int, out: *mut f32, iters: c_int, rotate_bytes: usize,
        us_per_launch: *mut f64) -> c_int;
    pub fn bh_time_probe(ctx: *mut bh_ctx, copy: c_int, bytes: usize, wgs: c_int, unroll: c_int, iters: c_int,
        us_per_launch: *mut f64) -> c_int;
    // ---- the device decoder (generate_cpu_inner_logits, cpu_engine.rs:2290-3064)
    pub fn bh_model_create(ctx: *mut bh_ctx, cfg: *const bh_model_config, out: *mut *mut bh_model) -> c_int;
    pub fn bh_model_destroy(m: *mut bh_model);
    pub fn bh_model_set_weight(m: *mut bh_model, name: *const c_char, data: *const c_void, bytes: usize,
        scales: *const c_void, scale_bytes: usize) -> c_int;
    pub fn bh_model_load_dir(m: *mut bh_model, dir: *const c_char, n_loaded: *mut c_int) -> c_int;
    pub fn bh_model_kv_read(m: *mut bh_model, slot: c_int, row0: i64, n: i64, k_out: *mut f32,
        v_out: *mut f32) -> c_int;
    pub fn bh_model_kv_write(m: *mut bh_model, slot: c_int, row0: i64, n: i64, k_in: *const f32,
        v_in: *const f32) -> c_int;
    pub fn bh_model_seq_len(m: *mut bh_model, slot: c_int, len: *mut i64) -> c_int;
    pub fn bh_model_set_sampling(m: *mut bh_model, temperature: f32, top_k: c_int, seed: u64) -> c_int;
    pub fn bh_sample_uniform(seed: u64, slot: c_int, pos: c_int) -> f32;
    pub fn bh_model_missing(m: *mut bh_model, n_missing: *mut c_int) -> c_int;
    pub fn bh_model_seq_open(m: *mut bh_model, slot: c_int, capacity: i64) -> c_int;
    pub fn bh_model_prefill(m: *mut bh_model, slot: c_int, tokens: *const u32, n: c_int) -> c_int;
    pub fn bh_model_prefill_batch(m: *mut bh_model, n_seqs: c_int, slots: *const i32, tokens: *const u32,
        counts: *const i32) -> c_int;
    pub fn bh_model_decode_setup(m: *mut bh_model, batch: c_int, slots: *const i32,
        first_tokens: *const u32) -> c_int;
    pub fn bh_model_decode_replace(m: *mut bh_model, b: c_int, slot: c_int, first_token: u32) -> c_int;
    pub fn bh_model_decode(m: *mut bh_model, n_steps: c_int, ids_out: *mut u32, raw_logits: *mut f32) -> c_int;
    pub fn bh_model_generate(m: *mut bh_model, slot: c_int, prompt: *const u32, n_prompt: c_int, max_new: c_int,
        ids_out: *mut u32, n_out: *mut c_int, raw_logits: *mut f32) -> c_int;
    pub fn bh_model_stream(m: *mut bh_model) -> *mut c_void;
    pub fn bh_model_time_kernels(m: *mut bh_model, n_steps: c_int, mean_us: *mut f64, launches: *mut i64) -> c_int;
    pub fn bh_model_kernel_bytes(m: *mut bh_model, kclass: c_int, bytes: *mut f64) -> c_int;
    // ---- host utilities (no device)
    pub fn bh_synth_normal(seed: u64, name: *const c_char, sigma: f32, n: i64, out: *mut f32) -> c_int;
    pub fn bh_synth_tokens(seed: u64, name: *const c_char, n: i64, vocab: u32, out: *mut u32) -> c_int;
    pub fn bh_quantize(fmt: c_int, w: *const f32, n: i64, k: i64, q: *mut c_void, scales: *mut c_void) -> c_int;
}
