//! Raw declarations of libcpb_moe's C ABI (include/cpb_moe.h, include/cpb_gguf.h,
//! include/cpb_head.h, include/cpb_attn.h).
//!
//! The MoE block of cpubrrr's engines (src/bin/engine_gpt2.rs:845-923,
//! src/bin/engine_qwen2.rs:395-433) becomes `cpb_moe_forward` (host x) or
//! `cpb_moe_forward_device` (device x); the expert-tensor part of the model
//! load (engine_gpt2.rs:1276-1324) becomes `cpb_gguf_open` +
//! `cpb_moe_load_gguf_layer`.  Every function returns 0 or a negative
//! `CPB_E*` code with the message in `cpb_moe_last_error()`.  Layouts mirror
//! the C structs field for field (`#[repr(C)]`).
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_long, c_void};

pub const CPB_OK: c_int = 0;
pub const CPB_EINVAL: c_int = -22;
pub const CPB_ENOMEM: c_int = -12;
pub const CPB_ENODEV: c_int = -19;
pub const CPB_ESTATE: c_int = -71;

pub const CPB_ROUTER_TOPK_SOFTMAX: c_int = 0;
pub const CPB_ROUTER_SOFTMAX_TOPK: c_int = 1;
pub const CPB_ACT_SWIGLU_OAI: c_int = 0;
pub const CPB_ACT_SILU: c_int = 1;
pub const CPB_NORM_GPTOSS: c_int = 0;
pub const CPB_NORM_QWEN: c_int = 1;
pub const CPB_GGUF_MXFP4: c_int = 39;
pub const CPB_GGUF_Q4_K: c_int = 12;
pub const CPB_GGUF_Q6_K: c_int = 14;

pub const CPB_GGML_F32: c_int = 0;
pub const CPB_GGML_F16: c_int = 1;
pub const CPB_GGML_Q8_0: c_int = 8;
pub const CPB_GGML_Q4_K: c_int = 12;
pub const CPB_GGML_Q6_K: c_int = 14;
pub const CPB_GGML_BF16: c_int = 30;
pub const CPB_GGML_MXFP4: c_int = 39;

/// Model shape and semantics (config.txt keys of engine_gpt2.rs:64-80).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cpb_moe_cfg {
    pub d: c_int,
    pub n_expert: c_int,
    pub top_k: c_int,
    pub d_ff: c_int,
    pub n_layer: c_int,
    pub router: c_int,
    pub act: c_int,
    pub norm: c_int,
    pub norm_nt: c_int,
    pub alpha: f32,
    pub limit: f32,
    pub rms_eps: f32,
    pub wtype_gate_up: c_int,
    pub wtype_down: c_int,
    pub has_bias: c_int,
    pub max_tokens: c_int,
}

/// Opaque handle: one device, one stream, n_layer MoE layers.
#[repr(C)]
pub struct cpb_moe_t {
    _private: [u8; 0],
}

/// Optional per-layer intermediates (host buffers, any may be null).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cpb_moe_trace {
    pub xn: *mut f32,
    pub xq: *mut i8,
    pub xsb: *mut f32,
    pub xsum: *mut i32,
    pub logits: *mut f32,
    pub ids: *mut i32,
    pub wts: *mut f32,
    pub gu: *mut f32,
    pub gu_sums: *mut i32,
    pub h: *mut f32,
    pub hq: *mut i8,
    pub hsb: *mut f32,
    pub hsum: *mut i32,
    pub dn: *mut f32,
    pub dn_sums: *mut i32,
    pub exact_router_fallbacks: i32,
}

/// Opaque mapped GGUF file.
#[repr(C)]
pub struct cpb_gguf_t {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cpb_gguf_tensor {
    pub name: *const c_char,
    pub type_: i32,
    pub n_dims: i32,
    pub dims: [u64; 4],
    pub n_elements: u64,
    pub offset: u64,
    pub n_bytes: u64,
    pub data: *const c_void,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cpb_gguf_hparams {
    pub arch: [c_char; 32],
    pub n_embd: i64,
    pub n_layer: i64,
    pub n_head: i64,
    pub n_head_kv: i64,
    pub head_dim: i64,
    pub n_expert: i64,
    pub n_expert_used: i64,
    pub n_ff_exp: i64,
    pub sliding_window: i64,
    pub n_vocab: i64,
    pub context_length: i64,
    pub rope_freq_base: f64,
    pub rms_eps: f64,
}

/// Two-stage LM head configuration (include/cpb_head.h).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cpb_head_cfg {
    pub d: c_int,
    pub n_vocab: c_int,
    pub n_slices: c_int,
    pub n_cand: c_int,
    pub rms_eps: f32,
}

/// Opaque head handle.
#[repr(C)]
pub struct cpb_head_t {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cpb_head_trace {
    pub cand_ids: *mut i32,
    pub cand_screen: *mut f32,
    pub cand_logits: *mut f32,
    pub xq: *mut i8,
    pub xsb: *mut f32,
    pub screen: *mut f32,
}

/// Attention block configuration (include/cpb_attn.h).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct cpb_attn_cfg {
    pub d: c_int,
    pub n_head: c_int,
    pub n_head_kv: c_int,
    pub head_dim: c_int,
    pub n_layer: c_int,
    pub max_seq: c_int,
    pub sliding_window: c_int,
    pub rope_base: f32,
    pub rms_eps: f32,
}

/// Opaque attention handle.
#[repr(C)]
pub struct cpb_attn_t {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct cpb_attn_trace {
    pub xq: *mut i8,
    pub xsb: *mut f32,
    pub q: *mut f32,
    pub k: *mut f32,
    pub v: *mut f32,
    pub ao: *mut f32,
    pub aq: *mut i8,
    pub asb: *mut f32,
}

#[link(name = "cpb_moe")]
extern "C" {
    // ---- include/cpb_moe.h ----
    pub fn cpb_moe_create(cfg: *const cpb_moe_cfg, device: c_int, out: *mut *mut cpb_moe_t) -> c_int;
    pub fn cpb_moe_load_layer(h: *mut cpb_moe_t, layer: c_int, gate: *const c_void, up: *const c_void,
                              down: *const c_void, gate_b: *const f32, up_b: *const f32, down_b: *const f32,
                              router_w: *const f32, router_b: *const f32, norm_w: *const f32) -> c_int;
    pub fn cpb_moe_load_layer_typed(h: *mut cpb_moe_t, layer: c_int, gate_type: c_int, up_type: c_int,
                                    down_type: c_int, gate: *const c_void, up: *const c_void, down: *const c_void,
                                    gate_b: *const f32, up_b: *const f32, down_b: *const f32,
                                    router_w: *const f32, router_b: *const f32, norm_w: *const f32) -> c_int;
    pub fn cpb_moe_forward(h: *mut cpb_moe_t, layer: c_int, x: *mut f32, n_tok: c_int, apply_norm: c_int,
                           trace: *mut cpb_moe_trace) -> c_int;
    pub fn cpb_moe_forward_device(h: *mut cpb_moe_t, layer0: c_int, n_layers: c_int, d_x: *mut f32, n_tok: c_int,
                                  apply_norm: c_int) -> c_int;
    pub fn cpb_moe_forward_device_noalloc(h: *mut cpb_moe_t, layer0: c_int, n_layers: c_int, d_x: *mut f32,
                                          n_tok: c_int, apply_norm: c_int) -> c_int;
    pub fn cpb_moe_set_stream(h: *mut cpb_moe_t, stream: *mut c_void) -> c_int;
    pub fn cpb_moe_sync(h: *mut cpb_moe_t) -> c_int;
    pub fn cpb_moe_destroy(h: *mut cpb_moe_t);
    pub fn cpb_moe_last_error() -> *const c_char;
    pub fn cpb_moe_config(h: *const cpb_moe_t, out: *mut cpb_moe_cfg) -> c_int;
    pub fn cpb_moe_layer_bytes(cfg: *const cpb_moe_cfg, out: *mut usize) -> c_int;
    pub fn cpb_moe_timing(h: *mut cpb_moe_t, enable: c_int) -> c_int;
    pub fn cpb_moe_kernel_times(h: *mut cpb_moe_t, ms: *mut f64, n: *mut c_long) -> c_int;
    pub fn cpb_moe_grouped_sums(h: *mut cpb_moe_t, layer: c_int, x: *mut f32, n_tok: c_int, apply_norm: c_int,
                                gu_sums: *mut i32, dn_sums: *mut i32) -> c_int;

    // ---- include/cpb_gguf.h ----
    pub fn cpb_gguf_open(path: *const c_char, out: *mut *mut cpb_gguf_t) -> c_int;
    pub fn cpb_gguf_close(g: *mut cpb_gguf_t);
    pub fn cpb_gguf_version(g: *const cpb_gguf_t, version: *mut u32, data_start: *mut u64,
                            alignment: *mut u64) -> c_int;
    pub fn cpb_gguf_n_tensors(g: *const cpb_gguf_t, n: *mut i64) -> c_int;
    pub fn cpb_gguf_tensor_at(g: *const cpb_gguf_t, i: i64, out: *mut cpb_gguf_tensor) -> c_int;
    pub fn cpb_gguf_find(g: *const cpb_gguf_t, name: *const c_char, out: *mut cpb_gguf_tensor) -> c_int;
    pub fn cpb_gguf_meta_i64(g: *const cpb_gguf_t, key: *const c_char, out: *mut i64) -> c_int;
    pub fn cpb_gguf_meta_f64(g: *const cpb_gguf_t, key: *const c_char, out: *mut f64) -> c_int;
    pub fn cpb_gguf_meta_str(g: *const cpb_gguf_t, key: *const c_char, out: *mut *const c_char) -> c_int;
    pub fn cpb_gguf_hparams_get(g: *const cpb_gguf_t, out: *mut cpb_gguf_hparams) -> c_int;
    pub fn cpb_gguf_write_manifest(g: *const cpb_gguf_t, path: *const c_char) -> c_int;
    pub fn cpb_moe_load_gguf_layer(h: *mut cpb_moe_t, g: *const cpb_gguf_t, layer: c_int) -> c_int;

    // ---- include/cpb_head.h ----
    pub fn cpb_head_create(cfg: *const cpb_head_cfg, device: c_int, out: *mut *mut cpb_head_t) -> c_int;
    pub fn cpb_head_load(h: *mut cpb_head_t, out_w: *const u16, out_norm: *const f32) -> c_int;
    pub fn cpb_head_forward(h: *mut cpb_head_t, x: *const f32, chosen: *mut i32, trace: *mut cpb_head_trace) -> c_int;
    pub fn cpb_head_forward_device(h: *mut cpb_head_t, d_x: *const f32, d_chosen: *mut i32) -> c_int;
    pub fn cpb_head_set_screen(h: *mut cpb_head_t, bits: c_int) -> c_int;
    pub fn cpb_head_set_stream(h: *mut cpb_head_t, stream: *mut c_void) -> c_int;
    pub fn cpb_head_sync(h: *mut cpb_head_t) -> c_int;
    pub fn cpb_head_destroy(h: *mut cpb_head_t);
    pub fn cpb_head_bytes(cfg: *const cpb_head_cfg, out: *mut usize) -> c_int;

    // ---- include/cpb_attn.h ----
    pub fn cpb_attn_create(cfg: *const cpb_attn_cfg, device: c_int, out: *mut *mut cpb_attn_t) -> c_int;
    pub fn cpb_attn_load_layer(h: *mut cpb_attn_t, layer: c_int, attn_norm: *const f32, wq: *const u16,
                               wk: *const u16, wv: *const u16, wo: *const u16, bq: *const f32, bk: *const f32,
                               bv: *const f32, bo: *const f32, sinks: *const f32) -> c_int;
    pub fn cpb_attn_forward(h: *mut cpb_attn_t, layer: c_int, pos: c_int, x: *mut f32,
                            trace: *mut cpb_attn_trace) -> c_int;
    pub fn cpb_attn_forward_device(h: *mut cpb_attn_t, layer: c_int, pos: c_int, d_x: *mut f32) -> c_int;
    pub fn cpb_attn_reset(h: *mut cpb_attn_t) -> c_int;
    pub fn cpb_attn_set_stream(h: *mut cpb_attn_t, stream: *mut c_void) -> c_int;
    pub fn cpb_attn_sync(h: *mut cpb_attn_t) -> c_int;
    pub fn cpb_attn_destroy(h: *mut cpb_attn_t);
}
