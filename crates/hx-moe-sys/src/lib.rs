//! Raw bindings to libhxmoe.so, one declaration per entry point of
//! include/hx_moe.h (same names, argument order and C types). The safe
//! wrapper a helexa maintainer puts in front of it (`HxMoeBlock`, a candle
//! `Module`) lives in neuron, next to the block it replaces
//! (crates/neuron/src/harness/arch/qwen3_5/moe.rs:55, 164-199).
//!
//! Status codes, storage formats and struct layouts mirror the header's
//! `#define`s and `typedef struct`s field for field.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_void};

// status codes
pub const HX_OK: c_int = 0;
pub const HX_ERR_INVALID_ARGUMENT: c_int = 1;
pub const HX_ERR_UNSUPPORTED: c_int = 2;
pub const HX_ERR_DEVICE: c_int = 3;
pub const HX_ERR_WORKSPACE_TOO_SMALL: c_int = 4;
pub const HX_ERR_OUT_OF_MEMORY: c_int = 5;

// storage formats: the GGML type ids
pub const HX_F32: i32 = 0;
pub const HX_F16: i32 = 1;
pub const HX_Q8_0: i32 = 8;
pub const HX_Q4_K: i32 = 12;
pub const HX_Q6_K: i32 = 14;
pub const HX_BF16: i32 = 30;

// where the pointers in hx_moe_weights live
pub const HX_HOST: i32 = 0;
pub const HX_DEVICE: i32 = 1;

// bytes of the fixed scratch behind hx_moe_forward_noalloc
pub const HX_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

/// MoE fields of TextConfig (crates/neuron/src/harness/arch/qwen3_5/mod.rs:270-302).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct hx_moe_config {
    pub hidden_size: i32,
    pub num_experts: i32,
    pub num_experts_per_tok: i32,
    pub moe_intermediate_size: i32,
    pub shared_expert_intermediate_size: i32,
    pub norm_topk_prob: i32,
    pub act_dtype: i32,
}

/// Checkpoint tensors of one block (moe.rs:73-102, mlp.rs:43-45); copied by
/// hx_moe_create, free after it returns.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct hx_moe_weights {
    pub location: i32,
    pub router_dtype: i32,
    pub router: *const c_void,
    pub gate_dtype: i32,
    pub experts_gate: *const c_void,
    pub up_dtype: i32,
    pub experts_up: *const c_void,
    pub down_dtype: i32,
    pub experts_down: *const c_void,
    pub shared_gate_dtype: i32,
    pub shared_gate: *const c_void,
    pub shared_up_dtype: i32,
    pub shared_up: *const c_void,
    pub shared_down_dtype: i32,
    pub shared_down: *const c_void,
    pub shared_expert_gate_dtype: i32,
    pub shared_expert_gate: *const c_void,
}

/// Opaque handle.
#[repr(C)]
pub struct hx_moe {
    _private: [u8; 0],
}

#[link(name = "hxmoe")]
extern "C" {
    pub fn hx_moe_create(cfg: *const hx_moe_config, w: *const hx_moe_weights, device: c_int, out: *mut *mut hx_moe) -> c_int;
    pub fn hx_moe_destroy(m: *mut hx_moe) -> c_int;
    pub fn hx_moe_workspace_size(m: *const hx_moe, n_tokens: i64, bytes: *mut usize) -> c_int;
    pub fn hx_moe_forward(m: *mut hx_moe, x: *const c_void, n_tokens: i64, y: *mut c_void, workspace: *mut c_void, workspace_bytes: usize, router_bias: *const f32, stream: *mut c_void) -> c_int;
    pub fn hx_moe_forward_noalloc(m: *mut hx_moe, x: *const c_void, n_tokens: i64, y: *mut c_void, router_bias: *const f32, stream: *mut c_void) -> c_int;
    pub fn hx_moe_forward_host(m: *mut hx_moe, x_host: *const c_void, n_tokens: i64, y_host: *mut c_void, router_bias_host: *const f32) -> c_int;
    pub fn hx_moe_route(m: *mut hx_moe, x: *const c_void, n_tokens: i64, router_bias: *const f32, topk_idx: *mut i32, topk_w: *mut f32, perm: *mut i32, offsets: *mut i32, inv: *mut i32, workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn hx_moe_router_logits(m: *mut hx_moe, x: *const c_void, n_tokens: i64, router_bias: *const f32, logits: *mut f32, stream: *mut c_void) -> c_int;
    pub fn hx_moe_decoder_mlp(m: *mut hx_moe, x: *mut c_void, n_tokens: i64, norm_w: *const f32, eps: f32, workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn hx_quantize(dtype: c_int, src: *const f32, rows: i64, cols: i64, dst: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn hx_dequantize(dtype: c_int, src: *const c_void, rows: i64, cols: i64, dst: *mut f32, stream: *mut c_void) -> c_int;
    pub fn hx_row_bytes(dtype: c_int, n: i64) -> i64;
    pub fn hx_quantize_activations(weight_dtype: c_int, x: *const c_void, x_dtype: c_int, rows: i64, cols: i64, codes: *mut i8, d: *mut f32, stream: *mut c_void) -> c_int;
    pub fn hx_moe_timing_begin(m: *mut hx_moe, max_calls: c_int) -> c_int;
    pub fn hx_moe_timing_read(m: *mut hx_moe, ms: *mut f64, launches: *mut i64, n_slots: *mut c_int) -> c_int;
    pub fn hx_moe_timing_end(m: *mut hx_moe, ms: *mut f64, launches: *mut i64, n_slots: *mut c_int) -> c_int;
    pub fn hx_moe_timing_name(slot: c_int) -> *const c_char;
    pub fn hx_last_error() -> *const c_char;
}
