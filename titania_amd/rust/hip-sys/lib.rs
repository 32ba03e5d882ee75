//! Raw bindings of include/titania_hip.h, the C ABI of the hip device (a
//! gfx950 backend behind model/device.rs's `Device` trait). Every function
//! returns TH_OK or an error code whose message th_last_error() gives; the
//! safe wrapper is model/hip.rs.
#![allow(non_camel_case_types)]
use std::ffi::{c_char, c_int};

#[repr(C)]
pub struct th_device {
    _p: [u8; 0],
}
#[repr(C)]
pub struct th_weight {
    _p: [u8; 0],
}
#[repr(C)]
pub struct th_buffer {
    _p: [u8; 0],
}
#[repr(C)]
pub struct th_model {
    _p: [u8; 0],
}
#[repr(C)]
pub struct th_state {
    _p: [u8; 0],
}
#[repr(C)]
pub struct th_graph {
    _p: [u8; 0],
}

/// model/config.rs:9-36 with head_dim resolved.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct th_config {
    pub hidden_size: i64,
    pub intermediate_size: i64,
    pub num_hidden_layers: i64,
    pub num_attention_heads: i64,
    pub num_key_value_heads: i64,
    pub head_dim: i64,
    pub vocab_size: i64,
    pub rms_norm_eps: f32,
    pub rope_theta: f32,
    pub tie_word_embeddings: i64,
}

pub const TH_OK: c_int = 0;
pub const TH_ERR_INVALID: c_int = 1;
pub const TH_ERR_HIP: c_int = 2;
pub const TH_ERR_NOMEM: c_int = 3;
pub const TH_KV_F32: c_int = 0;
pub const TH_KV_BF16: c_int = 1;
pub const TH_PATH_OPS: c_int = 0;
pub const TH_PATH_FUSED: c_int = 1;
pub const TH_PATH_TRAIT: c_int = 2;

unsafe extern "C" {
    pub fn th_last_error() -> *const c_char;
    pub fn th_device_create(ordinal: c_int, out: *mut *mut th_device) -> c_int;
    pub fn th_device_destroy(dev: *mut th_device);
    pub fn th_device_synchronize(dev: *mut th_device) -> c_int;

    // model/device.rs:17-42: memory.
    pub fn th_upload(dev: *mut th_device, data: *const u16, shape: *const usize, ndim: usize,
                     out: *mut *mut th_weight) -> c_int;
    pub fn th_weight_free(dev: *mut th_device, w: *mut th_weight);
    pub fn th_weight_shape(w: *const th_weight, shape: *mut usize, ndim: *mut usize) -> c_int;
    pub fn th_alloc(dev: *mut th_device, len: usize, out: *mut *mut th_buffer) -> c_int;
    pub fn th_buffer_free(dev: *mut th_device, buf: *mut th_buffer);
    pub fn th_resize(dev: *mut th_device, buf: *mut th_buffer, len: usize) -> c_int;
    pub fn th_buffer_len(buf: *const th_buffer) -> usize;
    pub fn th_read(dev: *mut th_device, buf: *const th_buffer, out: *mut f32, len: usize) -> c_int;
    pub fn th_write(dev: *mut th_device, buf: *mut th_buffer, data: *const f32, len: usize) -> c_int;
    pub fn th_copy(dev: *mut th_device, dst: *mut th_buffer, dst_offset: usize, src: *const th_buffer,
                   src_offset: usize, len: usize) -> c_int;

    // model/device.rs:44-88: compute.
    pub fn th_embed(dev: *mut th_device, out: *mut th_buffer, table: *const th_weight, tokens: *const u32,
                    n: usize) -> c_int;
    pub fn th_matmul(dev: *mut th_device, out: *mut th_buffer, w: *const th_weight, x: *const th_buffer) -> c_int;
    pub fn th_add(dev: *mut th_device, x: *mut th_buffer, y: *const th_buffer) -> c_int;
    pub fn th_rmsnorm(dev: *mut th_device, x: *mut th_buffer, weight: *const th_weight, eps: f32) -> c_int;
    pub fn th_rope(dev: *mut th_device, x: *mut th_buffer, table: *const th_buffer, pos: usize, n_heads: usize,
                   head_dim: usize) -> c_int;
    pub fn th_attention(dev: *mut th_device, out: *mut th_buffer, q: *const th_buffer, k_cache: *const th_buffer,
                        v_cache: *const th_buffer, pos: usize, n_heads: usize, head_dim: usize,
                        n_kv_heads: usize) -> c_int;
    pub fn th_attention_noalloc(dev: *mut th_device, out: *mut th_buffer, q: *const th_buffer,
                                k_cache: *const th_buffer, v_cache: *const th_buffer, pos: usize, n_heads: usize,
                                head_dim: usize, n_kv_heads: usize) -> c_int;
    pub fn th_silu_mul(dev: *mut th_device, gate: *mut th_buffer, up: *const th_buffer) -> c_int;

    // Timing and graphs of the device's stream.
    pub fn th_timer_begin(dev: *mut th_device) -> c_int;
    pub fn th_timer_end(dev: *mut th_device, ms: *mut f32) -> c_int;
    pub fn th_graph_begin(dev: *mut th_device) -> c_int;
    pub fn th_graph_end(dev: *mut th_device, out: *mut *mut th_graph) -> c_int;
    pub fn th_graph_launch(dev: *mut th_device, graph: *const th_graph) -> c_int;
    pub fn th_graph_free(dev: *mut th_device, graph: *mut th_graph);

    // Fused extensions.
    pub fn th_add_rmsnorm(dev: *mut th_device, x: *mut th_buffer, y: *const th_buffer, xb: *mut th_buffer,
                          weight: *const th_weight, eps: f32) -> c_int;
    pub fn th_qkv_rope_append(dev: *mut th_device, q: *mut th_buffer, k: *mut th_buffer, v: *mut th_buffer,
                              wq: *const th_weight, wk: *const th_weight, wv: *const th_weight,
                              q_norm: *const th_weight, k_norm: *const th_weight, xb: *const th_buffer,
                              rope: *const th_buffer, k_cache: *mut th_buffer, v_cache: *mut th_buffer, pos: usize,
                              n_heads: usize, n_kv_heads: usize, head_dim: usize, eps: f32) -> c_int;
    pub fn th_gate_up_silu(dev: *mut th_device, gate: *mut th_buffer, up: *mut th_buffer, w_gate: *const th_weight,
                           w_up: *const th_weight, xb: *const th_buffer) -> c_int;
    pub fn th_argmax(dev: *mut th_device, logits: *const th_buffer, token: *mut u32) -> c_int;
    pub fn th_sample(dev: *mut th_device, logits: *const th_buffer, temperature: f32, top_k: usize, top_p: f32,
                     rng: *mut u64, token: *mut u32) -> c_int;

    // The forward pass (model/model.rs) and the decode loops on the device.
    pub fn th_model_create(dev: *mut th_device, config: *const th_config, weights: *const *const th_weight,
                           n_weights: usize, out: *mut *mut th_model) -> c_int;
    pub fn th_model_destroy(model: *mut th_model);
    pub fn th_config_load(path: *const c_char, out: *mut th_config) -> c_int;
    pub fn th_model_load(dev: *mut th_device, dir: *const c_char, out: *mut *mut th_model) -> c_int;
    pub fn th_model_config(model: *const th_model, out: *mut th_config) -> c_int;
    pub fn th_state_create(model: *mut th_model, max_len: usize, kv_dtype: c_int, out: *mut *mut th_state)
                           -> c_int;
    pub fn th_state_destroy(state: *mut th_state);
    pub fn th_forward(model: *mut th_model, state: *mut th_state, tokens: *const u32, n: usize, pos: usize,
                      logits: *mut f32, path: c_int) -> c_int;
    pub fn th_decode(model: *mut th_model, state: *mut th_state, pos: usize, steps: usize, out_tokens: *mut u32,
                     out_logits: *mut f32) -> c_int;
    pub fn th_decode_sample(model: *mut th_model, state: *mut th_state, pos: usize, steps: usize,
                            temperature: f32, top_k: usize, top_p: f32, rng: *mut u64, out_tokens: *mut u32)
                            -> c_int;
    pub fn th_generate(model: *mut th_model, state: *mut th_state, pos: usize, max_tokens: usize, stop: *const u32,
                       n_stop: usize, temperature: f32, top_k: usize, top_p: f32, rng: *mut u64,
                       out_tokens: *mut u32, n_out: *mut usize) -> c_int;
}
