//! The hip device: model/device.rs's `Device` trait on an MI355X (gfx950)
//! through the C ABI of include/titania_hip.h (the titania-hip-sys crate).
//!
//! Added to the reference's model crate as `mod hip; pub use hip::{Hip,
//! HipModel};` with `titania-hip-sys` as a dependency. The trait is infallible
//! by signature and panics on misuse (model/cpu.rs:22,40,52-53), so every
//! non-zero status panics with the library's message; handles are freed on
//! drop, which the trait leaves to the buffer and weight types. Not compiled
//! in this repository's image (no Rust toolchain); tests/test_abi.py checks
//! the crate's declarations against the header.

use std::ffi::{CStr, CString};
use std::path::Path;

use titania_hip_sys as sys;

use crate::{Device, Tensor};

fn check(rc: i32) {
    if rc != sys::TH_OK {
        let msg = unsafe { CStr::from_ptr(sys::th_last_error()) };
        panic!("hip device: {}", msg.to_string_lossy());
    }
}

/// One GPU and the stream its work runs on (model/device.rs:9).
pub struct Hip {
    dev: *mut sys::th_device,
}

/// `Device::Buffer`: f32 activations in HBM.
pub struct HipBuffer {
    dev: *mut sys::th_device,
    ptr: *mut sys::th_buffer,
}

/// `Device::Weight`: a bf16 tensor in HBM, uploaded once.
pub struct HipWeight {
    dev: *mut sys::th_device,
    ptr: *mut sys::th_weight,
}

impl Hip {
    /// Opens GPU `ordinal` (cli/run.rs builds `Cpu` or `Titania` here).
    pub fn new(ordinal: i32) -> Hip {
        let mut dev = std::ptr::null_mut();
        check(unsafe { sys::th_device_create(ordinal, &mut dev) });
        Hip { dev }
    }
}

impl Drop for Hip {
    fn drop(&mut self) {
        unsafe { sys::th_device_destroy(self.dev) }
    }
}

impl Drop for HipBuffer {
    fn drop(&mut self) {
        unsafe { sys::th_buffer_free(self.dev, self.ptr) }
    }
}

impl Drop for HipWeight {
    fn drop(&mut self) {
        unsafe { sys::th_weight_free(self.dev, self.ptr) }
    }
}

impl Device for Hip {
    type Buffer = HipBuffer;
    type Weight = HipWeight;

    fn upload(&self, tensor: Tensor) -> HipWeight {
        let mut ptr = std::ptr::null_mut();
        check(unsafe {
            sys::th_upload(self.dev, tensor.data.as_ptr(), tensor.shape.as_ptr(), tensor.shape.len(), &mut ptr)
        });
        HipWeight { dev: self.dev, ptr }
    }

    fn alloc(&self, len: usize) -> HipBuffer {
        let mut ptr = std::ptr::null_mut();
        check(unsafe { sys::th_alloc(self.dev, len, &mut ptr) });
        HipBuffer { dev: self.dev, ptr }
    }

    fn resize(&self, buf: &mut HipBuffer, len: usize) {
        check(unsafe { sys::th_resize(self.dev, buf.ptr, len) })
    }

    fn read(&self, buf: &HipBuffer) -> Vec<f32> {
        let len = unsafe { sys::th_buffer_len(buf.ptr) };
        let mut out = vec![0.0f32; len];
        check(unsafe { sys::th_read(self.dev, buf.ptr, out.as_mut_ptr(), len) });
        out
    }

    fn write(&self, buf: &mut HipBuffer, data: &[f32]) {
        check(unsafe { sys::th_write(self.dev, buf.ptr, data.as_ptr(), data.len()) })
    }

    fn copy(&self, dst: &mut HipBuffer, dst_offset: usize, src: &HipBuffer, src_offset: usize, len: usize) {
        check(unsafe { sys::th_copy(self.dev, dst.ptr, dst_offset, src.ptr, src_offset, len) })
    }

    fn embed(&self, out: &mut HipBuffer, table: &HipWeight, tokens: &[u32]) {
        check(unsafe { sys::th_embed(self.dev, out.ptr, table.ptr, tokens.as_ptr(), tokens.len()) })
    }

    fn matmul(&self, out: &mut HipBuffer, w: &HipWeight, x: &HipBuffer) {
        check(unsafe { sys::th_matmul(self.dev, out.ptr, w.ptr, x.ptr) })
    }

    fn add(&self, x: &mut HipBuffer, y: &HipBuffer) {
        check(unsafe { sys::th_add(self.dev, x.ptr, y.ptr) })
    }

    fn rmsnorm(&self, x: &mut HipBuffer, weight: &HipWeight, eps: f32) {
        check(unsafe { sys::th_rmsnorm(self.dev, x.ptr, weight.ptr, eps) })
    }

    fn rope(&self, x: &mut HipBuffer, table: &HipBuffer, pos: usize, n_heads: usize, head_dim: usize) {
        check(unsafe { sys::th_rope(self.dev, x.ptr, table.ptr, pos, n_heads, head_dim) })
    }

    fn attention(
        &self,
        out: &mut HipBuffer,
        q: &HipBuffer,
        k_cache: &HipBuffer,
        v_cache: &HipBuffer,
        pos: usize,
        n_heads: usize,
        head_dim: usize,
        n_kv_heads: usize,
    ) {
        check(unsafe {
            sys::th_attention(self.dev, out.ptr, q.ptr, k_cache.ptr, v_cache.ptr, pos, n_heads, head_dim, n_kv_heads)
        })
    }

    fn silu_mul(&self, gate: &mut HipBuffer, up: &HipBuffer) {
        check(unsafe { sys::th_silu_mul(self.dev, gate.ptr, up.ptr) })
    }
}

/// The fused forward pass and the decode loop kept on the device
/// (th_model_load / th_state_create / th_forward / th_decode): the path a
/// `Chat` at temperature 0 takes instead of `Model::forward` +
/// `Sampler::sample`, reading 4 bytes per token instead of the logits.
pub struct HipModel {
    model: *mut sys::th_model,
    state: *mut sys::th_state,
    vocab: usize,
}

impl HipModel {
    /// model/model.rs:40-77 `Model::load` from a directory holding config.json
    /// and model.safetensors, with f32 caches of `max_len` positions.
    pub fn load(hip: &Hip, dir: &Path, max_len: usize) -> HipModel {
        let dir = CString::new(dir.to_string_lossy().as_bytes()).expect("path with a NUL byte");
        let mut model = std::ptr::null_mut();
        check(unsafe { sys::th_model_load(hip.dev, dir.as_ptr(), &mut model) });
        let mut config = sys::th_config::default();
        check(unsafe { sys::th_model_config(model, &mut config) });
        let mut state = std::ptr::null_mut();
        check(unsafe { sys::th_state_create(model, max_len, sys::TH_KV_F32, &mut state) });
        HipModel { model, state, vocab: config.vocab_size as usize }
    }

    /// model/model.rs:83-91 `Model::forward`: the logits after `tokens`, the
    /// first at position `pos`.
    pub fn forward(&mut self, tokens: &[u32], pos: usize) -> Vec<f32> {
        let mut logits = vec![0.0f32; self.vocab];
        check(unsafe {
            sys::th_forward(self.model, self.state, tokens.as_ptr(), tokens.len(), pos, logits.as_mut_ptr(),
                            sys::TH_PATH_FUSED)
        });
        logits
    }

    /// `steps` greedy tokens from the logits the last forward left, fed at
    /// positions pos, pos + 1, ... on the device.
    pub fn decode(&mut self, pos: usize, steps: usize) -> Vec<u32> {
        let mut tokens = vec![0u32; steps];
        check(unsafe {
            sys::th_decode(self.model, self.state, pos, steps, tokens.as_mut_ptr(), std::ptr::null_mut())
        });
        tokens
    }
}

impl Drop for HipModel {
    fn drop(&mut self) {
        unsafe {
            sys::th_state_destroy(self.state);
            sys::th_model_destroy(self.model);
        }
    }
}
