//! The hip device: model/device.rs's `Device` trait on an MI355X (gfx950)
//! through the C ABI of include/titania_hip.h (the titania-hip-sys crate).
//!
//! Added to the reference's model crate by titania_amd/rust/patches/
//! (model-lib.rs.patch: `mod hip; pub use hip::{Hip, HipModel};`,
//! model-Cargo.toml.patch: the titania-hip-sys dependency). The trait is
//! infallible by signature and panics on misuse (model/cpu.rs:22,40,52-53),
//! so every non-zero status panics with the library's message. Beside the
//! thirteen primitives, the fused methods of the trait extension
//! (model-device.rs.patch: add_rmsnorm, qkv_rope_append, gate_up_silu,
//! argmax) are overridden with the library's fused entry points, which the
//! patched forward_batch calls (model-model.rs.patch).
//!
//! Lifetimes: every buffer, weight and model holds a reference-counted
//! handle of its device, so the device is destroyed only after the last of
//! them is freed, whatever order the owner drops them in (`Model<D>`
//! declares `device` before its weights, model/model.rs:11-19, and a
//! `State<Hip>` may outlive its model). Not compiled in this repository's
//! image (no Rust toolchain); tests/test_abi.py checks the crate's
//! declarations against the header and these overrides against the patch.

use std::ffi::{CStr, CString};
use std::path::Path;
use std::rc::Rc;

use titania_hip_sys as sys;

use crate::{Device, Tensor};

fn check(rc: i32) {
    if rc != sys::TH_OK {
        let msg = unsafe { CStr::from_ptr(sys::th_last_error()) };
        panic!("hip device: {}", msg.to_string_lossy());
    }
}

/// The library's device handle, destroyed when the last owner drops it.
struct DeviceHandle(*mut sys::th_device);

impl Drop for DeviceHandle {
    fn drop(&mut self) {
        unsafe { sys::th_device_destroy(self.0) }
    }
}

/// One GPU and the stream its work runs on (model/device.rs:9).
pub struct Hip {
    dev: Rc<DeviceHandle>,
}

/// `Device::Buffer`: f32 activations in HBM.
pub struct HipBuffer {
    dev: Rc<DeviceHandle>,
    ptr: *mut sys::th_buffer,
}

/// `Device::Weight`: a bf16 tensor in HBM, uploaded once.
pub struct HipWeight {
    dev: Rc<DeviceHandle>,
    ptr: *mut sys::th_weight,
}

impl Hip {
    /// Opens GPU `ordinal` (cli/run.rs builds `Cpu` or `Titania` here).
    pub fn new(ordinal: i32) -> Hip {
        let mut dev = std::ptr::null_mut();
        check(unsafe { sys::th_device_create(ordinal, &mut dev) });
        Hip { dev: Rc::new(DeviceHandle(dev)) }
    }

    fn raw(&self) -> *mut sys::th_device {
        self.dev.0
    }
}

impl Drop for HipBuffer {
    fn drop(&mut self) {
        unsafe { sys::th_buffer_free(self.dev.0, self.ptr) }
    }
}

impl Drop for HipWeight {
    fn drop(&mut self) {
        unsafe { sys::th_weight_free(self.dev.0, self.ptr) }
    }
}

impl Device for Hip {
    type Buffer = HipBuffer;
    type Weight = HipWeight;

    fn upload(&self, tensor: Tensor) -> HipWeight {
        let mut ptr = std::ptr::null_mut();
        check(unsafe {
            sys::th_upload(self.raw(), tensor.data.as_ptr(), tensor.shape.as_ptr(), tensor.shape.len(), &mut ptr)
        });
        HipWeight { dev: Rc::clone(&self.dev), ptr }
    }

    fn alloc(&self, len: usize) -> HipBuffer {
        let mut ptr = std::ptr::null_mut();
        check(unsafe { sys::th_alloc(self.raw(), len, &mut ptr) });
        HipBuffer { dev: Rc::clone(&self.dev), ptr }
    }

    fn resize(&self, buf: &mut HipBuffer, len: usize) {
        check(unsafe { sys::th_resize(self.raw(), buf.ptr, len) })
    }

    fn read(&self, buf: &HipBuffer) -> Vec<f32> {
        let len = unsafe { sys::th_buffer_len(buf.ptr) };
        let mut out = vec![0.0f32; len];
        check(unsafe { sys::th_read(self.raw(), buf.ptr, out.as_mut_ptr(), len) });
        out
    }

    fn write(&self, buf: &mut HipBuffer, data: &[f32]) {
        check(unsafe { sys::th_write(self.raw(), buf.ptr, data.as_ptr(), data.len()) })
    }

    fn copy(&self, dst: &mut HipBuffer, dst_offset: usize, src: &HipBuffer, src_offset: usize, len: usize) {
        check(unsafe { sys::th_copy(self.raw(), dst.ptr, dst_offset, src.ptr, src_offset, len) })
    }

    fn embed(&self, out: &mut HipBuffer, table: &HipWeight, tokens: &[u32]) {
        check(unsafe { sys::th_embed(self.raw(), out.ptr, table.ptr, tokens.as_ptr(), tokens.len()) })
    }

    fn matmul(&self, out: &mut HipBuffer, w: &HipWeight, x: &HipBuffer) {
        check(unsafe { sys::th_matmul(self.raw(), out.ptr, w.ptr, x.ptr) })
    }

    fn add(&self, x: &mut HipBuffer, y: &HipBuffer) {
        check(unsafe { sys::th_add(self.raw(), x.ptr, y.ptr) })
    }

    fn rmsnorm(&self, x: &mut HipBuffer, weight: &HipWeight, eps: f32) {
        check(unsafe { sys::th_rmsnorm(self.raw(), x.ptr, weight.ptr, eps) })
    }

    fn rope(&self, x: &mut HipBuffer, table: &HipBuffer, pos: usize, n_heads: usize, head_dim: usize) {
        check(unsafe { sys::th_rope(self.raw(), x.ptr, table.ptr, pos, n_heads, head_dim) })
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
            sys::th_attention(self.raw(), out.ptr, q.ptr, k_cache.ptr, v_cache.ptr, pos, n_heads, head_dim,
                              n_kv_heads)
        })
    }

    fn silu_mul(&self, gate: &mut HipBuffer, up: &HipBuffer) {
        check(unsafe { sys::th_silu_mul(self.raw(), gate.ptr, up.ptr) })
    }

    // ---- the trait extension's fused methods ----

    fn add_rmsnorm(&self, x: &mut HipBuffer, xb: &mut HipBuffer, add: bool, weight: &HipWeight, eps: f32,
                   len: usize) {
        assert_eq!(unsafe { sys::th_buffer_len(x.ptr) }, len, "add_rmsnorm over all of x");
        // The residual is read from xb before xb is overwritten, row by row.
        let y = if add { xb.ptr as *const sys::th_buffer } else { std::ptr::null() };
        check(unsafe { sys::th_add_rmsnorm(self.raw(), x.ptr, y, xb.ptr, weight.ptr, eps) })
    }

    fn qkv_rope_append(
        &self,
        q: &mut HipBuffer,
        k: &mut HipBuffer,
        v: &mut HipBuffer,
        w: [&HipWeight; 3],
        q_norm: Option<&HipWeight>,
        k_norm: Option<&HipWeight>,
        xb: &HipBuffer,
        rope: &HipBuffer,
        k_cache: &mut HipBuffer,
        v_cache: &mut HipBuffer,
        pos: usize,
        n: usize,
        n_heads: usize,
        n_kv_heads: usize,
        head_dim: usize,
        eps: f32,
    ) {
        assert_eq!(unsafe { sys::th_buffer_len(q.ptr) }, n * n_heads * head_dim, "q holds the n tokens");
        let qn = q_norm.map_or(std::ptr::null(), |g| g.ptr as *const sys::th_weight);
        let kn = k_norm.map_or(std::ptr::null(), |g| g.ptr as *const sys::th_weight);
        check(unsafe {
            sys::th_qkv_rope_append(self.raw(), q.ptr, k.ptr, v.ptr, w[0].ptr, w[1].ptr, w[2].ptr, qn, kn, xb.ptr,
                                    rope.ptr, k_cache.ptr, v_cache.ptr, pos, n_heads, n_kv_heads, head_dim, eps)
        })
    }

    fn gate_up_silu(&self, gate: &mut HipBuffer, up: &mut HipBuffer, w_gate: &HipWeight, w_up: &HipWeight,
                    xb: &HipBuffer) {
        check(unsafe { sys::th_gate_up_silu(self.raw(), gate.ptr, up.ptr, w_gate.ptr, w_up.ptr, xb.ptr) })
    }

    fn argmax(&self, logits: &HipBuffer) -> u32 {
        let mut token = 0u32;
        check(unsafe { sys::th_argmax(self.raw(), logits.ptr, &mut token) });
        token
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
    // Dropped after Drop::drop has destroyed the state and the model.
    _dev: Rc<DeviceHandle>,
}

impl HipModel {
    /// model/model.rs:40-77 `Model::load` from a directory holding config.json
    /// and model.safetensors, with f32 caches of `max_len` positions.
    pub fn load(hip: &Hip, dir: &Path, max_len: usize) -> HipModel {
        let dir = CString::new(dir.to_string_lossy().as_bytes()).expect("path with a NUL byte");
        let mut model = std::ptr::null_mut();
        check(unsafe { sys::th_model_load(hip.raw(), dir.as_ptr(), &mut model) });
        let mut config = sys::th_config::default();
        check(unsafe { sys::th_model_config(model, &mut config) });
        let mut state = std::ptr::null_mut();
        check(unsafe { sys::th_state_create(model, max_len, sys::TH_KV_F32, &mut state) });
        HipModel { model, state, vocab: config.vocab_size as usize, _dev: Rc::clone(&hip.dev) }
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
