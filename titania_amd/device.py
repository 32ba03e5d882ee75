"""The hip device, as the reference's `Device` trait (model/device.rs:9-89)
presents it: weights are uploaded once, activations live in buffers allocated
on the device, and every operation runs there.

Method names, argument order and meaning follow the trait. Misuse that the
reference answers with a panic (its length asserts) raises InvalidArgument.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib


@dataclass
class Tensor:
    """A bf16 tensor as raw bits, row-major (model/weights.rs:13-17)."""

    shape: tuple
    data: np.ndarray  # uint16

    def __post_init__(self):
        self.shape = tuple(int(s) for s in self.shape)
        self.data = np.ascontiguousarray(self.data, dtype=np.uint16).reshape(-1)
        if self.data.size != int(np.prod(self.shape)):
            raise ValueError(f"{self.data.size} values for shape {self.shape}")


class Weight:
    """`Device::Weight` (model/device.rs:14-15): a bf16 tensor in device memory."""

    def __init__(self, dev: "Hip", handle: int, shape: tuple):
        self._dev = dev
        self.handle = handle
        self.shape = shape

    def free(self) -> None:
        if self.handle:
            self._dev._refuse_while_capturing("free a weight")
            lib().th_weight_free(self._dev.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self._dev.handle:
                self.free()
        except Exception:
            pass


class Graph:
    """A captured sequence of device calls (th_graph_end): each launch() queues
    one replay on the device's stream over the buffers named at capture time."""

    def __init__(self, dev: "Hip", handle: int):
        self._dev = dev
        self.handle = handle

    def launch(self) -> None:
        check(lib().th_graph_launch(self._dev.handle, self.handle))

    def free(self) -> None:
        if self.handle:
            self._dev._refuse_while_capturing("free a graph")
            lib().th_graph_free(self._dev.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self._dev.handle and not self._dev._capturing:
                self.free()
        except Exception:
            pass


class Buffer:
    """`Device::Buffer` (model/device.rs:10-13): f32 activations in device memory."""

    def __init__(self, dev: "Hip", handle: int):
        self._dev = dev
        self.handle = handle

    def __len__(self) -> int:
        return int(lib().th_buffer_len(self.handle))

    def free(self) -> None:
        if self.handle:
            self._dev._refuse_while_capturing("free a buffer")
            lib().th_buffer_free(self._dev.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self._dev.handle:
                self.free()
        except Exception:
            pass


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


class Hip:
    """A GPU running the model's operations (the `hip` device)."""

    def __init__(self, ordinal: int = 0):
        self._capturing = False
        h = C.c_void_p()
        check(lib().th_device_create(ordinal, C.byref(h)))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            lib().th_device_destroy(self.handle)
            self.handle = None

    def synchronize(self) -> None:
        check(lib().th_device_synchronize(self.handle))

    # ---- HIP graphs of the device's stream (th_graph_*) ----

    def graph_begin(self) -> None:
        """Starts capturing: the compute calls that follow are recorded, not run,
        until graph_end (calls that allocate, copy to or from the host or wait
        raise meanwhile)."""
        check(lib().th_graph_begin(self.handle))
        self._capturing = True

    def graph_end(self) -> Graph:
        self._capturing = False
        out = C.c_void_p()
        check(lib().th_graph_end(self.handle, C.byref(out)))
        return Graph(self, out.value)

    def _refuse_while_capturing(self, what: str) -> None:
        if self._capturing:
            raise RuntimeError(f"cannot {what} while the device's stream is being captured (graph_begin)")

    def timer_begin(self) -> None:
        check(lib().th_timer_begin(self.handle))

    def timer_end(self) -> float:
        """Milliseconds of GPU time since timer_begin (waits for the queued work)."""
        ms = C.c_float()
        check(lib().th_timer_end(self.handle, C.byref(ms)))
        return float(ms.value)

    # ---- memory (model/device.rs:17-42) ----

    def upload(self, tensor: Tensor) -> Weight:
        shape = (C.c_size_t * len(tensor.shape))(*tensor.shape)
        out = C.c_void_p()
        check(lib().th_upload(self.handle, tensor.data.ctypes.data, shape, len(tensor.shape), C.byref(out)))
        return Weight(self, out.value, tensor.shape)

    def alloc(self, length: int) -> Buffer:
        out = C.c_void_p()
        check(lib().th_alloc(self.handle, int(length), C.byref(out)))
        return Buffer(self, out.value)

    def resize(self, buf: Buffer, length: int) -> None:
        check(lib().th_resize(self.handle, buf.handle, int(length)))

    def read(self, buf: Buffer) -> np.ndarray:
        n = len(buf)
        out = np.empty(n, dtype=np.float32)
        check(lib().th_read(self.handle, buf.handle, out.ctypes.data, n))
        return out

    def write(self, buf: Buffer, data) -> None:
        d = _f32(data)
        check(lib().th_write(self.handle, buf.handle, d.ctypes.data, d.size))

    def copy(self, dst: Buffer, dst_offset: int, src: Buffer, src_offset: int, length: int) -> None:
        check(lib().th_copy(self.handle, dst.handle, int(dst_offset), src.handle, int(src_offset), int(length)))

    # ---- compute (model/device.rs:44-88) ----

    def embed(self, out: Buffer, table: Weight, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        check(lib().th_embed(self.handle, out.handle, table.handle, t.ctypes.data, t.size))

    def matmul(self, out: Buffer, w: Weight, x: Buffer) -> None:
        check(lib().th_matmul(self.handle, out.handle, w.handle, x.handle))

    def add(self, x: Buffer, y: Buffer) -> None:
        check(lib().th_add(self.handle, x.handle, y.handle))

    def rmsnorm(self, x: Buffer, weight: Weight, eps: float) -> None:
        check(lib().th_rmsnorm(self.handle, x.handle, weight.handle, float(eps)))

    def rope(self, x: Buffer, table: Buffer, pos: int, n_heads: int, head_dim: int) -> None:
        check(lib().th_rope(self.handle, x.handle, table.handle, int(pos), int(n_heads), int(head_dim)))

    def attention(self, out: Buffer, q: Buffer, k_cache: Buffer, v_cache: Buffer, pos: int, n_heads: int,
                  head_dim: int, n_kv_heads: int) -> None:
        check(lib().th_attention(self.handle, out.handle, q.handle, k_cache.handle, v_cache.handle, int(pos),
                                 int(n_heads), int(head_dim), int(n_kv_heads)))

    def attention_noalloc(self, out: Buffer, q: Buffer, k_cache: Buffer, v_cache: Buffer, pos: int, n_heads: int,
                          head_dim: int, n_kv_heads: int) -> None:
        """attention() with its split partials in the library's fixed per-GPU
        array (no allocation); calls whose partials exceed it raise."""
        check(lib().th_attention_noalloc(self.handle, out.handle, q.handle, k_cache.handle, v_cache.handle,
                                         int(pos), int(n_heads), int(head_dim), int(n_kv_heads)))

    def silu_mul(self, gate: Buffer, up: Buffer) -> None:
        check(lib().th_silu_mul(self.handle, gate.handle, up.handle))

    # ---- fused extensions ----

    def add_rmsnorm(self, x: Buffer, y: Buffer | None, xb: Buffer, weight: Weight, eps: float) -> None:
        check(lib().th_add_rmsnorm(self.handle, x.handle, y.handle if y is not None else None, xb.handle,
                                   weight.handle, float(eps)))

    def qkv_rope_append(self, q: Buffer, k: Buffer, v: Buffer, wq: Weight, wk: Weight, wv: Weight,
                        q_norm: Weight | None, k_norm: Weight | None, xb: Buffer, rope: Buffer, k_cache: Buffer,
                        v_cache: Buffer, pos: int, n_heads: int, n_kv_heads: int, head_dim: int, eps: float) -> None:
        """model.rs:108-120 in one call: the q/k/v projections of xb, the
        per-head norms, the rotations and the appends to position-major
        caches (k and v are left holding the raw projections)."""
        check(lib().th_qkv_rope_append(self.handle, q.handle, k.handle, v.handle, wq.handle, wk.handle, wv.handle,
                                       q_norm.handle if q_norm is not None else None,
                                       k_norm.handle if k_norm is not None else None, xb.handle, rope.handle,
                                       k_cache.handle, v_cache.handle, int(pos), int(n_heads), int(n_kv_heads),
                                       int(head_dim), float(eps)))

    def gate_up_silu(self, gate: Buffer, up: Buffer, w_gate: Weight, w_up: Weight, xb: Buffer) -> None:
        """gate = silu(w_gate . xb) * (w_up . xb) (model.rs:137-139); up is scratch."""
        check(lib().th_gate_up_silu(self.handle, gate.handle, up.handle, w_gate.handle, w_up.handle, xb.handle))

    def argmax(self, logits: Buffer) -> int:
        tok = C.c_uint32()
        check(lib().th_argmax(self.handle, logits.handle, C.byref(tok)))
        return int(tok.value)

    def sample(self, logits: Buffer, sampler) -> int:
        """A draw of `sampler` (titania_amd.sampler.Sampler) from the buffer's
        values (th_sample); advances sampler.rng."""
        tok = C.c_uint32()
        st = C.c_uint64(sampler.rng)
        check(lib().th_sample(self.handle, logits.handle, sampler.temperature, max(sampler.top_k, 0),
                              sampler.top_p, C.byref(st), C.byref(tok)))
        sampler.rng = st.value
        return int(tok.value)


__all__ = ["Hip", "Tensor", "Weight", "Buffer", "_lib"]
