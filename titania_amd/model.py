"""The forward pass on the hip device: Model (model/model.rs:10-77), State
(model/model.rs:152-211), Model::forward (model/model.rs:83-91) and the greedy
decode loop (model/chat.rs:149-178 at temperature 0), over the C ABI.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import TH_KV_BF16, TH_KV_F32, TH_PATH_FUSED, TH_PATH_OPS, TH_PATH_TRAIT, ThConfig, check, lib
from .config import Config
from .device import Hip, Tensor, Weight
from .synth import layer_names

BATCH = 64  # model/model.rs:8


class Model:
    """A decoder-only transformer with its weights on the hip device."""

    def __init__(self, device: Hip, config: Config, tensors: dict[str, Tensor]):
        """Uploads `tensors` (Hugging Face names) in the order model.rs:40-77 loads them."""
        self.device = device
        self.config = config
        self._weights: list[Weight | None] = []
        order: list[str | None] = []
        for i in range(config.num_hidden_layers):
            for name in layer_names(i):
                optional = name.endswith(("q_norm.weight", "k_norm.weight"))
                order.append(name if (name in tensors or not optional) else None)
        order += ["model.embed_tokens.weight", "model.norm.weight",
                  None if config.tie_word_embeddings else "lm_head.weight"]
        for name in order:
            if name is None:
                self._weights.append(None)
            else:
                if name not in tensors:
                    raise KeyError(f"missing tensor '{name}'")
                self._weights.append(device.upload(tensors[name]))
        arr = (C.c_void_p * len(self._weights))(*[w.handle if w else None for w in self._weights])
        cfg = config.to_c()
        out = C.c_void_p()
        check(lib().th_model_create(device.handle, C.byref(cfg), arr, len(self._weights), C.byref(out)))
        self.handle = out.value

    @classmethod
    def load(cls, device: Hip, directory) -> "Model":
        """model/model.rs:40-77 `Model::load`: config.json and model.safetensors
        from `directory`, read and uploaded by the library (th_model_load)."""
        out = C.c_void_p()
        check(lib().th_model_load(device.handle, str(directory).encode(), C.byref(out)))
        cfg = ThConfig()
        check(lib().th_model_config(out.value, C.byref(cfg)))
        self = cls.__new__(cls)
        self.device = device
        self.config = Config.from_c(cfg)
        self._weights = []  # owned by the library's model
        self.handle = out.value
        return self

    def close(self) -> None:
        if self.handle:
            lib().th_model_destroy(self.handle)
            self.handle = None
        for w in self._weights:
            if w is not None:
                w.free()
        self._weights = []

    def forward(self, state: "State", tokens, pos: int, path: int = TH_PATH_FUSED,
                want_logits: bool = True) -> np.ndarray | None:
        """model/model.rs:83-91: runs `tokens` from position `pos`; returns the
        logits of the token that follows the last of them."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        logits = np.empty(self.config.vocab_size, dtype=np.float32) if want_logits else None
        check(lib().th_forward(self.handle, state.handle, t.ctypes.data, t.size, int(pos),
                               logits.ctypes.data if want_logits else None, int(path)))
        return logits

    def decode(self, state: "State", pos: int, steps: int, keep_logits: bool = False, sampler=None):
        """Decode on the device from position `pos`: returns the `steps`
        tokens (and, with keep_logits, the logits after each fed token).
        Greedy, or drawn by `sampler` (titania_amd.sampler.Sampler, whose rng
        advances by `steps` draws)."""
        toks = np.empty(steps, dtype=np.uint32)
        if sampler is not None:
            if keep_logits:
                raise ValueError("a sampled decode keeps its logits on the device")
            st = C.c_uint64(sampler.rng)
            check(lib().th_decode_sample(self.handle, state.handle, int(pos), int(steps), sampler.temperature,
                                         max(sampler.top_k, 0), sampler.top_p, C.byref(st), toks.ctypes.data))
            sampler.rng = st.value
            return toks
        logits = np.empty((steps, self.config.vocab_size), dtype=np.float32) if keep_logits else None
        check(lib().th_decode(self.handle, state.handle, int(pos), int(steps), toks.ctypes.data,
                              logits.ctypes.data if keep_logits else None))
        return (toks, logits) if keep_logits else toks


    def decode_until(self, state: "State", pos: int, max_tokens: int, stop, sampler=None) -> np.ndarray:
        """th_generate: from position `pos`, picks (or draws, with `sampler`)
        and feeds tokens until one in `stop` (1 to 8 ids) is picked, at most
        `max_tokens` in all. Returns the tokens; a stop token, if reached, is
        the last and was not fed."""
        stops = np.ascontiguousarray(stop, dtype=np.uint32).reshape(-1)
        toks = np.empty(max(int(max_tokens), 0), dtype=np.uint32)
        n = C.c_size_t()
        rng = C.c_uint64(sampler.rng if sampler is not None else 0)
        t = float(sampler.temperature) if sampler is not None else 0.0
        k = max(sampler.top_k, 0) if sampler is not None else 0
        p = float(sampler.top_p) if sampler is not None else 1.0
        check(lib().th_generate(self.handle, state.handle, int(pos), toks.size, stops.ctypes.data, stops.size, t, k, p,
                                C.byref(rng) if sampler is not None else None, toks.ctypes.data, C.byref(n)))
        if sampler is not None:
            sampler.rng = rng.value
        return toks[: n.value].copy()


class State:
    """Caches and buffers for sequences of up to max_len tokens (model.rs:176-211)."""

    def __init__(self, model: Model, max_len: int, kv_dtype: int = TH_KV_F32):
        out = C.c_void_p()
        check(lib().th_state_create(model.handle, int(max_len), int(kv_dtype), C.byref(out)))
        self.handle = out.value
        self.max_len = max_len

    def close(self) -> None:
        if self.handle:
            lib().th_state_destroy(self.handle)
            self.handle = None


def generate(model: Model, state: State, prompt, steps: int, keep_logits: bool = False):
    """Feeds the prompt at position 0, then greedily decodes `steps` tokens."""
    model.forward(state, prompt, 0, TH_PATH_FUSED, want_logits=False)
    return model.decode(state, len(prompt), steps, keep_logits)


__all__ = ["Model", "State", "generate", "BATCH", "TH_PATH_OPS", "TH_PATH_FUSED", "TH_PATH_TRAIT", "TH_KV_F32",
           "TH_KV_BF16"]
