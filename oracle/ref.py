"""ctypes binding of the CPU oracle (liboracle.so, built from cpu_ref.c).

Test infrastructure: only tests/, the smoke check and bench.py's CPU-baseline
leg use it, as the results to compare against or as the timed baseline, never
as the product.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_P, _SZ = C.c_void_p, C.c_size_t
_lib = None


def build() -> Path:
    r = subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB


class RefConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int64), ("intermediate", C.c_int64), ("layers", C.c_int64), ("heads", C.c_int64),
        ("kv_heads", C.c_int64), ("head_dim", C.c_int64), ("vocab", C.c_int64), ("eps", C.c_float),
        ("theta", C.c_float), ("tied", C.c_int64),
    ]


class RefLayer(C.Structure):
    _fields_ = [(n, _P) for n in
                ("attn_norm", "q", "k", "v", "o", "q_norm", "k_norm", "mlp_norm", "gate", "up", "down")]


class RefModelC(C.Structure):
    _fields_ = [("c", RefConfig), ("embed", _P), ("norm", _P), ("lm_head", _P), ("layers", C.POINTER(RefLayer))]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        sig = {
            "ref_set_threads": (None, [C.c_int]),
            "ref_get_threads": (C.c_int, []),
            "ref_copy": (None, [_P, _SZ, _P, _SZ, _SZ]),
            "ref_embed": (None, [_P, _P, _SZ, _P, _SZ]),
            "ref_matmul": (None, [_P, _P, _SZ, _SZ, _P, _SZ]),
            "ref_add": (None, [_P, _P, _SZ]),
            "ref_rmsnorm": (None, [_P, _SZ, _P, _SZ, C.c_float]),
            "ref_rope": (None, [_P, _SZ, _P, _SZ, _SZ, _SZ]),
            "ref_attention": (None, [_P, _P, _SZ, _P, _P, _SZ, _SZ, _SZ, _SZ]),
            "ref_silu_mul": (None, [_P, _P, _SZ]),
            "ref_rope_table": (None, [_P, _SZ, _SZ, C.c_float]),
            "ref_argmax": (C.c_uint32, [_P, _SZ]),
            "ref_state_new": (_P, [C.POINTER(RefConfig), _SZ, _SZ]),
            "ref_state_free": (None, [_P]),
            "ref_state_k_cache": (_P, [_P, C.c_int64]),
            "ref_state_v_cache": (_P, [_P, C.c_int64]),
            "ref_forward": (C.c_int, [C.POINTER(RefModelC), _P, _P, _SZ, _SZ, _P]),
            "ref_generate": (C.c_int, [C.POINTER(RefModelC), _P, _P, _SZ, _SZ, _P, _P, _P]),
            "ref_rng_next_u64": (C.c_uint64, [C.POINTER(C.c_uint64)]),
            "ref_sample": (C.c_uint32, [_P, _SZ, C.c_float, _SZ, C.c_float, C.POINTER(C.c_uint64)]),
            "ref_generate_sampled": (C.c_int, [C.POINTER(RefModelC), _P, _P, _SZ, _SZ, C.c_float, _SZ, C.c_float,
                                               C.POINTER(C.c_uint64), _P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint16)


def set_threads(n: int) -> None:
    lib().ref_set_threads(int(n))


# ---- single operations, each returning a new array ----

def embed(table: np.ndarray, dim: int, tokens) -> np.ndarray:
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.empty(t.size * dim, dtype=np.float32)
    tb = _u16(table)
    lib().ref_embed(out.ctypes.data, tb.ctypes.data, dim, t.ctypes.data, t.size)
    return out


def matmul(w: np.ndarray, rows: int, cols: int, x) -> np.ndarray:
    xx = _f32(x).reshape(-1)
    n = xx.size // cols
    out = np.empty(n * rows, dtype=np.float32)
    ww = _u16(w)
    lib().ref_matmul(out.ctypes.data, ww.ctypes.data, rows, cols, xx.ctypes.data, n)
    return out


def add(x, y) -> np.ndarray:
    out = _f32(x).reshape(-1).copy()
    yy = _f32(y).reshape(-1)
    lib().ref_add(out.ctypes.data, yy.ctypes.data, min(out.size, yy.size))
    return out


def rmsnorm(x, weight: np.ndarray, eps: float) -> np.ndarray:
    out = _f32(x).reshape(-1).copy()
    w = _u16(weight)
    lib().ref_rmsnorm(out.ctypes.data, out.size, w.ctypes.data, w.size, eps)
    return out


def rope(x, table, pos: int, n_heads: int, head_dim: int) -> np.ndarray:
    out = _f32(x).reshape(-1).copy()
    tb = _f32(table).reshape(-1)
    lib().ref_rope(out.ctypes.data, out.size, tb.ctypes.data, pos, n_heads, head_dim)
    return out


def attention(q, k_cache, v_cache, pos: int, n_heads: int, head_dim: int, n_kv_heads: int) -> np.ndarray:
    qq = _f32(q).reshape(-1)
    n = qq.size // (n_heads * head_dim)
    out = np.empty_like(qq)
    k, v = _f32(k_cache).reshape(-1), _f32(v_cache).reshape(-1)
    lib().ref_attention(out.ctypes.data, qq.ctypes.data, n, k.ctypes.data, v.ctypes.data, pos, n_heads, head_dim,
                        n_kv_heads)
    return out


def silu_mul(gate, up) -> np.ndarray:
    out = _f32(gate).reshape(-1).copy()
    u = _f32(up).reshape(-1)
    lib().ref_silu_mul(out.ctypes.data, u.ctypes.data, min(out.size, u.size))
    return out


def copy(dst, dst_offset: int, src, src_offset: int, length: int) -> np.ndarray:
    out = _f32(dst).reshape(-1).copy()
    s = _f32(src).reshape(-1)
    lib().ref_copy(out.ctypes.data, dst_offset, s.ctypes.data, src_offset, length)
    return out


def rope_table(max_len: int, head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(max_len * head_dim, dtype=np.float32)
    lib().ref_rope_table(out.ctypes.data, max_len, head_dim, theta)
    return out


def argmax(logits) -> int:
    x = _f32(logits).reshape(-1)
    return int(lib().ref_argmax(x.ctypes.data, x.size))


class Sampler:
    """model/sampler.rs:1-59: top-k, then top-p, at a temperature, drawing with
    xorshift64* seeded by max(seed, 1). `state` is the generator's state."""

    def __init__(self, temperature: float, top_k: int, top_p: float, seed: int):
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.state = max(int(seed), 1) & 0xFFFFFFFFFFFFFFFF

    def sample(self, logits) -> int:
        x = _f32(logits).reshape(-1)
        st = C.c_uint64(self.state)
        tok = lib().ref_sample(x.ctypes.data, x.size, self.temperature, max(int(self.top_k), 0), self.top_p,
                               C.byref(st))
        self.state = st.value
        return int(tok)


def rng_next_u64(state: int) -> tuple[int, int]:
    """One step of the oracle's xorshift64*: (output, new state)."""
    st = C.c_uint64(state)
    out = lib().ref_rng_next_u64(C.byref(st))
    return int(out), st.value


# ---- the forward pass ----

class RefModel:
    """The oracle's model over host weights (dict of HF name -> Tensor-like with .data)."""

    def __init__(self, config, tensors: dict, batch: int = 64):
        self.config = config
        self._keep = []
        c = config

        def ptr(name, optional=False):
            if name not in tensors:
                if optional:
                    return None
                raise KeyError(name)
            a = _u16(tensors[name].data)
            self._keep.append(a)
            return a.ctypes.data

        layers = (RefLayer * c.num_hidden_layers)()
        for i in range(c.num_hidden_layers):
            p = f"model.layers.{i}"
            layers[i] = RefLayer(
                ptr(f"{p}.input_layernorm.weight"), ptr(f"{p}.self_attn.q_proj.weight"),
                ptr(f"{p}.self_attn.k_proj.weight"), ptr(f"{p}.self_attn.v_proj.weight"),
                ptr(f"{p}.self_attn.o_proj.weight"), ptr(f"{p}.self_attn.q_norm.weight", True),
                ptr(f"{p}.self_attn.k_norm.weight", True), ptr(f"{p}.post_attention_layernorm.weight"),
                ptr(f"{p}.mlp.gate_proj.weight"), ptr(f"{p}.mlp.up_proj.weight"), ptr(f"{p}.mlp.down_proj.weight"))
        self._layers = layers
        cfg = RefConfig(c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
                        c.num_key_value_heads, c.head_dim(), c.vocab_size, c.rms_norm_eps, c.rope_theta,
                        1 if c.tie_word_embeddings else 0)
        self.c_model = RefModelC(cfg, ptr("model.embed_tokens.weight"), ptr("model.norm.weight"),
                                 None if c.tie_word_embeddings else ptr("lm_head.weight"),
                                 C.cast(layers, C.POINTER(RefLayer)))
        self.batch = batch

    def state(self, max_len: int) -> "RefState":
        return RefState(self, max_len)

    def forward(self, state: "RefState", tokens, pos: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        rc = lib().ref_forward(C.byref(self.c_model), state.handle, t.ctypes.data, t.size, pos, out.ctypes.data)
        if rc != 0:
            raise ValueError("oracle forward: tokens past the end of the cache")
        return out

    def generate(self, state: "RefState", prompt, steps: int):
        """Returns (tokens, top-2 gaps, logits after the last fed token)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.empty(steps, dtype=np.uint32)
        gaps = np.empty(steps, dtype=np.float32)
        last = np.empty(self.config.vocab_size, dtype=np.float32)
        rc = lib().ref_generate(C.byref(self.c_model), state.handle, p.ctypes.data, p.size, steps,
                                toks.ctypes.data, gaps.ctypes.data, last.ctypes.data)
        if rc != 0:
            raise ValueError("oracle generate: tokens past the end of the cache")
        return toks, gaps, last

    def generate_sampled(self, state: "RefState", prompt, steps: int, sampler: Sampler):
        """The prompt, then `steps` tokens drawn by `sampler` (whose state advances)."""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.empty(steps, dtype=np.uint32)
        st = C.c_uint64(sampler.state)
        rc = lib().ref_generate_sampled(C.byref(self.c_model), state.handle, p.ctypes.data, p.size, steps,
                                        sampler.temperature, max(int(sampler.top_k), 0), sampler.top_p,
                                        C.byref(st), toks.ctypes.data)
        if rc != 0:
            raise ValueError("oracle generate: tokens past the end of the cache")
        sampler.state = st.value
        return toks


class RefChat:
    """model/chat.rs:24-196 at the token level: the conversation stays in the
    caches and each call runs the model over its new tokens only (`feed`,
    chat.rs:189-196); a reply samples, stops at a stop token without feeding
    it, and otherwise feeds each token (chat.rs:132-187). `sampler` None is
    the temperature-0 pick (sampler.rs:27-33). max_tokens bounds a reply (the
    reference's loop has no bound)."""

    def __init__(self, model: RefModel, max_len: int, sampler: Sampler | None = None):
        self.model = model
        self.state = model.state(max_len)
        self.sampler = sampler
        self.len = 0
        self.logits = None

    def feed(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        if self.len + t.size > self.state.max_len:
            raise ValueError("the conversation no longer fits in the context window")
        if t.size:
            self.logits = self.model.forward(self.state, t, self.len)
        self.len += t.size
        return self.logits

    def generate(self, prompt, stop, end, max_tokens: int) -> np.ndarray:
        stops = {int(x) for x in np.asarray(stop).reshape(-1)}
        logits = self.feed(prompt)
        out = []
        while len(out) < max_tokens:
            tok = self.sampler.sample(logits) if self.sampler is not None else argmax(logits)
            out.append(tok)
            if tok in stops:
                break
            logits = self.feed([tok])
        self.feed(end)
        return np.array(out, dtype=np.uint32)


class RefState:
    def __init__(self, model: RefModel, max_len: int):
        self.model = model
        self.max_len = max_len
        self.handle = lib().ref_state_new(C.byref(model.c_model.c), max_len, model.batch)

    def k_cache(self, layer: int) -> np.ndarray:
        c = self.model.config
        n = self.max_len * c.num_key_value_heads * c.head_dim()
        p = lib().ref_state_k_cache(self.handle, layer)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n,)).copy()

    def __del__(self):
        try:
            if self.handle:
                lib().ref_state_free(self.handle)
                self.handle = None
        except Exception:
            pass
