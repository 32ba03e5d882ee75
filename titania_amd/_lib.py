"""ctypes binding of the hip device's C ABI (include/titania_hip.h).

The library is loaded from this package directory; there is no fallback: if
libtitania_hip.so is missing, importing the device raises.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libtitania_hip.so"
SYNTH_PATH = PKG / "libtitania_synth.so"

TH_OK, TH_ERR_INVALID, TH_ERR_HIP, TH_ERR_NOMEM = 0, 1, 2, 3
TH_KV_F32, TH_KV_BF16 = 0, 1
TH_PATH_OPS, TH_PATH_FUSED, TH_PATH_TRAIT = 0, 1, 2


class HipError(RuntimeError):
    """A failed call into the hip device; `code` is the TH_ERR_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class InvalidArgument(HipError):
    """TH_ERR_INVALID: the misuse the reference's asserts panic on."""


class ThConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int64),
        ("intermediate_size", C.c_int64),
        ("num_hidden_layers", C.c_int64),
        ("num_attention_heads", C.c_int64),
        ("num_key_value_heads", C.c_int64),
        ("head_dim", C.c_int64),
        ("vocab_size", C.c_int64),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("tie_word_embeddings", C.c_int64),
    ]


_P = C.c_void_p
_SZ = C.c_size_t
_I = C.c_int

# name -> (restype, argtypes); mirrors include/titania_hip.h.
SIGNATURES: dict[str, tuple] = {
    "th_last_error": (C.c_char_p, []),
    "th_device_create": (_I, [_I, C.POINTER(_P)]),
    "th_device_destroy": (None, [_P]),
    "th_device_synchronize": (_I, [_P]),
    "th_timer_begin": (_I, [_P]),
    "th_timer_end": (_I, [_P, C.POINTER(C.c_float)]),
    "th_graph_begin": (_I, [_P]),
    "th_graph_end": (_I, [_P, C.POINTER(_P)]),
    "th_graph_launch": (_I, [_P, _P]),
    "th_graph_free": (None, [_P, _P]),
    "th_upload": (_I, [_P, _P, C.POINTER(_SZ), _SZ, C.POINTER(_P)]),
    "th_weight_free": (None, [_P, _P]),
    "th_weight_shape": (_I, [_P, C.POINTER(_SZ), C.POINTER(_SZ)]),
    "th_alloc": (_I, [_P, _SZ, C.POINTER(_P)]),
    "th_buffer_free": (None, [_P, _P]),
    "th_resize": (_I, [_P, _P, _SZ]),
    "th_buffer_len": (_SZ, [_P]),
    "th_read": (_I, [_P, _P, _P, _SZ]),
    "th_write": (_I, [_P, _P, _P, _SZ]),
    "th_copy": (_I, [_P, _P, _SZ, _P, _SZ, _SZ]),
    "th_embed": (_I, [_P, _P, _P, _P, _SZ]),
    "th_matmul": (_I, [_P, _P, _P, _P]),
    "th_add": (_I, [_P, _P, _P]),
    "th_rmsnorm": (_I, [_P, _P, _P, C.c_float]),
    "th_rope": (_I, [_P, _P, _P, _SZ, _SZ, _SZ]),
    "th_attention": (_I, [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ]),
    "th_attention_noalloc": (_I, [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ]),
    "th_silu_mul": (_I, [_P, _P, _P]),
    "th_add_rmsnorm": (_I, [_P, _P, _P, _P, _P, C.c_float]),
    "th_qkv_rope_append": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _SZ, _SZ, _SZ, C.c_float]),
    "th_gate_up_silu": (_I, [_P, _P, _P, _P, _P, _P]),
    "th_argmax": (_I, [_P, _P, C.POINTER(C.c_uint32)]),
    "th_sample": (_I, [_P, _P, C.c_float, _SZ, C.c_float, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)]),
    "th_model_create": (_I, [_P, C.POINTER(ThConfig), C.POINTER(_P), _SZ, C.POINTER(_P)]),
    "th_model_destroy": (None, [_P]),
    "th_config_load": (_I, [C.c_char_p, C.POINTER(ThConfig)]),
    "th_model_load": (_I, [_P, C.c_char_p, C.POINTER(_P)]),
    "th_model_config": (_I, [_P, C.POINTER(ThConfig)]),
    "th_state_create": (_I, [_P, _SZ, _I, C.POINTER(_P)]),
    "th_state_destroy": (None, [_P]),
    "th_forward": (_I, [_P, _P, _P, _SZ, _SZ, _P, _I]),
    "th_decode": (_I, [_P, _P, _SZ, _SZ, _P, _P]),
    "th_decode_sample": (_I, [_P, _P, _SZ, _SZ, C.c_float, _SZ, C.c_float, C.POINTER(C.c_uint64), _P]),
    "th_generate": (_I, [_P, _P, _SZ, _SZ, _P, _SZ, C.c_float, _SZ, C.c_float, C.POINTER(C.c_uint64), _P,
                         C.POINTER(_SZ)]),
}

_lib: C.CDLL | None = None
_synth: C.CDLL | None = None


def lib() -> C.CDLL:
    """The loaded hip device library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m titania_amd.build`")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def synth_lib() -> C.CDLL:
    global _synth
    if _synth is None:
        if not SYNTH_PATH.exists():
            raise ImportError(f"{SYNTH_PATH} is missing: build it with `python -m titania_amd.build`")
        L = C.CDLL(str(SYNTH_PATH))
        L.synth_key.restype = C.c_uint64
        L.synth_key.argtypes = [C.c_uint64, C.c_char_p]
        L.synth_normal_bf16.restype = None
        L.synth_normal_bf16.argtypes = [_P, C.c_uint64, C.c_uint64, C.c_float]
        L.synth_tokens.restype = None
        L.synth_tokens.argtypes = [_P, C.c_uint64, C.c_uint64, C.c_uint32]
        _synth = L
    return _synth


def check(rc: int) -> None:
    """Raises the error the last call reported."""
    if rc != TH_OK:
        msg = lib().th_last_error().decode(errors="replace")
        cls = InvalidArgument if rc == TH_ERR_INVALID else HipError
        raise cls(rc, msg)
