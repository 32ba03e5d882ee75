"""Seeded synthetic Qwen3 weights and prompts.

Weights: every projection and the embedding table are N(0, 0.02) rounded to
bf16, every RMSNorm gain is exactly 1.0 (bf16 0x3F80), embeddings are tied.
Each tensor's values depend only on (seed, Hugging Face tensor name), so any
tensor can be generated alone. The generator itself is synth.c.
"""

from __future__ import annotations

import numpy as np

from ._lib import synth_lib
from .config import Config
from .device import Tensor

ONE_BF16 = 0x3F80
STD = 0.02


def layer_names(i: int) -> list[str]:
    """The 11 per-layer tensors in the order model/model.rs:50-60 loads them."""
    p = f"model.layers.{i}"
    return [
        f"{p}.input_layernorm.weight",
        f"{p}.self_attn.q_proj.weight",
        f"{p}.self_attn.k_proj.weight",
        f"{p}.self_attn.v_proj.weight",
        f"{p}.self_attn.o_proj.weight",
        f"{p}.self_attn.q_norm.weight",
        f"{p}.self_attn.k_norm.weight",
        f"{p}.post_attention_layernorm.weight",
        f"{p}.mlp.gate_proj.weight",
        f"{p}.mlp.up_proj.weight",
        f"{p}.mlp.down_proj.weight",
    ]


def shapes(c: Config) -> dict[str, tuple]:
    """Tensor name -> shape for a Qwen3-style model (HF layout: [out, in])."""
    H, I, hd = c.hidden_size, c.intermediate_size, c.head_dim()
    qd, kvd = c.num_attention_heads * hd, c.num_key_value_heads * hd
    out: dict[str, tuple] = {}
    for i in range(c.num_hidden_layers):
        n = layer_names(i)
        out[n[0]] = (H,)
        out[n[1]] = (qd, H)
        out[n[2]] = (kvd, H)
        out[n[3]] = (kvd, H)
        out[n[4]] = (H, qd)
        if c.qk_norm:
            out[n[5]] = (hd,)
            out[n[6]] = (hd,)
        out[n[7]] = (H,)
        out[n[8]] = (I, H)
        out[n[9]] = (I, H)
        out[n[10]] = (H, I)
    out["model.embed_tokens.weight"] = (c.vocab_size, H)
    out["model.norm.weight"] = (H,)
    if not c.tie_word_embeddings:
        out["lm_head.weight"] = (c.vocab_size, H)
    return out


def tensor(name: str, shape: tuple, seed: int, std: float = STD, random_gains: bool = False) -> Tensor:
    """One synthetic tensor: gains (1-D) are ones (or 1 + N(0, 0.1) with
    random_gains, which tests use to tell gains apart), matrices N(0, std) in bf16."""
    n = int(np.prod(shape))
    if len(shape) == 1:
        if random_gains:
            g = 1.0 + bf16_to_f32(normal_bf16(n, seed, name, 0.1))
            return Tensor(shape, f32_to_bf16(g))
        return Tensor(shape, np.full(n, ONE_BF16, dtype=np.uint16))
    data = np.empty(n, dtype=np.uint16)
    L = synth_lib()
    L.synth_normal_bf16(data.ctypes.data, n, L.synth_key(seed, name.encode()), std)
    return Tensor(shape, data)


def normal_bf16(n: int, seed: int, name: str = "", std: float = 1.0) -> np.ndarray:
    """n values N(0, std) as bf16 bits."""
    data = np.empty(n, dtype=np.uint16)
    L = synth_lib()
    L.synth_normal_bf16(data.ctypes.data, n, L.synth_key(seed, name.encode()), std)
    return data


def weights(c: Config, seed: int = 0, random_gains: bool = False) -> dict[str, Tensor]:
    return {name: tensor(name, shape, seed, random_gains=random_gains) for name, shape in shapes(c).items()}


def prompt(n: int, vocab: int, seed: int = 0) -> np.ndarray:
    """n token ids uniform in [0, vocab)."""
    out = np.empty(n, dtype=np.uint32)
    L = synth_lib()
    L.synth_tokens(out.ctypes.data, n, L.synth_key(seed, b"prompt"), vocab)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
