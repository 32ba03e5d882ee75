"""Inputs and checks shared by the tests.

numbers/tensor restate the closed-form xorshift32 inputs of the reference's
differential tests (model/titania.rs:231-249), so the same cases run here.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from titania_amd.device import Tensor


def numbers(n: int, seed: int) -> np.ndarray:
    """Pseudorandom numbers in [-1, 1) (model/titania.rs:231-241)."""
    state = (seed * 2654435761) & 0xFFFFFFFF
    state = max(state, 1)
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        state ^= (state << 13) & 0xFFFFFFFF
        state ^= state >> 17
        state ^= (state << 5) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 23) - np.float32(1.0)
    return out


def tensor(shape, seed: int) -> Tensor:
    """numbers() truncated to bf16 (model/titania.rs:243-249)."""
    n = int(np.prod(shape))
    return Tensor(tuple(shape), (numbers(n, seed).view(np.uint32) >> 16).astype(np.uint16))


def assert_close(actual, expected, rel: float = 1e-4, abs_: float = 1e-5, what: str = "") -> None:
    """|a - e| <= abs_ + rel * |e| elementwise (model/titania.rs:259-266)."""
    a = np.asarray(actual, dtype=np.float32).reshape(-1)
    e = np.asarray(expected, dtype=np.float32).reshape(-1)
    assert a.shape == e.shape, f"{what}: {a.shape} vs {e.shape}"
    tol = abs_ + rel * np.abs(e)
    bad = np.nonzero(~(np.abs(a - e) <= tol))[0]
    if bad.size:
        i = int(bad[0])
        raise AssertionError(f"{what}: {bad.size} elements off; element {i}: got {a[i]}, expected {e[i]}")


def rel_error(actual, expected) -> float:
    """Normwise relative error ||a - e|| / ||e||."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))


GOLDEN = Path(__file__).resolve().parent / "golden"


def load_fixture(name: str):
    """A Hugging Face Qwen3 fixture (tests/golden/make_hf_qwen3.py): the
    config, the generator's metadata, the token sequence (prompt then greedy
    tokens) and the logits at every position."""
    from titania_amd.config import Config

    f = np.load(GOLDEN / f"hf_qwen3_{name}.npz")
    meta = json.loads(str(f["meta"]))
    return Config(**meta["config"]), meta, f["tokens"], f["logits"]


def attention_f64(q, kc, vc, pos, H, KVH):
    """Causal GQA attention in float64 (model/cpu.rs:113-149 in exact
    arithmetic): q [n][H][128], caches [KVH][positions][128]."""
    hd = 128
    n, G = q.size // (H * hd), H // KVH
    qh = q.reshape(n, H, hd).astype(np.float64)
    out = np.empty((n, H, hd))
    mask = np.arange(pos + n)[None, :] > (pos + np.arange(n))[:, None]
    for h in range(H):
        k = kc[h // G, :pos + n].astype(np.float64)
        v = vc[h // G, :pos + n].astype(np.float64)
        s = qh[:, h] @ k.T / np.sqrt(hd)
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p @ v) / p.sum(axis=1, keepdims=True)
    return out.reshape(-1)
